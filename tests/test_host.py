"""Host-side logic of the product library (CPU only, no GPU calls): the C
ABI exports, the block quantizers, request packing, state keys and state
files, config validation and the exported-directory round trip — each
against the oracle or against the reference's own format definitions."""
from __future__ import annotations

import ctypes as C
import re
import struct
from pathlib import Path

import numpy as np
import pytest

import grande_amd as g
import oracle
from grande_amd import _lib as L
from grande_amd import BranchTokens as B, Group
from tests.common import gemma3_tiny, gguf_tiny

HEADER = Path(__file__).resolve().parents[1] / "include" / "omg_hip.h"


def test_library_exports_every_declared_symbol():
    text = HEADER.read_text()
    names = sorted(set(re.findall(r"\b(omg_[a-z0-9_]+)\s*\(", text)))
    assert len(names) > 30
    lib = L.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


@pytest.mark.parametrize("dtype", [g.Q8, g.Q4])
def test_quantize_matches_oracle(dtype):
    rng = np.random.default_rng(dtype)
    v = (rng.standard_normal(32 * 700) * np.exp2(rng.uniform(-8, 4, 32 * 700))).astype(np.float32)
    v[:32] = 0.0                       # an all-zero block
    v[32:64] = 0.25                    # a constant block
    v[64:96] = -v[64:96]               # sign flips
    d1, s1 = g.quantize(dtype, v)
    d2, s2 = oracle.quantize(dtype, v)
    assert np.array_equal(d1, d2) and np.array_equal(s1, s2)
    with pytest.raises(L.OmgError):
        g.quantize(dtype, v[:31])


@pytest.mark.parametrize("linear,embed", [(g.F16, g.F16), (g.Q8, g.Q4), (g.Q4, g.Q8)])
def test_synth_follows_reference_generator(linear, embed):
    """reference.rs:106-139: one xorshift stream from `seed | 1` over the
    tensor catalogue in order; the embedding at scale 1."""
    cfg = gguf_tiny()
    ts = list(g.Weights.synth(cfg, 6, linear, embed).tensors())
    assert ts[0].name == "embed"
    vals, _ = oracle.rng_values(7, 64 * 64, 1.0)
    if embed == g.F16:
        assert np.array_equal(ts[0].to_f32().ravel(), vals.astype(np.float16).astype(np.float32))
    else:
        d, s = oracle.quantize(embed, vals)
        assert np.array_equal(ts[0].data, d) and np.array_equal(ts[0].scales, s)


def random_groups(rng, ngroups):
    out = []
    for _ in range(ngroups):
        prefix = rng.integers(0, 64, int(rng.integers(1, 20))).tolist()
        branches = []
        for _ in range(int(rng.integers(1, 6))):
            n = int(rng.integers(1, 9))
            want = sorted(rng.choice(n, int(rng.integers(0, n + 1)), replace=False).tolist())
            branches.append(B(rng.integers(0, 64, n).tolist(), want))
        out.append(Group(prefix, branches))
    return out


def test_pack_matches_oracle():
    rng = np.random.default_rng(11)
    for trial in range(40):
        groups = random_groups(rng, int(rng.integers(1, 5)))
        first = int(rng.integers(0, len(groups)))
        resident = bool(trial % 2)
        ids, meta, wanted = g.pack(groups, first, resident)
        oids, ometa, owanted, _ = oracle.pack(groups, first, resident)
        assert np.array_equal(ids, oids)
        assert np.array_equal(meta, ometa)
        assert np.array_equal(wanted, owanted)


def test_aligned_pack_is_the_reference_layout_with_groups_moved():
    """The engine's layout (align_groups): the reference's packing with every
    group after the first moved up to a multiple of `align` cache rows.
    Real tokens keep their ids, positions and sequence ids in order; a
    group's first key row is its new first row; padding rows between
    groups carry token 0 and sequence id -1 and see only themselves;
    wanted rows still point at the same tokens; a layout that would need
    more rows than available stays the reference's."""
    rng = np.random.default_rng(12)
    for trial in range(60):
        groups = random_groups(rng, int(rng.integers(1, 6)))
        first = int(rng.integers(0, len(groups)))
        resident = bool(trial % 2)
        align = [32, 64][trial % 2]
        ids, meta, wanted = g.pack(groups, first, resident)
        aids, ameta, awanted = g.pack(groups, first, resident, align=align, rows=1 << 20)
        base = len(groups[first].prefix) if resident else 0
        real = ameta[:, 1] >= 0
        assert np.array_equal(aids[real], ids) and np.array_equal(ameta[real][:, :2], meta[:, :2])
        assert (aids[~real] == 0).all() and (ameta[~real][:, 0] == 0).all()
        rows = base + np.arange(len(aids))
        assert np.array_equal(ameta[:, 3], rows + 1)
        assert np.array_equal(ameta[~real][:, 2], rows[~real])
        groups_seen = ameta[real][:, 1] >> 12
        starts = [int(rows[real][np.argmax(groups_seen == k)]) for k in np.unique(groups_seen) if k > 0]
        assert all(r % align == 0 for r in starts)
        for k in np.unique(groups_seen):
            sel = real & ((ameta[:, 1] >> 12) == k)
            lo = ameta[sel][:, 2]
            assert (lo == lo[0]).all()
            assert lo[0] == (0 if k == 0 else rows[sel][0])
        assert np.array_equal(wanted[:, :3], awanted[:, :3])
        assert np.array_equal(aids[awanted[:, 3]], ids[wanted[:, 3]])
        # no room: the reference's layout
        tight = g.pack(groups, first, resident, align=align, rows=base + len(ids))
        assert np.array_equal(tight[1], meta)


def test_pack_errors():
    # engine.rs:1537-1562: too many branches, wanted past the branch
    with pytest.raises(L.OmgError, match="past"):
        g.pack([Group([1, 2], [B([3, 4], [2])])])
    with pytest.raises(L.OmgError, match="branches"):
        g.pack([Group([1], [B([2], [0])] * 4096)])


@pytest.mark.parametrize("model_id,n", [("", 0), ("hip", 5), ("gemma-3-270m-q4", 2000)])
def test_state_key_matches_oracle(model_id, n):
    prefix = np.random.default_rng(n).integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    assert g.state_key(model_id, prefix) == oracle.state_key(model_id, prefix)


def grws1(model_id: str, prefix, layers) -> bytes:
    """The state file of engine.rs:515-533, written from its definition."""
    out = b"GRWS1\0" + struct.pack("<I", len(model_id)) + model_id.encode()
    out += struct.pack("<I", len(prefix)) + np.asarray(prefix, "<u4").tobytes()
    out += struct.pack("<I", len(layers))
    for layer, row0, data in layers:
        out += struct.pack("<III", layer, row0, len(data)) + data
    return out


def test_state_file_format():
    data = grws1("m", [5, 6, 7], [(0, 0, b"\1\2" * 8), (1, 2, b"\3\4")])
    assert g.state_check(data, "m") == (3, 2)
    with pytest.raises(L.OmgError, match="different model"):
        g.state_check(data, "other")
    with pytest.raises(L.OmgError, match="truncated"):
        g.state_check(data[:-1], "m")
    with pytest.raises(L.OmgError, match="state file"):
        g.state_check(b"GRWS2\0" + data[6:], "m")
    with pytest.raises(L.OmgError):
        g.state_check(b"", "m")


@pytest.mark.parametrize("edit,match", [
    (lambda c: c.pop("hidden_size"), "hidden_size"),
    (lambda c: c.update(num_attention_heads=3, num_key_value_heads=2), "head"),
    (lambda c: c.update(head_dim=128), "head_dim"),
])
def test_config_validation(edit, match):
    import json
    c = json.loads(gemma3_tiny())
    edit(c)
    with pytest.raises(L.OmgError, match=match):
        g.EngineBuilder(json.dumps(c))


def test_builder_checks_tensors():
    b = g.EngineBuilder(gemma3_tiny())
    ts = list(g.Weights.synth(gemma3_tiny(), 7, g.F16, g.F16).tensors())
    assert "embed" in b.missing() and len(b.missing()) == len(ts)
    bad = ts[0]
    bad = g.QTensor(bad.name, bad.dtype, (bad.shape[0] + 1, bad.shape[1]), bad.data, bad.scales)
    with pytest.raises(L.OmgError, match="shape"):
        b.push(bad)
    with pytest.raises(L.OmgError, match="unexpected"):
        b.push(g.QTensor("blk.99.o", ts[1].dtype, ts[1].shape, ts[1].data, ts[1].scales))


def test_export_dir_round_trip(tmp_path):
    w = g.Weights.synth(gguf_tiny(), 3, g.Q4, g.Q8)
    g.export_dir(w, tmp_path / "m")
    w2 = g.Weights.load_dir(tmp_path / "m")
    a, b = list(w.tensors()), list(w2.tensors())
    assert [t.name for t in a] == [t.name for t in b]
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and x.shape == y.shape
        assert np.array_equal(x.data, y.data) and np.array_equal(x.scales, y.scales)


def test_gemma4_export_dir_round_trip(tmp_path):
    """A Gemma 4 checkpoint's per-layer token table travels in
    per_layer_table.bin under the manifest's per_layer_table entry
    (model.rs:744-750) and reads back unchanged."""
    import json
    from tests.common import gemma4_tiny
    cfg = gemma4_tiny()
    w = g.Weights.synth(cfg, 23, g.Q4, g.Q8)
    ts = {t.name: t for t in w.tensors()}
    assert ts["per_layer_table"].shape == (64, 4 * 32) and list(ts)[-1] == "per_layer_table"
    g.export_dir(w, tmp_path)
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert man["per_layer_table"]["path"] == "per_layer_table.bin"
    assert all(f["path"] != "per_layer_table.bin" for f in man["files"])
    back = {t.name: t for t in g.Weights.load_dir(tmp_path).tensors()}
    assert set(back) == set(ts)
    for k, t in ts.items():
        assert np.array_equal(t.data, back[k].data) and np.array_equal(t.scales, back[k].scales), k


@pytest.mark.parametrize("edit,match", [
    (lambda c: c.update(global_head_dim=384), "head_dim"),
    (lambda c: c.update(hidden_size_per_layer_input=48), "per_layer_input"),
    (lambda c: c.update(num_kv_shared_layers=4), "num_kv_shared_layers"),
])
def test_gemma4_config_validation(edit, match):
    import json
    from tests.common import gemma4_tiny
    c = json.loads(gemma4_tiny())
    edit(c)
    with pytest.raises(L.OmgError, match=match):
        g.EngineBuilder(json.dumps(c))


def test_state_bytes_mutations_fail_cleanly():
    """GRWS1 parsing (SavedState::from_bytes) of randomly changed or cut
    bytes: parsed or refused with OmgError, never a crash."""
    import random
    import struct
    rnd = random.Random(5)
    refused = 0
    for i in range(400):
        b = b"GRWS1\0" + struct.pack("<I", 1) + b"m" + struct.pack("<I", 3) + struct.pack("<III", 1, 2, 3)
        b += struct.pack("<I", 2)
        for layer in range(2):
            b += struct.pack("<III", layer, 0, 16) + bytes(16)
        b = bytearray(b)
        for _ in range(rnd.randint(1, 3)):
            b[rnd.randrange(len(b))] = rnd.choice([0, 0xFF, rnd.randrange(256)])
        if rnd.random() < 0.3:
            b = b[: rnd.randrange(len(b) + 1)]
        try:
            g.state_check(bytes(b), "m")
        except L.OmgError:
            refused += 1
    assert refused > 0
