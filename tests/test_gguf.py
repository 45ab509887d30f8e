"""GGUF loading (omg_load_gguf): a llama.cpp Gemma 3 or Gemma 4 file read directly,
mapped as tools/export_wgpu_gguf.py:112-296 maps it; the files are written
by tests/gguf_writer.py from seeded checkpoints.  CPU only: the tensors
must come back bit-equal to the checkpoint they were written from (f32
norms return as the f16 values they hold; bf16 ones as f16(bf16))."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
from tests.common import gemma4_tiny, gguf_tiny
from tests.gguf_writer import write_gemma3


@pytest.mark.parametrize("dtype", [g.Q8, g.Q4, g.F16])
def test_gguf_tensors_round_trip(tmp_path, dtype):
    cfg = gguf_tiny(heads=4, kv_heads=2)
    w = g.Weights.synth(cfg, 3, dtype, dtype)
    path = tmp_path / "m.gguf"
    write_gemma3(path, cfg, w)
    back = {t.name: t for t in g.Weights.load_gguf(path).tensors()}
    orig = {t.name: t for t in w.tensors()}
    assert sorted(back) == sorted(orig)
    for name, t in orig.items():
        b = back[name]
        assert (b.dtype, tuple(b.shape)) == (t.dtype, tuple(t.shape)), name
        assert np.array_equal(b.data, t.data) and np.array_equal(b.scales, t.scales), name


@pytest.mark.parametrize("dtype", [g.Q8, g.Q4, g.F16])
@pytest.mark.parametrize("heads,kv", [(4, 1), (8, 2)])
def test_gguf_gemma4_tensors_round_trip(tmp_path, dtype, heads, kv):
    """A gemma4 GGUF (export_wgpu_gguf.py:140-290): shared-K/V layers
    without k / v tensors, head_dim 512 global layers whose partial RoPE
    rides in rope_freqs, per-layer ff lengths, the per-layer input tensors
    and token table, per-layer output scalars."""
    cfg = gemma4_tiny(heads, kv)
    w = g.Weights.synth(cfg, 3, dtype, dtype)
    path = tmp_path / "m4.gguf"
    write_gemma3(path, cfg, w)
    loaded = g.Weights.load_gguf(path)
    back = {t.name: t for t in loaded.tensors()}
    orig = {t.name: t for t in w.tensors()}
    assert sorted(back) == sorted(orig)
    for name, t in orig.items():
        b = back[name]
        assert (b.dtype, tuple(b.shape)) == (t.dtype, tuple(t.shape)), name
        assert np.array_equal(b.data, t.data) and np.array_equal(b.scales, t.scales), name


def test_gguf_bf16_norms(tmp_path):
    cfg = gguf_tiny()
    w = g.Weights.synth(cfg, 4, g.Q8, g.Q8)
    path = tmp_path / "m.gguf"
    write_gemma3(path, cfg, w, bf16=("blk.1.attn_k_norm.weight",))
    back = {t.name: t for t in g.Weights.load_gguf(path).tensors()}
    v = {t.name: t for t in w.tensors()}["blk.1.k_norm"].data.view(np.float16).astype(np.float32)
    exp = ((v.view(np.uint32) >> 16) << 16).view(np.float32).astype(np.float16)
    assert np.array_equal(back["blk.1.k_norm"].data.view(np.float16), exp)


def test_gguf_rejections(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + bytes(32))
    with pytest.raises(g.OmgError, match="not a GGUF"):
        g.Weights.load_gguf(bad)
    cfg = gguf_tiny()
    w = g.Weights.synth(cfg, 4, g.Q8, g.Q8)
    good = tmp_path / "m.gguf"
    write_gemma3(good, cfg, w)
    raw = good.read_bytes()
    (tmp_path / "llama.gguf").write_bytes(raw.replace(b"gemma3", b"llama3", 1))
    with pytest.raises(g.OmgError, match="architecture"):
        g.Weights.load_gguf(tmp_path / "llama.gguf")
    (tmp_path / "short.gguf").write_bytes(raw[: len(raw) // 2])
    with pytest.raises(g.OmgError, match="past the end|truncated"):
        g.Weights.load_gguf(tmp_path / "short.gguf")


@pytest.mark.gpu
def test_engine_from_gguf_matches_engine_from_checkpoint(tmp_path):
    """The engine opened from the GGUF gives bit-equal rows to the engine
    built from the checkpoint the file was written from."""
    cfg = gguf_tiny(heads=4, kv_heads=2)
    w = g.Weights.synth(cfg, 8, g.Q4, g.Q8)
    path = tmp_path / "m.gguf"
    write_gemma3(path, cfg, w)
    a = g.Engine.new(w, 128, 16)
    b = g.Engine.open_gguf(path, 128, 16)
    rng = np.random.default_rng(1)
    prefix = rng.integers(0, 64, 30).tolist()
    branches = [g.BranchTokens(rng.integers(0, 64, 7).tolist(), [6]) for _ in range(3)]
    for x, y in zip(a.evaluate(prefix, branches, g.Want.HIDDEN), b.evaluate(prefix, branches, g.Want.HIDDEN)):
        assert np.array_equal(x.rows[0], y.rows[0])


@pytest.mark.gpu
def test_engine_from_gemma4_gguf_matches_engine_from_checkpoint(tmp_path):
    """Gemma 4: the engine opened from the GGUF (config from its metadata)
    gives bit-equal rows to the engine built from the checkpoint."""
    cfg = gemma4_tiny(8, 2)
    w = g.Weights.synth(cfg, 8, g.Q4, g.Q8)
    path = tmp_path / "m4.gguf"
    write_gemma3(path, cfg, w)
    a = g.Engine.new(w, 128, 16)
    b = g.Engine.open_gguf(path, 128, 16)
    rng = np.random.default_rng(2)
    prefix = rng.integers(0, 64, 30).tolist()
    branches = [g.BranchTokens(rng.integers(0, 64, 7).tolist(), [6]) for _ in range(3)]
    for x, y in zip(a.evaluate(prefix, branches, g.Want.HIDDEN), b.evaluate(prefix, branches, g.Want.HIDDEN)):
        assert np.array_equal(x.rows[0], y.rows[0])


def test_gguf_mutated_headers_fail_cleanly(tmp_path):
    """Random byte changes in the header, metadata and tensor infos, and
    truncations: every file either loads or is refused with OmgError (the
    parser bounds-checks every read against the file)."""
    import random
    cfg = gemma4_tiny()
    w = g.Weights.synth(cfg, 3, g.Q8, g.Q8)
    src = tmp_path / "src.gguf"
    write_gemma3(src, cfg, w)
    raw = src.read_bytes()
    rnd = random.Random(11)
    refused = 0
    for i in range(150):
        b = bytearray(raw)
        for _ in range(rnd.randint(1, 4)):
            pos = rnd.randrange(min(len(b), 6000))
            b[pos] = rnd.choice([0, 0xFF, rnd.randrange(256)])
        if rnd.random() < 0.2:
            b = b[: rnd.randrange(len(b))]
        p = tmp_path / "m.gguf"
        p.write_bytes(bytes(b))
        try:
            g.Weights.load_gguf(p)
        except g.OmgError:
            refused += 1
    assert refused > 0
