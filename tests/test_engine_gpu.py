"""The engine against the CPU oracle on identical seeded weights and token
ids, and the reference's invariants, through the C ABI on the GPU.  Each
test mirrors one of crates/omg-wgpu/tests/reference.rs:380-735."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
import oracle
from grande_amd import _lib as L
from grande_amd import BranchTokens, Group, PrefixSource, Want
from tests.common import (assert_close, build, gemma3_tiny, gemma4_tiny, gguf_tiny, oracle_rows, rel_diff,
                          tiled_oracle, worst_rel)

pytestmark = pytest.mark.gpu

PREFIX = [2, 5, 9, 14, 20, 31, 7, 8, 3, 22]
BRANCHES = [BranchTokens([11, 12, 13, 14, 15], [1, 4]), BranchTokens([30, 31, 32, 33, 34, 35, 36, 37], [0, 7])]


def check_hidden(cfg: str, seed: int, linear: int, embed: int, tol: float = 2e-2, tight: float = 4e-3,
                 prefix=PREFIX, branches=BRANCHES):
    """reference.rs:380-407: rows at the wanted positions within `tol`
    (relative to the row's largest magnitude) of the plain f32 forward, and
    within `tight` of the forward with the GPU path's f16 rounding points."""
    eng, plain, gpu_r, _ = build(cfg, seed, linear, embed)
    out = eng.evaluate(prefix, branches, Want.HIDDEN)
    exp_plain = oracle_rows(plain, prefix, branches)
    exp_gpu = oracle_rows(gpu_r, prefix, branches)
    worst_p = worst_g = 0.0
    for o, ep, eg in zip(out, exp_plain, exp_gpu):
        for got, a, b in zip(o.rows, ep, eg):
            worst_p = max(worst_p, rel_diff(got, a))
            worst_g = max(worst_g, rel_diff(got, b))
    print(f"rel diff vs f32 oracle {worst_p:.2e}, vs f16-rounding oracle {worst_g:.2e}")
    assert worst_p < tol, f"relative diff {worst_p} vs the f32 oracle"
    assert worst_g < tight, f"relative diff {worst_g} vs the f16-rounding oracle"


def test_gemma3_matches_cpu_reference():
    check_hidden(gemma3_tiny(), 7, g.F16, g.F16)


def test_q8_matches_cpu_reference():
    check_hidden(gguf_tiny(), 7, g.Q8, g.Q8)


def test_q4_matches_cpu_reference():
    check_hidden(gguf_tiny(), 9, g.Q4, g.Q8)


@pytest.mark.parametrize("heads,kv", [(8, 2), (4, 2), (2, 2), (16, 1)])
def test_gqa_q4_matches_cpu_reference(heads, kv):
    """Every query-heads-per-KV-head grouping the attention kernel packs."""
    check_hidden(gguf_tiny(heads, kv), 11, g.Q4, g.Q8)


def test_long_prefix_sliding_window_matches_cpu_reference():
    """Keys beyond one 64-row tile, windows cutting through tiles, branches
    straddling tile boundaries."""
    rng = np.random.default_rng(3)
    cfg = gguf_tiny(4, 1, window=37, vocab=64)
    prefix = rng.integers(0, 64, 150).tolist()
    branches = [BranchTokens(rng.integers(0, 64, n).tolist(), [n - 1, n // 2]) for n in (23, 9, 41)]
    eng, plain, gpu_r, _ = build(cfg, 21, g.Q4, g.Q8, capacity=256)
    out = eng.evaluate(prefix, branches, Want.HIDDEN)
    for o, ep, eg in zip(out, oracle_rows(plain, prefix, branches), oracle_rows(gpu_r, prefix, branches)):
        for got, a, b in zip(o.rows, ep, eg):
            assert rel_diff(got, a) < 2e-2
            assert rel_diff(got, b) < 4e-3


@pytest.mark.parametrize("heads,kv", [(8, 2), (4, 4)])
def test_split_key_ranges_with_several_kv_heads(heads, kv):
    """A prefix long enough that global layers cut query tiles' key ranges
    into chunks (partials merged afterwards), with more than one KV head;
    a branch's rows must not change when its siblings' tokens do
    (reference.rs:533-562, same layout)."""
    rng = np.random.default_rng(5)
    cfg = gguf_tiny(heads, kv, window=37, vocab=64)
    prefix = rng.integers(0, 64, 1400).tolist()
    branches = [BranchTokens(rng.integers(0, 64, n).tolist(), [n - 1, 0]) for n in (20, 7, 33)]
    eng, plain, gpu_r, _ = build(cfg, 23, g.Q4, g.Q8, capacity=1536)
    out = eng.evaluate(prefix, branches, Want.HIDDEN)
    for o, ep, eg in zip(out, oracle_rows(plain, prefix, branches), oracle_rows(gpu_r, prefix, branches)):
        for got, a, b in zip(o.rows, ep, eg):
            assert rel_diff(got, a) < 2e-2
            assert rel_diff(got, b) < 4e-3
    eng.evict_resident()
    changed = [BranchTokens(rng.integers(0, 64, len(b.tokens)).tolist(), b.want) for b in branches]
    changed[1] = branches[1]
    again = eng.evaluate(prefix, changed, Want.HIDDEN)
    assert all(np.array_equal(x, y) for x, y in zip(again[1].rows, out[1].rows))


def test_resident_prefix_matches_full_pass():
    """reference.rs:430-480: bit-equal rows over a resident prefix."""
    for cfg, lin, emb in [(gemma3_tiny(), g.F16, g.F16), (gguf_tiny(), g.Q4, g.Q8), (gguf_tiny(8, 2), g.Q4, g.Q8)]:
        eng, _, _, _ = build(cfg, 13, lin, emb, oracle_models=False)
        prefix = [2, 5, 9, 14, 20, 31, 7]
        branches = [BranchTokens([11, 12, 13, 14, 15], [1, 4]), BranchTokens([30, 31, 32], [0, 2])]
        other = [BranchTokens([33, 34, 35, 36, 37, 38], [5])]
        full = eng.evaluate(prefix, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.DECODED
        cont = eng.evaluate(prefix, other, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.RESIDENT
        eng.evict_resident()
        cold = eng.evaluate(prefix, other, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.DECODED
        assert all(np.array_equal(a, b) for a, b in zip(cont[0].rows, cold[0].rows))
        again = eng.evaluate(prefix, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.RESIDENT
        for a, b in zip(full, again):
            assert all(np.array_equal(x, y) for x, y in zip(a.rows, b.rows))
        prefix2 = [2, 3, 4]
        p2 = eng.evaluate(prefix2, branches, Want.LOGITS)
        assert eng.prefix_source() == PrefixSource.DECODED
        p2r = eng.evaluate(prefix2, branches, Want.LOGITS)
        assert eng.prefix_source() == PrefixSource.RESIDENT
        for a, b in zip(p2, p2r):
            assert all(np.array_equal(x, y) for x, y in zip(a.rows, b.rows))


@pytest.mark.parametrize("d,ff", [(2304, 4096), (64, 16384)])
def test_deep_k_chunks_same_rows_in_long_and_short_passes(d, ff):
    """Down projections deep enough to sum K in 1,024-wide pieces: width
    2,304 > 2,048 (one split of K 4,096, four pieces) and width 64 (four
    splits of 4,096, four pieces each: the residual norm adds the short
    pass's sixteen parts in four runs of four, over two rounds of loads).
    The long cold pass adds the pieces in the GEMM's registers, the short
    warm pass on the resident prefix runs a piece per workgroup and the
    norm adds the parts in the same order — bit-equal rows, and within the
    f32 oracle's reach."""
    cfg = gemma3_tiny(d=d, ff=ff, layers=1, sliding=[False])
    eng, plain, _, _ = build(cfg, 21, g.Q4, g.F16, capacity=1024)
    rng = np.random.default_rng(21)
    prefix = rng.integers(0, 40, 520).tolist()
    branches = [BranchTokens(rng.integers(0, 40, 12).tolist(), [3, 11]), BranchTokens(rng.integers(0, 40, 9).tolist(), [8])]
    eng.evict_resident()
    cold = eng.evaluate(prefix, branches, Want.HIDDEN)  # 541 rows: pieces added in registers
    assert eng.prefix_source() == PrefixSource.DECODED
    warm = eng.evaluate(prefix, branches, Want.HIDDEN)  # 21 rows: a piece per workgroup
    assert eng.prefix_source() == PrefixSource.RESIDENT
    for a, b in zip(cold, warm):
        assert all(np.array_equal(x, y) for x, y in zip(a.rows, b.rows))
    ref = oracle_rows(plain, prefix, branches)
    assert max(rel_diff(x, y) for a, b in zip(cold, ref) for x, y in zip(a.rows, b)) < 2e-2


def test_state_cache_restores_exactly(tmp_path):
    """reference.rs:482-522: RAM cache and GRWS1 bytes restore bit-equal rows;
    a foreign model id is refused."""
    for cfg, lin, emb in [(gemma3_tiny(), g.F16, g.F16), (gguf_tiny(), g.Q4, g.Q8), (gguf_tiny(8, 2), g.Q4, g.Q8)]:
        eng, _, _, _ = build(cfg, 17, lin, emb, oracle_models=False)
        eng.set_state_cache(64 << 20, None, "test")
        a = [2, 5, 9, 14, 20, 31, 7, 8, 3, 22, 4, 6]
        b = [2, 3, 4]
        branches = [BranchTokens([11, 12, 13, 14, 15], [0, 2, 4])]
        full_a = eng.evaluate(a, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.DECODED
        saved = eng.save_state(a, "test")
        eng.evaluate(b, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.DECODED
        ram_a = eng.evaluate(a, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.RAM
        assert all(np.array_equal(x, y) for x, y in zip(full_a[0].rows, ram_a[0].rows))
        assert g.state_check(saved, "test")[0] == len(a)
        with pytest.raises(g.OmgError):
            g.state_check(saved, "other")
        with pytest.raises(g.OmgError):
            eng.restore_state(saved, "other")
        eng.evaluate(b, branches, Want.HIDDEN)
        eng.evict_resident()
        eng.restore_state(saved, "test")
        assert eng.is_resident(a)
        file_a = eng.evaluate(a, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.RESIDENT
        assert all(np.array_equal(x, y) for x, y in zip(full_a[0].rows, file_a[0].rows))
        # The on-disk cache: a fresh RAM budget of 0, files only.
        eng.set_state_cache(0, tmp_path / "states", "test")
        eng.evict_resident()
        eng.evaluate(a, branches, Want.HIDDEN)
        eng.evaluate(b, branches, Want.HIDDEN)
        disk_a = eng.evaluate(a, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.DISK
        assert all(np.array_equal(x, y) for x, y in zip(full_a[0].rows, disk_a[0].rows))
        name = f"{g.state_key('test', a):016x}.state"
        assert (tmp_path / "states" / name).exists()
        # The API's bytes (serialised from the pinned staging buffer) and the
        # cache's file (SavedState::to_bytes) are the same GRWS1 bytes.
        assert (tmp_path / "states" / name).read_bytes() == eng.save_state(a, "test")


def test_branches_do_not_see_each_other():
    """reference.rs:533-562: a branch's rows are bit-equal whatever its
    siblings are."""
    for cfg, lin, emb in [(gemma3_tiny(), g.F16, g.F16), (gguf_tiny(), g.Q8, g.Q8), (gguf_tiny(8, 2), g.Q4, g.Q8)]:
        eng, _, _, _ = build(cfg, 11, lin, emb, oracle_models=False)
        prefix = [2, 4, 6, 8]
        a = BranchTokens([10, 11, 12], [2])
        b1 = BranchTokens([20, 21, 22, 23], [3])
        b2 = BranchTokens([30, 31], [1])
        with_b1 = eng.evaluate(prefix, [a, b1], Want.HIDDEN)
        with_b2 = eng.evaluate(prefix, [a, b2], Want.HIDDEN)
        alone = eng.evaluate(prefix, [a], Want.HIDDEN)
        assert np.array_equal(with_b1[0].rows[0], with_b2[0].rows[0])
        assert np.array_equal(with_b1[0].rows[0], alone[0].rows[0])


def test_logits_are_hidden_times_embedding():
    """reference.rs:564-598 (Gemma 3 has no softcap)."""
    for cfg, lin, emb in [(gemma3_tiny(), g.F16, g.F16), (gguf_tiny(), g.Q8, g.Q8), (gguf_tiny(), g.Q4, g.Q4)]:
        eng, plain, _, w = build(cfg, 3, lin, emb)
        prefix = [2, 1, 3]
        branches = [BranchTokens([4, 5], [1])]
        hidden = eng.evaluate(prefix, branches, Want.HIDDEN)[0].rows[0]
        logits = eng.evaluate(prefix, branches, Want.LOGITS)[0].rows[0]
        expected = plain.logits(hidden[None, :])[0]
        scale = max(float(np.max(np.abs(expected))), 1.0)
        assert np.max(np.abs(logits - expected)) / scale < 1e-3
        labels = [1, 7, 3, 30]
        lab = eng.evaluate(prefix, branches, Want.LABELS, labels)[0].rows[0]
        assert np.array_equal(lab, logits[labels])


# The reference bounds batched rows by 1e-4 of separate ones
# (reference.rs:720-735).  Here they are bit-equal: the engine starts every
# group after the first on a key tile and query tile (align_groups), so a
# group meets its keys in the same tiles as alone, and the kernel's
# whole-power-of-two running max makes the remaining differences (other
# maxima) exact powers of two.
GROUPS_TOL = 0.0


def test_groups_match_separate_passes():
    """reference.rs:612-715: several requests in one pass give each the rows
    it gets alone (bit-equal here, within 1e-4 in the reference); the batch
    restores / decodes / remembers prefixes as the reference's admit + run
    do."""
    for cfg, lin, emb in [(gemma3_tiny(), g.F16, g.F16), (gguf_tiny(), g.Q4, g.Q8), (gguf_tiny(8, 2), g.Q4, g.Q8)]:
        eng, _, _, _ = build(cfg, 19, lin, emb, oracle_models=False)
        eng.set_state_cache(64 << 20, None, "test")
        prefixes = [[2, 5, 9, 14, 20, 31, 7, 8, 3], [2, 3, 4], [2, 22, 4, 6, 9, 9, 14, 1, 30, 31, 5]]
        branches = [
            [BranchTokens([11, 12, 13, 14, 15], [1, 4]), BranchTokens([30, 31, 32], [0, 2])],
            [BranchTokens([33, 34, 35, 36, 37, 38], [5])],
            [BranchTokens([7, 8], [1]), BranchTokens([11, 12, 13, 14, 15, 16, 17], [3, 6]),
             BranchTokens([1, 2, 3], [2])],
        ]
        groups = [Group(p, b) for p, b in zip(prefixes, branches)]
        for want in (Want.HIDDEN, Want.LOGITS):
            alone = []
            for gr in groups:
                eng.evict_resident()
                alone.append(eng.evaluate(gr.prefix, gr.branches, want))
            eng.evict_resident()
            together = eng.evaluate_groups(groups, want)
            for i, (a, t) in enumerate(zip(alone, together)):
                assert len(t.branches) == len(a)
                for x, y in zip(a, t.branches):
                    assert_close(x.rows, y.rows, f"group {i} in the batch", GROUPS_TOL)
            assert together[0].prefix_source == PrefixSource.RAM
            assert together[1].prefix_source == PrefixSource.DECODED
            assert together[2].prefix_source == PrefixSource.DECODED
            assert eng.is_resident(prefixes[0])
            eng.evaluate(prefixes[1], branches[1], want)
            again = eng.evaluate_groups(groups, want)
            assert again[1].prefix_source == PrefixSource.RESIDENT
            for i, (a, t) in enumerate(zip(alone, again)):
                for x, y in zip(a, t.branches):
                    assert_close(x.rows, y.rows, f"group {i} with group 1 resident", GROUPS_TOL)
            eng.evaluate(prefixes[1], branches[1], want)
            from_cache = eng.evaluate(prefixes[2], branches[2], want)
            assert eng.prefix_source() == PrefixSource.RAM
            for x, y in zip(alone[2], from_cache):
                assert_close(x.rows, y.rows, "group 2 from the state cache", GROUPS_TOL)


def test_request_errors_are_reported_not_raised_on_device():
    """engine.rs:1503-1581: every bad request fails with an error and leaves
    the engine usable."""
    eng, _, _, _ = build(gemma3_tiny(), 5, g.F16, g.F16, capacity=32, max_rows=4, oracle_models=False)
    ok = eng.evaluate([2, 3], [BranchTokens([4, 5], [1])], Want.HIDDEN)
    cases = [
        ([2] * 30, [BranchTokens([4, 5, 6], [0])], "capacity"),
        ([2, 3], [BranchTokens([4, 5], [0, 1])] * 3, "rows"),
        ([2, 3], [BranchTokens([40], [0])], "vocabulary"),
        ([2, 3], [BranchTokens([4, 5], [2])], "past"),
    ]
    for prefix, branches, what in cases:
        with pytest.raises(g.OmgError) as e:
            eng.evaluate(prefix, branches, Want.HIDDEN)
        assert what in e.value.message, e.value.message
    with pytest.raises(g.OmgError):
        eng.evaluate([2], [BranchTokens([3], [0])] * 4096, Want.HIDDEN)
    with pytest.raises(g.OmgError):
        eng.evaluate_groups([], Want.HIDDEN)
    again = eng.evaluate([2, 3], [BranchTokens([4, 5], [1])], Want.HIDDEN)
    assert np.array_equal(ok[0].rows[0], again[0].rows[0])


def test_open_dir_loads_an_exported_directory(tmp_path):
    """backend.rs:28-71 over the tools/export_wgpu_gguf.py layout."""
    cfg = gguf_tiny()
    w = g.Weights.synth(cfg, 23, g.Q4, g.Q8)
    g.export_dir(w, tmp_path / "model")
    a = g.Engine.new(w, 64, 8)
    b = g.Engine.open_dir(tmp_path / "model", 64, 8)
    prefix, branches = [2, 5, 9], [BranchTokens([4, 6, 8], [2])]
    ra = a.evaluate(prefix, branches, Want.HIDDEN)[0].rows[0]
    rb = b.evaluate(prefix, branches, Want.HIDDEN)[0].rows[0]
    assert np.array_equal(ra, rb)


def test_split_k_products_match_cpu_reference():
    """The deep o / down products that split K (output width 1536 > 1280,
    K 4096: down in 2 ranges summed by the residual norm) against the
    oracle, and rows over the resident prefix still bit-equal."""
    cfg = gguf_tiny(vocab=64, d=1536, layers=2, ff=4096, sliding=[True, False])
    check_hidden(cfg, 5, g.Q4, g.Q8)
    eng, _, _, _ = build(cfg, 5, g.Q4, g.Q8, oracle_models=False)
    full = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    again = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.RESIDENT
    for a, b in zip(full, again):
        assert all(np.array_equal(x, y) for x, y in zip(a.rows, b.rows))


def group_rows(model: oracle.Model, groups):
    """The oracle's rows at every wanted position of a multi-group request,
    in (group, branch, want) order: the groups packed one after another,
    sequence ids (group << 12) | (branch + 1) (engine.rs:24, 1512-1571)."""
    ids, pos, seq, at = [], [], [], []
    for gi, gr in enumerate(groups):
        ids += list(gr.prefix)
        pos += list(range(len(gr.prefix)))
        seq += [gi << 12] * len(gr.prefix)
        rows = []
        for bi, b in enumerate(gr.branches):
            start = len(ids)
            ids += list(b.tokens)
            pos += [len(gr.prefix) + j for j in range(len(b.tokens))]
            seq += [(gi << 12) | (bi + 1)] * len(b.tokens)
            rows.append([start + w for w in b.want])
        at.append(rows)
    hidden = model.forward(np.array(ids, np.uint32), np.array(pos, np.int32), np.array(seq, np.int32))
    return [[[hidden[i] for i in r] for r in g_rows] for g_rows in at]


def golden_groups():
    """The multi-group request of the transformers fixture
    (tests/golden/hf_gemma3.npz, gguf_q8_groups) with its config and seed."""
    import json
    from pathlib import Path

    z = np.load(Path(__file__).parent / "golden" / "hf_gemma3.npz")
    cfg = z["gguf_q8_groups/config"].tobytes().decode()
    seed, lin, emb = (int(x) for x in z["gguf_q8_groups/meta"])
    req = json.loads(z["gguf_q8_groups/request"].tobytes().decode())
    groups = [Group(p, [BranchTokens(b, list(range(len(b)))) for b in br]) for p, br in req]
    return cfg, seed, lin, emb, groups, z["gguf_q8_groups/hidden"]


def test_groups_match_cpu_reference():
    """reference.rs:616-715 checks a batch of groups against the same groups
    run apart; here the batch is checked against the oracle itself: the
    transformers fixture's two-group request (every branch position
    wanted) and a random three-group request with longer prefixes, each
    within the reference's 2e-2 of the f32 forward and 4e-3 of the forward
    with the kernel's rounding points, and the fixture's float64 rows."""
    cfg, seed, lin, emb, groups, hf = golden_groups()
    eng, plain, _, w = build(cfg, seed, lin, emb)
    ts = list(w.tensors())
    out = eng.evaluate_groups(groups, Want.HIDDEN)
    got = [[r for r in b.rows] for go in out for b in go.branches]
    exp = [b for gr in group_rows(plain, groups) for b in gr]
    tiled = [b for gr in group_rows(tiled_oracle(cfg, ts, 64), groups) for b in gr]
    assert worst_rel(got, exp) < 2e-2 and worst_rel(got, tiled) < 4e-3
    # the fixture holds every token's row in request order
    at, hf_rows = 0, []
    for gr in groups:
        at += len(gr.prefix)
        for b in gr.branches:
            hf_rows.append([hf[at + j] for j in range(len(b.tokens))])
            at += len(b.tokens)
    assert worst_rel(got, hf_rows) < 2e-2

    rng = np.random.default_rng(8)
    cfg = gguf_tiny(8, 2, window=9)
    eng, plain, _, w = build(cfg, 31, g.Q4, g.Q8, capacity=512)
    groups = [Group(rng.integers(0, 64, p).tolist(),
                    [BranchTokens(rng.integers(0, 64, n).tolist(), [0, n - 1]) for n in ns])
              for p, ns in ((70, (5, 17)), (33, (9,)), (101, (3, 12, 8)))]
    out = eng.evaluate_groups(groups, Want.HIDDEN)
    got = [[r for r in b.rows] for go in out for b in go.branches]
    exp = [b for gr in group_rows(plain, groups) for b in gr]
    tiled = [b for gr in group_rows(tiled_oracle(cfg, list(w.tensors()), 512), groups) for b in gr]
    print(f"groups: rel diff vs f32 {worst_rel(got, exp):.2e}, vs kernel rounding {worst_rel(got, tiled):.2e}")
    assert worst_rel(got, exp) < 2e-2 and worst_rel(got, tiled) < 4e-3


def test_label_lse_readout():
    """Readout::distribution's inputs (readout.rs:124-146) without the full
    row: LABELS_LSE returns the label logits, bit-equal to the LOGITS
    row's columns, then log_sum_exp of the whole row (math.rs:13-17)
    within 1e-5 relative of the float64 value from that row; candidate
    mass and probabilities match the oracle's label readout of the
    oracle's own logits within the readout bar."""
    for cfg, lin, emb in [(gguf_tiny(vocab=64), g.Q4, g.Q8), (gemma3_tiny(), g.F16, g.F16)]:
        eng, plain, _, w = build(cfg, 5, lin, emb)
        prefix, branches = [2, 5, 9, 14, 20], [BranchTokens([11, 12, 13], [0, 2]), BranchTokens([30, 31], [1])]
        labels = [3, 7, 1, 30, 12]
        full = eng.evaluate(prefix, branches, Want.LOGITS)
        lse = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
        hid = oracle_rows(plain, prefix, branches)
        for fo, lo, ho in zip(full, lse, hid):
            for row, got, h in zip(fo.rows, lo.rows, ho):
                assert got.shape == (len(labels) + 1,)
                assert np.array_equal(got[:-1], row[labels])
                r64 = row.astype(np.float64)
                m = r64.max()
                exp_lse = m + np.log(np.exp(r64 - m).sum())
                assert abs(got[-1] - exp_lse) <= 1e-5 * max(1.0, abs(exp_lse))
                # readout.rs:139-146 from these k + 1 floats vs the oracle's readout of its own row
                mass = np.exp(oracle.log_sum_exp(got[:-1]) - float(got[-1]))
                _, probs, exp_mass = oracle.label_readout(plain.logits(np.asarray(h)[None, :])[0], labels)
                assert abs(mass - exp_mass) < 2e-2
                assert np.max(np.abs(oracle.softmax(got[:-1]) - probs)) < 2e-2


def test_logits_many_rows_and_wide_rows():
    """The logits kernel's edges: more readout rows than one pass of the
    kernel takes (44 rows: three passes of 16), a model width spanning two
    staged K chunks (d 576 = 512 + 64) and a vocabulary that ends inside a
    workgroup's 64 columns (300).  Every row against the oracle's logits
    of the engine's own hidden rows (reference.rs:564-598's 1e-3 of the
    scale); label columns and LABELS_LSE's columns bit-equal to the full
    row; the log-sum-exp within 1e-5 of the float64 one."""
    cfg = gemma3_tiny(d=576, vocab=300)
    eng, plain, _, w = build(cfg, 12, g.F16, g.F16, max_rows=48)
    rng = np.random.default_rng(3)
    prefix = rng.integers(0, 300, 9).tolist()
    branches = [BranchTokens(rng.integers(0, 300, n).tolist(), list(range(n))) for n in (12, 15, 17)]
    hid = eng.evaluate(prefix, branches, Want.HIDDEN)
    full = eng.evaluate(prefix, branches, Want.LOGITS)
    labels = [0, 299, 64, 63, 7, 128, 250]
    lab = eng.evaluate(prefix, branches, Want.LABELS, labels)
    lse = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    nrows = 0
    for ho, fo, la, lo in zip(hid, full, lab, lse):
        for h, row, lr, ls in zip(ho.rows, fo.rows, la.rows, lo.rows):
            nrows += 1
            exp = plain.logits(np.asarray(h)[None, :])[0]
            assert np.max(np.abs(row - exp)) <= 1e-3 * max(float(np.max(np.abs(exp))), 1.0)
            assert np.array_equal(lr, row[labels]) and np.array_equal(ls[:-1], row[labels])
            r64 = row.astype(np.float64)
            m = r64.max()
            exp_lse = m + np.log(np.exp(r64 - m).sum())
            assert abs(ls[-1] - exp_lse) <= 1e-5 * max(1.0, abs(exp_lse))
    assert nrows == 44


def test_refused_request_leaves_resident_prefix_intact():
    """A request refused for a bad label id changes nothing on the device: a
    later pass over the resident prefix equals a fresh pass.  A prepared
    measurement pass that overwrote the cache rows drops the resident
    prefix instead of leaving it stale."""
    eng, _, _, _ = build(gguf_tiny(), 9, g.Q4, g.Q8, oracle_models=False)
    a, b = [2, 5, 9, 14, 20, 31, 7], [3, 3, 4, 1]
    branches = [BranchTokens([11, 12, 13], [2])]
    first = eng.evaluate(a, branches, Want.HIDDEN)
    for bad in ([1, 999], [64]):
        with pytest.raises(g.OmgError):
            eng.evaluate(b, branches, Want.LABELS, bad)
    assert eng.is_resident(a)
    again = eng.evaluate(a, branches, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.RESIDENT
    assert np.array_equal(first[0].rows[0], again[0].rows[0])
    eng.prepare([Group(b, branches)], Want.HIDDEN)
    eng.launch()
    eng.sync()
    assert not eng.is_resident(a)
    third = eng.evaluate(a, branches, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.DECODED
    assert np.array_equal(first[0].rows[0], third[0].rows[0])


@pytest.mark.parametrize("heads,kv", [(4, 1), (8, 2), (2, 2)])
def test_long_groups_bit_equal_to_separate_passes(heads, kv):
    """Groups long enough that their key ranges are cut into chunks (256
    keys on sliding layers, 512 on global ones), batched after a resident
    prefix of odd length: every group's rows are bit-equal to its rows
    alone (chunks count from the group's aligned first row)."""
    rng = np.random.default_rng(17)
    cfg = gguf_tiny(heads, kv, window=300)
    eng, _, _, _ = build(cfg, 37, g.Q4, g.Q8, capacity=3072, oracle_models=False)
    groups = [Group(rng.integers(0, 64, p).tolist(),
                    [BranchTokens(rng.integers(0, 64, n).tolist(), [0, n - 1]) for n in ns])
              for p, ns in ((333, (21, 5)), (701, (40,)), (517, (9, 30, 3)), (3, (7,)))]
    alone = []
    for gr in groups:
        eng.evict_resident()
        alone.append(eng.evaluate(gr.prefix, gr.branches, Want.HIDDEN))
    eng.evaluate(groups[3].prefix, groups[3].branches, Want.HIDDEN)  # group 3 resident: base 3
    together = eng.evaluate_groups(groups, Want.HIDDEN)
    assert together[3].prefix_source == PrefixSource.RESIDENT
    for i, (a, t) in enumerate(zip(alone, together)):
        for x, y in zip(a, t.branches):
            for r, s in zip(x.rows, y.rows):
                assert np.array_equal(r, s), f"group {i}"


def test_graph_replay_matches_eager_pass():
    """omg_pass_graph: the prepared pass captured once and replayed gives
    the eager launch's rows bit for bit on every replay, with other eager
    work (another engine's passes) and synchronisations between replays;
    the same rows as evaluate; a new prepare drops the graph."""
    eng, _, _, _ = build(gguf_tiny(8, 2, window=9), 41, g.Q4, g.Q8, capacity=512, oracle_models=False)
    other, _, _, _ = build(gemma3_tiny(), 3, g.F16, g.F16, oracle_models=False)
    rng = np.random.default_rng(5)
    prefix = rng.integers(0, 64, 300).tolist()
    branches = [BranchTokens(rng.integers(0, 64, n).tolist(), [n - 1]) for n in (9, 17, 4)]
    labels = [3, 9, 27, 40]
    ref = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    eng.evict_resident()
    eng.prepare([Group(prefix, branches)], Want.LABELS_LSE, labels)
    eng.launch()
    eager = eng.read_prepared(1 << 12)
    assert np.array_equal(eager.reshape(3, 5), np.stack([b.rows[0] for b in ref]))
    eng.graph(True)
    for rep in range(4):
        eng.launch()
        got = eng.read_prepared(1 << 12)
        assert np.array_equal(got, eager), f"replay {rep}"
        other.evaluate([2, 3, 4], [BranchTokens([5, 6], [1])], Want.HIDDEN)
        other.sync()
    eng.prepare([Group(prefix[:100], branches)], Want.LABELS_LSE, labels)  # drops the graph
    eng.launch()
    short = eng.read_prepared(1 << 12)
    assert not np.array_equal(short, eager)


def test_evaluate_cancels_a_prepared_pass():
    """A prepared pass reads inputs that any evaluate or state restore
    uploads over: after one, launching, capturing or reading the prepared
    pass is refused ("no prepared pass") until the next prepare, and the
    engine still answers correctly."""
    eng, _, _, _ = build(gguf_tiny(8, 2, window=9), 43, g.Q4, g.Q8, capacity=256, oracle_models=False)
    rng = np.random.default_rng(8)
    prefix = rng.integers(0, 64, 40).tolist()
    branches = [BranchTokens(rng.integers(0, 64, n).tolist(), [n - 1]) for n in (5, 7)]
    labels = [3, 9, 27]
    ref = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    saved = eng.save_state(prefix, "t")
    for interrupt in ("evaluate", "restore", "pointer-free evaluate without labels"):
        eng.evict_resident()
        eng.prepare([Group(prefix, branches)], Want.LABELS_LSE, labels)
        eng.launch()
        assert np.array_equal(eng.read_prepared(64).reshape(2, 4), np.stack([b.rows[0] for b in ref]))
        if interrupt == "evaluate":
            eng.evaluate(prefix[:7], branches[:1], Want.LABELS_LSE, labels[:1])
        elif interrupt == "restore":
            eng.restore_state(saved, "t")
        else:
            eng.evaluate([1, 2], [BranchTokens([3], [0])], Want.HIDDEN)
        for call in (eng.launch, lambda: eng.graph(True), lambda: eng.read_prepared(64)):
            with pytest.raises(L.OmgError, match="no prepared pass"):
                call()
    eng.evict_resident()
    again = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
    for a, b in zip(ref, again):
        assert np.array_equal(a.rows[0], b.rows[0])


@pytest.mark.parametrize("model,prefix_len,heads,kv", [("gemma3", 2000, 4, 1), ("gemma3", 2000, 8, 2),
                                                       ("gemma3-wide", 2000, 4, 1), ("gemma4", 2000, 4, 1),
                                                       ("gemma3", 8300, 8, 2), ("gemma3", 12400, 8, 2)])
def test_pass_split_over_streams_is_bit_equal(model, prefix_len, heads, kv):
    """A long pass runs as consecutive row ranges on streams of their own
    (from 1,025 rows two ranges cut at 55%, or three cut at 40% and 72%
    for models 1,024 wide and for passes from 12,288 rows), each range's
    attention
    waiting for the earlier ranges' K/V of the same layer.  Its rows are bit
    for bit those of the same pass as one range (profiling runs passes as
    one range), of the branches over the resident prefix, and of a captured
    graph of the split pass replayed several times.  At 2,000 tokens with
    one KV head the second range (under 1,024 rows) runs 2-wave attention
    items on the sliding layers while the first runs 4-wave ones, at the
    same time: their chunk partials must not share memory.  The Gemma 4
    model's layers differ in width (head_dim 256 / 512, double-wide MLP),
    and a range runs one layer while the other runs the next: their rows in
    the per-row buffers must not meet either."""
    if model == "gemma4":
        cfg = gemma4_tiny(heads, kv, window=37, vocab=64)
    else:
        cfg = gguf_tiny(heads, kv, window=37, vocab=64, **({"d": 1024} if model == "gemma3-wide" else {}))
    eng, _, _, _ = build(cfg, 47, g.Q4, g.Q8, capacity=prefix_len + 256, oracle_models=False)
    rng = np.random.default_rng(prefix_len)
    prefix = rng.integers(0, 64, prefix_len).tolist()
    branches = [BranchTokens(rng.integers(0, 64, n).tolist(), [0, n - 1]) for n in (9, 40, 17)]
    split = eng.evaluate(prefix, branches, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.DECODED
    eng.evict_resident()
    eng.profile(True)
    one = eng.evaluate(prefix, branches, Want.HIDDEN)
    eng.profile(False)
    warm = eng.evaluate(prefix, branches, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.RESIDENT
    for a, b, c in zip(split, one, warm):
        for x, y, z in zip(a.rows, b.rows, c.rows):
            assert np.array_equal(x, y), "split pass differs from the one-range pass"
            assert np.array_equal(x, z), "split pass differs from the branches over the resident prefix"
    eng.evict_resident()
    eng.prepare([Group(prefix, branches)], Want.HIDDEN)
    eng.graph(True)
    exp = np.concatenate([r for b in split for r in b.rows])
    for rep in range(3):
        eng.launch()
        got = eng.read_prepared(1 << 14)
        assert np.array_equal(got, exp), f"graph replay {rep}"


@pytest.mark.parametrize("case", ["split-global", "split-sliding", "short", "deep-k", "groups", "gemma4-split",
                                  "gemma4-short"])
def test_last_layer_on_answer_rows_is_bit_equal(case):
    """The last layer past its attention runs for the read-out rows only
    (the query tiles that hold them, then o, the norms, gate/up and down on
    the gathered rows) unless the engine is told to run it for every row,
    as the reference does: the rows a pass returns are bit for bit the same
    — split passes on two streams whose last layer is global or sliding, a
    short pass, deep-K down products (a piece per workgroup on the gathered
    rows, added in registers in the full long pass), several groups, and
    Gemma 4 (a head_dim 512 last layer reading shared K/V, the per-layer
    input block on the gathered rows) — and so are the label logits and
    log-sum-exp, cold and over the resident prefix."""
    rng = np.random.default_rng(61)
    if case.startswith("gemma4"):
        cfg = gemma4_tiny(4, 1, window=37, vocab=64)
        plen, sizes = (2000 if case == "gemma4-split" else 120), (9, 40, 17)
    elif case == "deep-k":
        cfg = gemma3_tiny(d=2304, ff=4096, layers=2, sliding=[True, False])
        plen, sizes = 600, (12, 9)  # 621 rows: the full pass adds the pieces in registers
    elif case == "split-sliding":
        cfg = gguf_tiny(4, 1, window=37, vocab=64, layers=3, sliding=[False, True, True])
        plen, sizes = 2000, (9, 40, 17)
    else:
        cfg = gguf_tiny(4, 1, window=37, vocab=64)
        plen, sizes = (2000, (9, 40, 17)) if case in ("split-global", "groups") else (120, (9, 40, 17))
    vocab = 40 if case == "deep-k" else 64
    eng, _, _, _ = build(cfg, 53, g.Q4, g.Q8, capacity=2 * plen + 256, max_rows=32, oracle_models=False)
    prefix = rng.integers(0, vocab, plen).tolist()
    branches = [BranchTokens(rng.integers(0, vocab, n).tolist(), [0, n // 2, n - 1]) for n in sizes]
    labels = list(range(1, 9))

    def passes():
        if case == "groups":
            other = rng.integers(0, vocab, 300).tolist()
            groups = [Group(prefix, branches), Group(other, branches[:2])]
            eng.evict_resident()
            return [eng.evaluate_groups(groups, Want.HIDDEN)]
        eng.evict_resident()
        cold = eng.evaluate(prefix, branches, Want.HIDDEN)
        warm = eng.evaluate(prefix, branches, Want.HIDDEN)
        assert eng.prefix_source() == PrefixSource.RESIDENT
        eng.evict_resident()
        lse = eng.evaluate(prefix, branches, Want.LABELS_LSE, labels)
        return [cold, warm, lse]

    def gathers() -> bool:  # whether a (profiled, one-range) pass runs the answer-row last layer
        eng.profile(True)
        eng.evaluate(prefix, branches, Want.HIDDEN)
        ran = "gather_out" in eng.profile_report()
        eng.profile(False)
        return ran

    state = rng.bit_generator.state
    answer = passes()
    assert gathers()
    eng.full_last_layer(True)
    rng.bit_generator.state = state
    full = passes()
    assert not gathers()
    eng.full_last_layer(False)
    def rows(out):  # a pass's rows in order, for branch or group outputs
        return [r for o in out for b in (o.branches if hasattr(o, "branches") else [o]) for r in b.rows]

    for a, b in zip(answer, full):
        ra, rb = rows(a), rows(b)
        assert len(ra) == len(rb) > 0
        for u, v in zip(ra, rb):
            assert np.array_equal(u, v), f"{case}: answer-row last layer differs from the full one"
