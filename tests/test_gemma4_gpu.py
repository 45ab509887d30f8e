"""Gemma 4 layers on the engine against the CPU oracle (reference.rs:66-104,
415-440): head_dim 512 global layers with RoPE on a quarter of their
dims, K/V shared by the last two layers, V RMS-norm, per-layer inputs
from the [vocab, layers x P] token table, per-layer output scales and the
logit softcap — plus the reference's invariants on these configs."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
import oracle
from grande_amd import BranchTokens, PrefixSource, Want
from tests.common import (assert_close, build, gemma4_tiny, oracle_rows, rel_diff, rounding_spread, tiled_oracle,
                          worst_rel)

pytestmark = pytest.mark.gpu

PREFIX = [2, 5, 9, 14, 20, 31, 7, 8, 3, 22]
BRANCHES = [BranchTokens([11, 12, 13, 14, 15], [1, 4]), BranchTokens([30, 31, 32, 33, 34, 35, 36, 37], [0, 7])]


def check_hidden(cfg: str, seed: int, linear: int, embed: int, tol: float = 2e-2, tight: float = 1e-2,
                 prefix=PREFIX, branches=BRANCHES, capacity: int = 64):
    """reference.rs:380-407 on a Gemma 4 config: within the reference's 2e-2
    of the f32 forward.  The check against the f16-rounding forward is
    looser here than on Gemma 3 (1e-2, not 4e-3): with query scale 1 and
    normed q / k the softmax is sharp enough that rounding differences are
    amplified — the two CPU forwards alone differ by up to 4.5e-3 on these
    configs (3e-4 on the Gemma 3 ones)."""
    eng, plain, gpu_r, _ = build(cfg, seed, linear, embed, capacity=capacity)
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
    return eng, plain


def test_gemma4_q8_matches_cpu_reference():
    check_hidden(gemma4_tiny(), 7, g.Q8, g.Q8)


def test_gemma4_q4_matches_cpu_reference():
    check_hidden(gemma4_tiny(), 9, g.Q4, g.Q8)


def test_gemma4_f16_matches_cpu_reference():
    check_hidden(gemma4_tiny(), 5, g.F16, g.F16)


def test_gemma4_gqa_q4_matches_cpu_reference():
    """reference.rs:525-531: 8 query heads over 2 KV heads."""
    check_hidden(gemma4_tiny(8, 2), 11, g.Q4, g.Q8)


def engine_of(cfg: str, ts, capacity: int, max_rows: int = 16) -> g.Engine:
    b = g.EngineBuilder(cfg)
    for t in ts:
        b.push(t)
    return b.finish(capacity, max_rows)


def check_chaotic(out, cfg: str, ts, prefix, branches, capacity: int, what: str, tiled_bar: float,
                  f32_bar: float | None = None):
    """Rows of a long-prefix Gemma 4 pass on the reference's own weight
    distribution.  With query scale 1 and normed q / k over 256 / 512 dims
    the scores reach several tens and near-ties between keys are common
    over hundreds of keys, so any rounding difference is amplified layer by
    layer: the three CPU forwards that differ only in where they round
    (f32, f16 operands, f16 operands + the flash kernel's rounding) sit up
    to 4e-2 apart here (`rounding_spread`), beyond the reference's 2e-2 bar
    that holds on its short-prefix tests.  The forward with the kernel's
    own rounding points is held to a fixed bar (`tiled_bar`); the f32
    forward to `f32_bar` when given (the reference's 2e-2 where the spread
    allows it) and the f32 / f16-operand forwards otherwise within twice
    the CPU spread, so a real defect (O(1) errors, a lost mask or window)
    fails either way; the depth-limited cases in
    test_gemma4_long_prefix_by_depth hold the reference's 2e-2 bar."""
    f32, f16, tiled, spread = rounding_spread(cfg, ts, prefix, branches, capacity)
    hip = [o.rows for o in out]
    d = {k: worst_rel(hip, v) for k, v in (("f32", f32), ("f16", f16), ("tiled", tiled))}
    print(f"{what}: CPU rounding spread {spread:.2e}; GPU vs f32 {d['f32']:.2e}, "
          f"vs f16 operands {d['f16']:.2e}, vs kernel rounding {d['tiled']:.2e}")
    assert d["tiled"] < tiled_bar, f"{what}: {d['tiled']} from the kernel-rounding forward (bar {tiled_bar})"
    if f32_bar is not None:
        assert d["f32"] < f32_bar, f"{what}: {d['f32']} from the f32 forward (bar {f32_bar})"
    bound = max(2e-2, 2.0 * spread)
    for k in ("f32", "f16"):
        assert d[k] < bound, f"{what}: {d[k]} from the {k} forward (bound {bound})"


@pytest.mark.parametrize("capacity", [1024, 8192])
@pytest.mark.parametrize("heads,kv", [(8, 2), (4, 1)])
def test_gemma4_long_prefix_global_key_ranges(capacity, heads, kv):
    """A 700-token prefix on the reference's gemma4 configs and weights
    (reference.rs:66-104, 108-139): at capacity 1024 the head_dim-512 global
    layers' key ranges are cut into 384-key chunks and merged, at 8192 they
    are not (1024-key chunks).  Four layers deep the GPU rows stay within
    1.2e-2 of the forward with the kernel's own rounding points (measured
    6.4e-3 .. 9.2e-3)."""
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, 64, 700).tolist()
    branches = [BranchTokens(rng.integers(0, 64, 37).tolist(), [0, 20, 36]) for _ in range(3)]
    cfg = gemma4_tiny(heads, kv)
    ts = list(g.Weights.synth(cfg, 13, g.Q4, g.Q8).tensors())
    out = engine_of(cfg, ts, capacity).evaluate(prefix, branches, Want.HIDDEN)
    check_chaotic(out, cfg, ts, prefix, branches, capacity, f"{heads}/{kv} heads, capacity {capacity}",
                  tiled_bar=1.2e-2)


@pytest.mark.parametrize("layers", [1, 2])
@pytest.mark.parametrize("heads,kv", [(8, 2), (4, 1)])
def test_gemma4_long_prefix_by_depth(layers, heads, kv):
    """The same 700-token request and weight distribution through one global
    layer, or a sliding then a global layer (no K/V sharing): before the
    amplification compounds, the GPU rows hold the reference's 2e-2 bar
    against the f32 forward and sit within 3e-3 of the forward with the
    kernel's own rounding points (measured 2e-4 .. 1.2e-3)."""
    rng = np.random.default_rng(4)
    prefix = rng.integers(0, 64, 700).tolist()
    branches = [BranchTokens(rng.integers(0, 64, 37).tolist(), [0, 20, 36]) for _ in range(3)]
    sliding = [False] if layers == 1 else [True, False]
    cfg = gemma4_tiny(heads, kv, layers=layers, sliding=sliding, shared_kv_layers=0, ff=96, double_wide_mlp=False)
    ts = list(g.Weights.synth(cfg, 13, g.Q4, g.Q8).tensors())
    out = engine_of(cfg, ts, 1024).evaluate(prefix, branches, Want.HIDDEN)
    hip = [o.rows for o in out]
    f32 = oracle_rows(oracle.Model(cfg, ts), prefix, branches)
    tiled = oracle_rows(tiled_oracle(cfg, ts, 1024), prefix, branches)
    dp, dt = worst_rel(hip, f32), worst_rel(hip, tiled)
    print(f"{layers} layer(s), {heads}/{kv} heads: GPU vs f32 {dp:.2e}, vs kernel rounding {dt:.2e}")
    assert dp < 2e-2 and dt < 3e-3


def test_gemma4_logits_apply_softcap():
    """reference.rs:564-598: logits = cap * tanh(hidden . E^T / cap), cap 30."""
    eng, plain, _, w = build(gemma4_tiny(), 3, g.Q8, g.Q8)
    hid = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    log = eng.evaluate(PREFIX, BRANCHES, Want.LOGITS)
    emb = next(t for t in w.tensors() if t.name == "embed").to_f32().reshape(64, 64).astype(np.float64)
    for h, lo in zip(hid, log):
        for r, l in zip(h.rows, lo.rows):
            exp = 30.0 * np.tanh((np.asarray(r, np.float64) @ emb.T) / 30.0)
            assert np.max(np.abs(np.asarray(l) - exp)) <= 1e-3 * max(1.0, np.max(np.abs(exp)))
            assert np.max(np.abs(np.asarray(l))) < 30.0


@pytest.mark.parametrize("heads,kv", [(4, 1), (8, 2)])
def test_gemma4_resident_prefix_matches_full_pass(heads, kv):
    """reference.rs:432-470: a second request over the resident prefix
    reproduces the full pass bit for bit (shared K/V layers included)."""
    eng, _, _, _ = build(gemma4_tiny(heads, kv), 17, g.Q4, g.Q8, oracle_models=False)
    first = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    again = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.RESIDENT
    for a, b in zip(first, again):
        for x, y in zip(a.rows, b.rows):
            assert np.array_equal(x, y)


def test_gemma4_state_round_trip_is_exact():
    """reference.rs:472-522: save -> evict -> restore reproduces the rows."""
    eng, _, _, _ = build(gemma4_tiny(8, 2), 19, g.Q4, g.Q8, oracle_models=False)
    full = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    data = eng.save_state(PREFIX, "g4")
    eng.evict_resident()
    eng.restore_state(data, "g4")
    assert eng.is_resident(PREFIX)
    again = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    assert eng.prefix_source() == PrefixSource.RESIDENT
    for a, b in zip(full, again):
        for x, y in zip(a.rows, b.rows):
            assert np.array_equal(x, y)


def test_gemma4_branches_do_not_see_each_other():
    """reference.rs:533-562: a branch's rows do not depend on its siblings."""
    eng, _, _, _ = build(gemma4_tiny(), 11, g.Q8, g.Q8, oracle_models=False)
    both = eng.evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    eng.evict_resident()
    alone = eng.evaluate(PREFIX, BRANCHES[1:], Want.HIDDEN)
    assert_close(both[1].rows, alone[0].rows, "branch isolation", 1e-6)


def test_gemma4_open_dir_loads_the_per_layer_table(tmp_path):
    """An exported directory with per_layer_table.bin under the manifest's
    per_layer_table entry loads to the same engine."""
    cfg = gemma4_tiny()
    w = g.Weights.synth(cfg, 23, g.Q4, g.Q8)
    g.export_dir(w, tmp_path)
    a = g.Engine.new(w, 64, 16).evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    b = g.Engine.open_dir(tmp_path, 64, 16).evaluate(PREFIX, BRANCHES, Want.HIDDEN)
    for x, y in zip(a, b):
        for r, s in zip(x.rows, y.rows):
            assert np.array_equal(r, s)


@pytest.mark.parametrize("heads,kv", [(2, 2), (4, 2), (8, 1), (16, 1)])
def test_gemma4_every_head_grouping(heads, kv):
    """Every query-heads-per-K/V-head grouping of the head_dim 256 and 512
    kernels (1, 2, 8, 16 per group; 4 is covered above), on a prefix long
    enough for split key ranges, on the reference's weight distribution:
    the reference's 2e-2 bar against the f32 forward (measured 3.3e-3 ..
    7.4e-3) and the same bar against the kernel-rounding forward (measured
    3.3e-3 .. 1.3e-2)."""
    rng = np.random.default_rng(6)
    prefix = rng.integers(0, 64, 300).tolist()
    branches = [BranchTokens(rng.integers(0, 64, 21).tolist(), [0, 20]) for _ in range(2)]
    cfg = gemma4_tiny(heads, kv)
    ts = list(g.Weights.synth(cfg, 29, g.Q4, g.Q8).tensors())
    out = engine_of(cfg, ts, 512).evaluate(prefix, branches, Want.HIDDEN)
    check_chaotic(out, cfg, ts, prefix, branches, 512, f"{heads}/{kv} heads", tiled_bar=2e-2, f32_bar=2e-2)
