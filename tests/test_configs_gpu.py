"""The BASELINE.json configurations on the GPU against the CPU oracle
(crates/omg-wgpu/tests/reference.rs restated), at their real shapes.

C1 and C2 run the whole configuration through the oracle; C3 (1B) runs the
500-token state through the oracle with the pointer readout and checks the
2,000-token state by the properties a pass must have (resident and restored
states bit-equal to the full pass); C5 (4B) checks the full 8,000 + 208 x 40
pass by those properties and isolation, and the oracle on the same shapes
with two layers.  The readout bar is BASELINE.json's: after softmax within
2e-2 of the oracle, identical argmax per question."""
from __future__ import annotations


import numpy as np
import pytest

import grande_amd as g
import oracle
from grande_amd import BranchTokens, Want
from tests.common import rel_diff, tiled_oracle

pytestmark = pytest.mark.gpu

LABELS = g.LABEL_IDS
SEED = 0x5EED


def request(spec, seed, state=None):
    rng = np.random.default_rng(seed)
    vocab = spec["model"]["vocab"]
    p = spec["state"] if state is None else state
    prefix = rng.integers(0, vocab, p).tolist()
    bt = spec["branch_tokens"]
    branches = [BranchTokens(rng.integers(0, vocab, bt).tolist(), [bt - 1]) for _ in range(spec["branches"])]
    return prefix, branches


def oracle_wanted_rows(model, prefix, branches):
    ids, pos, seq = oracle.pack_single(prefix, branches)
    hidden = model.forward(ids, pos, seq)
    rows, at = [], len(prefix)
    for b in branches:
        rows.append(hidden[at + b.want[0]])
        at += len(b.tokens)
    return np.stack(rows)


def assert_readout(got_logits, exp_logits, what):
    """within 2e-2 after softmax, identical argmax."""
    worst = 0.0
    for i, (a, b) in enumerate(zip(got_logits, exp_logits)):
        pa, pb = oracle.softmax(a), oracle.softmax(b)
        worst = max(worst, float(np.max(np.abs(pa - pb))))
        assert int(np.argmax(pa)) == int(np.argmax(pb)), f"{what}: question {i} argmax"
    print(f"{what}: max |dp| {worst:.2e}")
    assert worst <= 2e-2, f"{what}: max |dp| {worst}"


def label_config_check(name):
    spec = g.BASELINE_CONFIGS[name]
    cfg = g.config_json(**spec["model"])
    prefix, branches = request(spec, SEED)
    w = g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"])
    eng = g.Engine.new(w, len(prefix) + sum(len(b.tokens) for b in branches) + 64, len(branches))
    got = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.LABELS, LABELS)])
    hid = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.HIDDEN)])
    model = oracle.Model(cfg, list(w.tensors()))
    rows = oracle_wanted_rows(model, prefix, branches)
    exp = model.logits(rows)[:, LABELS]
    assert max(rel_diff(h, r) for h, r in zip(hid, rows)) < 2e-2
    assert_readout(got, exp, name)


def test_c1_270m_q8_label_readout():
    label_config_check("c1")


def test_c2_270m_q4_label_readout():
    label_config_check("c2")


def test_c2_270m_q4_label_lse_route():
    """The metric's configuration through the route the bench times
    (OMG_WANT_LABELS_LSE on a cold pass: 26 label logits and the full
    row's log-sum-exp per question), at full size: the label logits are
    bit-equal to the same columns of the full-vocabulary logits, the
    log-sum-exp is within 1e-5 of the float64 value over those logits, the
    candidate mass and the label distribution (readout.rs:124-146) within
    2e-2 of the oracle's with the same argmax, and the hidden rows within
    4e-3 of the forward with the kernel's rounding points."""
    spec = g.BASELINE_CONFIGS["c2"]
    cfg = g.config_json(**spec["model"])
    prefix, branches = request(spec, SEED)
    cap = len(prefix) + sum(len(b.tokens) for b in branches) + 64
    w = g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"])
    eng = g.Engine.new(w, cap, len(branches))
    lse_rows = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.LABELS_LSE, LABELS)])
    assert eng.prefix_source() == g.PrefixSource.DECODED
    eng.evict_resident()
    full = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.LOGITS)])
    eng.evict_resident()
    hid = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.HIDDEN)])
    assert lse_rows.shape == (len(branches), len(LABELS) + 1)
    assert np.array_equal(lse_rows[:, :-1], full[:, LABELS])
    lse64 = np.array([oracle.log_sum_exp(r.astype(np.float64)) for r in full])
    assert np.max(np.abs(lse_rows[:, -1] - lse64) / np.maximum(np.abs(lse64), 1.0)) < 1e-5
    ts = list(w.tensors())
    tiled = oracle_wanted_rows(tiled_oracle(cfg, ts, cap), prefix, branches)
    dt = max(rel_diff(h, r) for h, r in zip(hid, tiled))
    model = oracle.Model(cfg, ts)
    rows = oracle_wanted_rows(model, prefix, branches)
    exp_full = model.logits(rows)
    dmass = 0.0
    for i in range(len(branches)):
        _, _, mass_c = oracle.label_readout(exp_full[i], LABELS)
        mass_g = float(np.exp(oracle.log_sum_exp(lse_rows[i, :-1].astype(np.float64)) - float(lse_rows[i, -1])))
        dmass = max(dmass, abs(mass_g - mass_c))
    print(f"c2 LSE route: hidden vs kernel rounding {dt:.2e}, candidate mass |d| {dmass:.2e}")
    assert dt < 4e-3
    assert dmass < 2e-2
    assert_readout(lse_rows[:, :-1], exp_full[:, LABELS], "c2 LSE route")


def pointer_head(d: int, options: int = 52) -> np.ndarray:
    """The seeded [d x 52] f32 pointer head of BASELINE.json configs[2]."""
    return (np.random.default_rng(52).standard_normal((d, options)) / np.sqrt(d)).astype(np.float32)


def test_c3_1b_q4_pointer_readout_500_state():
    spec = g.BASELINE_CONFIGS["c3"]
    cfg = g.config_json(**spec["model"])
    prefix, branches = request(spec, SEED, state=500)
    w = g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"])
    eng = g.Engine.new(w, 500 + 12 * 32 + 64, 12)
    hid = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.HIDDEN)])
    model = oracle.Model(cfg, list(w.tensors()))
    rows = oracle_wanted_rows(model, prefix, branches)
    assert max(rel_diff(h, r) for h, r in zip(hid, rows)) < 2e-2
    head = pointer_head(spec["model"]["d"])
    assert_readout(hid @ head, rows @ head, "c3 pointer")


def test_c3_1b_q4_2000_state_resident_and_restored():
    spec = g.BASELINE_CONFIGS["c3"]
    cfg = g.config_json(**spec["model"])
    prefix, branches = request(spec, SEED + 1)
    eng = g.Engine.new(g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"]), 2000 + 12 * 32 + 64, 12)
    cold = eng.evaluate(prefix, branches, Want.HIDDEN)
    assert eng.prefix_source() == g.PrefixSource.DECODED
    warm = eng.evaluate(prefix, branches, Want.HIDDEN)
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(cold, warm))
    state = eng.save_state(prefix, "c3")
    eng.evict_resident()
    eng.restore_state(state, "c3")
    again = eng.evaluate(prefix, branches, Want.HIDDEN)
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(cold, again))
    head = pointer_head(spec["model"]["d"])
    z = np.stack([b.rows[0] for b in cold]) @ head
    assert np.isfinite(z).all()


def test_c5_4b_q4_full_pass_properties():
    """8,000-token state + 52 questions x 4 option orders (208 branches of
    40): the warm pass over the resident state and a pass with other
    sibling branches give bit-equal rows; the order-averaged readout is a
    distribution per question (crates/omg-core/src/plan.rs:223-303)."""
    spec = g.BASELINE_CONFIGS["c5"]
    cfg = g.config_json(**spec["model"])
    prefix, branches = request(spec, SEED)
    eng = g.Engine.new(g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"]), 8000 + 208 * 40 + 64, 208)
    cold = eng.evaluate(prefix, branches, Want.LABELS, LABELS)
    warm = eng.evaluate(prefix, branches, Want.LABELS, LABELS)
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(cold, warm))
    rng = np.random.default_rng(1)
    others = [BranchTokens(rng.integers(0, spec["model"]["vocab"], 40).tolist(), [39]) if i % 2 else b
              for i, b in enumerate(branches)]
    mixed = eng.evaluate(prefix, others, Want.LABELS, LABELS)
    assert all(np.array_equal(a.rows[0], b.rows[0]) for i, (a, b) in enumerate(zip(cold, mixed)) if i % 2 == 0)
    # the first questions alone on the resident state (their rows keep their
    # cache rows): 40- and 120-row passes, whose deep-K down products run a
    # K chunk per workgroup (the long passes above fold the chunks in
    # registers) — the same rows
    for n in (1, 3):
        few = eng.evaluate(prefix, branches[:n], Want.LABELS, LABELS)
        assert eng.prefix_source() == g.PrefixSource.RESIDENT
        assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(few, cold[:n])), n
    k = 4  # options per question; 4 orders each
    orders = np.array(oracle.option_orders(k, 4))
    logits = np.stack([b.rows[0][:k] for b in cold]).reshape(52, 4, k)
    for q in range(52):
        folded = oracle.fold_mean(orders, logits[q])
        p = oracle.softmax(folded)
        assert np.isfinite(folded).all() and abs(p.sum() - 1.0) < 1e-9


def test_c5_shapes_two_layers_match_cpu_reference():
    """The 4B shapes (d 2560, 8 query / 4 KV heads, ff 10240, window 1024)
    through the oracle, with two layers (one sliding, one global)."""
    m = dict(g.BASELINE_CONFIGS["c5"]["model"], layers=2)
    cfg = g.config_json(**m, sliding=[True, False])
    spec = dict(g.BASELINE_CONFIGS["c5"], branches=8, state=1500)
    prefix, branches = request(spec, SEED)
    w = g.Weights.synth(cfg, SEED, g.Q4, g.Q4)
    eng = g.Engine.new(w, 1500 + 8 * 40 + 64, 8)
    hid = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.HIDDEN)])
    got = np.stack([b.rows[0] for b in eng.evaluate(prefix, branches, Want.LABELS, LABELS)])
    ts = list(w.tensors())
    plain = oracle.Model(cfg, ts)
    rows = oracle_wanted_rows(plain, prefix, branches)
    rows16 = oracle_wanted_rows(oracle.Model(cfg, ts, gpu_rounding=True), prefix, branches)
    assert max(rel_diff(h, r) for h, r in zip(hid, rows)) < 2e-2
    assert max(rel_diff(h, r) for h, r in zip(hid, rows16)) < 4e-3
    assert_readout(got, plain.logits(rows)[:, LABELS], "c5 two layers")


def test_e2b_full_pass_properties():
    """The Gemma 4 E2B-shaped model of bench.py --config e2b at full size
    (35 layers, head_dim 256 / 512, 20 K/V-sharing double-wide layers,
    per-layer inputs, split-K down products): 2,000-token state + 12
    branches; the warm pass and a save -> evict -> restore give bit-equal
    label logits, all finite and inside the softcap."""
    spec = g.GEMMA4_CONFIGS["e2b"]
    mc = spec["model"]
    cfg = g.gemma4_config_json(**mc)
    rng = np.random.default_rng(SEED)
    prefix = rng.integers(0, mc["vocab"], spec["state"]).tolist()
    branches = [BranchTokens(rng.integers(0, mc["vocab"], bt).tolist(), [bt - 1]) for bt in spec["branch_tokens"]]
    eng = g.Engine.new(g.Weights.synth(cfg, SEED, spec["dtype"], spec["dtype"]), 2000 + 663 + 64, 16)
    cold = eng.evaluate(prefix, branches, Want.LABELS, LABELS)
    warm = eng.evaluate(prefix, branches, Want.LABELS, LABELS)
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(cold, warm))
    state = eng.save_state(prefix, "e2b")
    eng.evict_resident()
    eng.restore_state(state, "e2b")
    again = eng.evaluate(prefix, branches, Want.LABELS, LABELS)
    assert all(np.array_equal(a.rows[0], b.rows[0]) for a, b in zip(cold, again))
    z = np.stack([b.rows[0] for b in cold])
    assert np.isfinite(z).all() and np.abs(z).max() < 30.0


def test_e2b_shapes_five_layers_match_cpu_reference():
    """The E2B shapes (d 1536, 8 query heads over 1 K/V head, ff 6144 /
    12288, head_dim 512 global layer, per-layer inputs of 256) through the
    oracle, with five layers (sliding, sliding, global, sliding, global),
    the last two sharing the K/V of layers 1 and 2 with double-wide
    feed-forwards and split-K down products."""
    mc = dict(g.GEMMA4_CONFIGS["e2b"]["model"], layers=5, shared_kv_layers=2,
              sliding=[True, True, False, True, False])
    cfg = g.gemma4_config_json(**mc)
    rng = np.random.default_rng(3)
    prefix = rng.integers(0, mc["vocab"], 40).tolist()
    branches = [BranchTokens(rng.integers(0, mc["vocab"], 9).tolist(), [8]) for _ in range(3)]
    from tests.test_gemma4_gpu import check_chaotic, engine_of
    ts = list(g.Weights.synth(cfg, SEED, g.Q4, g.Q4).tensors())
    out = engine_of(cfg, ts, 128, 8).evaluate(prefix, branches, Want.HIDDEN)
    check_chaotic(out, cfg, ts, prefix, branches, 128, "E2B shapes, five layers", tiled_bar=1e-2, f32_bar=2e-2)
