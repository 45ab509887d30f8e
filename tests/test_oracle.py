"""Pins of the CPU oracle (CPU only).

Every oracle function is checked against something other than a retyping
of its own formula: the reference's own unit-test answers, published test
vectors, an independent implementation (numpy's IEEE binary16, Hugging Face
transformers' Gemma 3 and Gemma 4 in float64 via tests/golden/hf_gemma3.npz
and hf_gemma4.npz), closed
forms, or answers worked out by hand from the reference's definitions.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import grande_amd as g
import oracle

from tests.common import rel_diff

GOLDEN = Path(__file__).resolve().parent / "golden" / "hf_gemma3.npz"
GOLDEN4 = Path(__file__).resolve().parent / "golden" / "hf_gemma4.npz"


# ----------------------------------------------------------- f16 rounding

def test_f16_to_f32_reference_answers():
    # crates/omg-core/src/readout.rs f16_conversion test
    assert oracle.f16_to_f32(0x3C00) == 1.0
    assert oracle.f16_to_f32(0xC000) == -2.0
    assert oracle.f16_to_f32(0x0000) == 0.0


def test_f16_to_f32_exhaustive_vs_numpy():
    bits = np.arange(1 << 16, dtype=np.uint16)
    exp = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    # Random magnitudes across the whole f16 range and beyond, both signs,
    # plus ties exactly halfway between neighbours (even and odd mantissas).
    x = (rng.standard_normal(40000) * np.exp2(rng.uniform(-26, 17, 40000))).astype(np.float32)
    h = np.arange(0, 0x7BFF, 7, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, np.inf, -np.inf],
                       np.float32)
    with np.errstate(over="ignore"):
        wants = np.concatenate([x, ties, -ties, special]).astype(np.float16).view(np.uint16)
    for v, want in zip(np.concatenate([x, ties, -ties, special]), wants):
        want = int(want)
        assert oracle.f32_to_f16(float(v)) == want, (v, hex(want))


# -------------------------------------------------------------- xorshift

def test_rng_known_answer():
    # reference.rs:17-28 by hand from state 1: 1 ^ 1<<13 = 8193,
    # ^ >>7 -> 8257, ^ <<17 -> 1082269761; (1082269761 >> 40) = 0 -> -1.0.
    v, state = oracle.rng_values(1, 1)
    assert state == 1082269761
    assert v[0] == -1.0


def test_rng_stream_vs_python_integers():
    def stream(s, n):
        out = []
        m = (1 << 64) - 1
        for _ in range(n):
            s ^= (s << 13) & m
            s ^= s >> 7
            s ^= (s << 17) & m
            out.append(np.float32(np.float32(s >> 40) / np.float32(1 << 24)) * np.float32(2) - np.float32(1))
        return np.array(out, np.float32), s

    for seed in (1, 5, 7, 19, 0xDEADBEEF):
        got, st = oracle.rng_values(seed, 500)
        exp, est = stream(seed, 500)
        assert st == est and np.array_equal(got, exp)
        assert got.min() >= -1.0 and got.max() < 1.0


# ---------------------------------------------------------- Q8_0 / Q4_0

def decode(dtype, data, scales):
    """Block decode written from the block layout (model.rs:507-529):
    Q8: int8 codes * d; Q4: 16 bytes per block, low nibble = element j,
    high nibble = element j + 16, value (code - 8) * d."""
    d = scales.view(np.float16).astype(np.float32)
    if dtype == oracle.Q8:
        return (data.view(np.int8).reshape(-1, 32).astype(np.float32) * d[:, None]).ravel()
    b = data.reshape(-1, 16)
    codes = np.concatenate([b & 15, b >> 4], axis=1).astype(np.float32)
    return ((codes - 8) * d[:, None]).ravel()


def test_quantization_roundtrips_reference_bounds():
    # reference.rs:600-610: Rng(5), 256 values at scale 0.3
    v, _ = oracle.rng_values(5, 256, 0.3)
    for dt, bound in ((oracle.Q8, 0.3 / 127 * 1.01), (oracle.Q4, 0.3 / 8 * 1.01)):
        data, scales = oracle.quantize(dt, v)
        err = np.max(np.abs(decode(dt, data, scales) - v))
        assert err < bound, (dt, err)
        got = oracle.get(dt, data, scales, v.size)
        assert np.array_equal(got, decode(dt, data, scales))


def test_q8_known_codes():
    # amax = 1 -> d = 1/127 (f16), code = round half away from zero of v*127
    v = np.zeros(32, np.float32)
    v[0], v[1], v[2], v[3], v[4] = 1.0, -1.0, 0.5 / 127, -0.5 / 127, 1.49 / 127
    data, scales = oracle.quantize(oracle.Q8, v)
    assert scales.view(np.float16)[0] == np.float16(1 / 127)
    assert data.view(np.int8)[:6].tolist() == [127, -127, 1, -1, 1, 0]
    # an all-zero block gets d = 0 and zero codes
    data, scales = oracle.quantize(oracle.Q8, np.zeros(32, np.float32))
    assert not data.any() and not scales.any()


def test_q4_known_codes():
    # The value of largest magnitude is -1 -> d = max / -8 = 0.125;
    # code = min(15, trunc(v / d + 8.5)).
    v = np.zeros(32, np.float32)
    v[0], v[1], v[2], v[17], v[18] = -1.0, 0.875, 0.9, 0.0625, 0.06
    data, scales = oracle.quantize(oracle.Q4, v)
    assert scales.view(np.float16)[0] == np.float16(0.125)
    codes = np.concatenate([data & 15, data >> 4])
    # 0.0625 / 0.125 + 8.5 = 9.0 -> 9; 0.06 -> 8.98 -> 8; 0 -> 8
    assert codes[0] == 0 and codes[1] == 15 and codes[2] == 15
    assert codes[17] == 9 and codes[18] == 8 and codes[5] == 8
    # Largest magnitude positive: d = -0.125, so +1 -> code 0 and -0.875 -> 15.
    v = np.zeros(32, np.float32)
    v[3], v[20] = 1.0, -0.875
    data, scales = oracle.quantize(oracle.Q4, v)
    assert scales.view(np.float16)[0] == np.float16(-0.125)
    codes = np.concatenate([data & 15, data >> 4])
    assert codes[3] == 0 and codes[20] == 15
    with pytest.raises(ValueError):
        oracle.quantize(oracle.Q4, np.zeros(33, np.float32))


# -------------------------------------------------------------- forward

def golden_cases(path=GOLDEN):
    z = np.load(path)
    names = sorted({k.split("/")[0] for k in z.files})
    for n in names:
        cfg = z[n + "/config"].tobytes().decode()
        seed, lin, emb = (int(x) for x in z[n + "/meta"])
        request = json.loads(z[n + "/request"].tobytes().decode())
        yield n, cfg, seed, lin, emb, request, z[n + "/hidden"]


def flat_request(request):
    """Tokens in request order with the oracle's sequence ids
    (group << 12 | branch + 1, prefix 0 within its group)."""
    ids, pos, seq = [], [], []
    for gi, (prefix, branches) in enumerate(request):
        for i, t in enumerate(prefix):
            ids.append(t), pos.append(i), seq.append(gi << 12)
        for bi, toks in enumerate(branches):
            for j, t in enumerate(toks):
                ids.append(t), pos.append(len(prefix) + j), seq.append((gi << 12) | (bi + 1))
    return np.array(ids, np.uint32), np.array(pos, np.int32), np.array(seq, np.int32)


@pytest.mark.parametrize("case", [c[0] for c in golden_cases()])
def test_forward_matches_hf_gemma3(case):
    n, cfg, seed, lin, emb, request, hidden = next(c for c in golden_cases() if c[0] == case)
    w = g.Weights.synth(cfg, seed, lin, emb)
    ts = list(w.tensors())
    ids, pos, seq = flat_request(request)
    got = oracle.Model(cfg, ts).forward(ids, pos, seq)
    assert got.shape == hidden.shape
    assert rel_diff(got, hidden) < 2e-6, rel_diff(got, hidden)
    # the GPU rounding points (f16 operands) stay within f16 precision
    got16 = oracle.Model(cfg, ts, gpu_rounding=True).forward(ids, pos, seq)
    assert rel_diff(got16, hidden) < 2e-3


@pytest.mark.parametrize("case", [c[0] for c in golden_cases(GOLDEN4)])
def test_forward_matches_hf_gemma4(case):
    """Gemma 4 (reference.rs:66-104 shapes): head_dim 512 global layers with
    partial RoPE, shared K/V, V norm, per-layer inputs and output scalars,
    against transformers' Gemma4TextModel in float64 (whose RMSNorm runs
    in float32, hence the looser bound)."""
    n, cfg, seed, lin, emb, request, hidden = next(c for c in golden_cases(GOLDEN4) if c[0] == case)
    ts = list(g.Weights.synth(cfg, seed, lin, emb).tensors())
    ids, pos, seq = flat_request(request)
    got = oracle.Model(cfg, ts).forward(ids, pos, seq)
    assert got.shape == hidden.shape
    assert rel_diff(got, hidden) < 3e-5, rel_diff(got, hidden)  # measured 5.7e-6 and 9.9e-6
    got16 = oracle.Model(cfg, ts, gpu_rounding=True).forward(ids, pos, seq)
    assert rel_diff(got16, hidden) < 2e-2


def test_gemma4_forward_mistakes_would_be_caught():
    """Planted mistakes in the Gemma 4 pieces miss the fixture by far more
    than the tolerance: no per-layer inputs (table zeroed), K/V not shared
    (the shared layers' own K/V: a config without sharing, the same weights
    where they exist), full RoPE on the global layers."""
    n, cfg, seed, lin, emb, request, hidden = next(golden_cases(GOLDEN4))
    ts = list(g.Weights.synth(cfg, seed, lin, emb).tensors())
    ids, pos, seq = flat_request(request)
    zeroed = [g.QTensor(t.name, t.dtype, t.shape, np.zeros_like(t.data), np.zeros_like(t.scales))
              if t.name == "per_layer_table" else t for t in ts]
    assert rel_diff(oracle.Model(cfg, zeroed).forward(ids, pos, seq), hidden) > 1e-2
    c = json.loads(cfg)
    c["rope_parameters"]["full_attention"]["partial_rotary_factor"] = 1.0
    assert rel_diff(oracle.Model(json.dumps(c), ts).forward(ids, pos, seq), hidden) > 1e-2
    c = json.loads(cfg)
    c["num_kv_shared_layers"], c["use_double_wide_mlp"], c["intermediate_size"] = 0, False, [96, 96, 192, 192]
    by_name = {t.name: t for t in ts}
    # The shared layers (2, 3) get their sources' (0, 1) K/V rows and k_norm.
    extra = [(l, by_name[f"blk.{l}.qkv"], by_name[f"blk.{l - 2}.qkv"]) for l in (2, 3)]
    rebuilt = []
    for t in ts:
        hit = next((e for e in extra if t.name == f"blk.{e[0]}.qkv"), None)
        if hit is None:
            rebuilt.append(t)
            continue
        l, q, src = hit
        rows_q = q.shape[0]
        per_row = q.data.size // rows_q
        kv_rows = src.shape[0] - rows_q
        data = np.concatenate([q.data.reshape(rows_q, per_row), src.data.reshape(src.shape[0], per_row)[rows_q:]])
        sp = q.scales.size // rows_q if q.scales.size else 0
        scales = (np.concatenate([q.scales.reshape(rows_q, sp), src.scales.reshape(src.shape[0], sp)[rows_q:]])
                  if sp else q.scales)
        rebuilt.append(g.QTensor(t.name, t.dtype, (rows_q + kv_rows, q.shape[1]), data.ravel(), scales.ravel()))
        rebuilt.append(g.QTensor(f"blk.{l}.k_norm", by_name[f"blk.{l - 2}.k_norm"].dtype,
                                 by_name[f"blk.{l - 2}.k_norm"].shape, by_name[f"blk.{l - 2}.k_norm"].data,
                                 by_name[f"blk.{l - 2}.k_norm"].scales))
    unshared = oracle.Model(json.dumps(c), rebuilt).forward(ids, pos, seq)
    # Same K/V projections and norms as the source layers, but each layer
    # projects its own input: the rows move well outside the bound.
    assert rel_diff(unshared, hidden) > 1e-2


def test_forward_mistakes_would_be_caught():
    """A forward that ignored the branch mask (every key visible) or the
    window would miss the fixture by far more than the tolerance above."""
    n, cfg, seed, lin, emb, request, hidden = next(golden_cases())
    w = g.Weights.synth(cfg, seed, lin, emb)
    m = oracle.Model(cfg, list(w.tensors()))
    ids, pos, seq = flat_request(request)
    one_seq = m.forward(ids, pos, np.zeros_like(seq))
    assert rel_diff(one_seq, hidden) > 1e-2
    cfg_nowin = json.loads(cfg)
    cfg_nowin["sliding_window"] = 4096
    m2 = oracle.Model(json.dumps(cfg_nowin), list(w.tensors()))
    assert rel_diff(m2.forward(ids, pos, seq), hidden) > 1e-2


def test_forward_order_independent():
    """Rows depend on (id, pos, seq) only, not on where a token sits."""
    n, cfg, seed, lin, emb, request, hidden = next(golden_cases())
    w = g.Weights.synth(cfg, seed, lin, emb)
    m = oracle.Model(cfg, list(w.tensors()))
    ids, pos, seq = flat_request(request)
    perm = np.random.default_rng(3).permutation(ids.size)
    a = m.forward(ids, pos, seq)
    b = m.forward(ids[perm], pos[perm], seq[perm])
    assert rel_diff(b, a[perm]) < 1e-6  # only the key summation order differs


def test_logits_are_hidden_times_embedding():
    # reference.rs:564-598: logits = hidden . embed^T (+ softcap when set)
    cfg = g.config_json(vocab=64, d=64, layers=1, heads=2, kv_heads=1, head_dim=256, ff=96, window=4,
                        sliding=[False], norm_offset=0.0)
    w = g.Weights.synth(cfg, 3, g.Q8, g.Q4)
    ts = list(w.tensors())
    emb = next(t for t in ts if t.name == "embed").to_f32().astype(np.float64)
    rows = np.random.default_rng(1).standard_normal((5, 64)).astype(np.float32)
    got = oracle.Model(cfg, ts).logits(rows)
    assert np.max(np.abs(got - rows.astype(np.float64) @ emb.T)) < 1e-4
    c = json.loads(cfg)
    c["final_logit_softcapping"] = 3.0
    got = oracle.Model(json.dumps(c), ts).logits(rows)
    assert np.max(np.abs(got - 3.0 * np.tanh(rows.astype(np.float64) @ emb.T / 3.0))) < 1e-5


# ----------------------------------------------------------------- pack

def pack_groups():
    B = g.BranchTokens
    return [g.Group([1, 2, 3], [B([4, 5], [1]), B([6], [0])]),
            g.Group([7, 8], [B([9, 10, 11], [2, 0])])]


def test_pack_known_layout():
    """engine.rs:1512-1571 worked by hand: group 1 first, then group 0;
    meta = (position, sequence id, first key row of the group, row + 1)."""
    ids, meta, wanted, decoded = oracle.pack(pack_groups(), first=1, resident=False)
    assert ids.tolist() == [7, 8, 9, 10, 11, 1, 2, 3, 4, 5, 6]
    assert meta.tolist() == [
        [0, 0, 0, 1], [1, 0, 0, 2], [2, 1, 0, 3], [3, 1, 0, 4], [4, 1, 0, 5],
        [0, 4096, 5, 6], [1, 4096, 5, 7], [2, 4096, 5, 8],
        [3, 4097, 5, 9], [4, 4097, 5, 10], [3, 4098, 5, 11]]
    assert wanted.tolist() == [[1, 0, 0, 4], [1, 0, 1, 2], [0, 0, 0, 9], [0, 1, 0, 10]]
    assert decoded.tolist() == [[1, 0], [0, 5]]


def test_pack_known_layout_resident():
    """The first group's prefix is resident (cache rows 0..2): its tokens are
    not packed and this pass's tokens take cache rows 2..; workspace rows
    (wanted) restart at 0."""
    ids, meta, wanted, decoded = oracle.pack(pack_groups(), first=1, resident=True)
    assert ids.tolist() == [9, 10, 11, 1, 2, 3, 4, 5, 6]
    assert meta.tolist() == [
        [2, 1, 0, 3], [3, 1, 0, 4], [4, 1, 0, 5],
        [0, 4096, 5, 6], [1, 4096, 5, 7], [2, 4096, 5, 8],
        [3, 4097, 5, 9], [4, 4097, 5, 10], [3, 4098, 5, 11]]
    assert wanted.tolist() == [[1, 0, 0, 2], [1, 0, 1, 0], [0, 0, 0, 7], [0, 1, 0, 8]]
    assert decoded.tolist() == [[0, 5]]


# ---------------------------------------------------------------- state

def fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) % (1 << 64)
    return h


def test_fnv1a_published_vectors():
    # FNV-1a 64-bit test vectors published with the algorithm (isthe.com/chongo/tech/comp/fnv)
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8


@pytest.mark.parametrize("model_id,prefix", [("", []), ("a", []), ("foobar", [1, 2, 0xFFFFFFFF]),
                                             ("gemma-3-270m-q4", list(range(300)))])
def test_state_key(model_id, prefix):
    # engine.rs:625-641: model id bytes, one zero byte, then each token's
    # four little-endian bytes, through FNV-1a.
    data = model_id.encode() + b"\0" + np.array(prefix, "<u4").tobytes()
    assert oracle.state_key(model_id, prefix) == fnv1a64(data)
    # one step past a published vector: FNV-1a("a") then the zero byte
    if model_id == "a":
        assert oracle.state_key("a", []) == (0xAF63DC4C8601EC8C * 0x100000001B3) % (1 << 64)


def test_state_rows():
    # engine.rs:1967-1974
    assert oracle.state_rows(True, 512, 2000) == (1488, 2000)
    assert oracle.state_rows(True, 512, 300) == (0, 300)
    assert oracle.state_rows(False, 512, 2000) == (0, 2000)
    assert oracle.state_rows(True, 0, 2000) == (0, 2000)


# -------------------------------------------------------------- readout

def test_softmax_reference_answers():
    # crates/omg-core/src/math.rs tests
    p = oracle.softmax([1.0, 2.0, 3.0])
    assert abs(p.sum() - 1.0) < 1e-12 and p[2] > p[1] > p[0]
    assert oracle.softmax([0.0, 4.0])[1] > oracle.softmax([0.0, 4.0], 4.0)[1]
    # closed form for two logits: p1 = 1 / (1 + e^-4)
    assert abs(oracle.softmax([0.0, 4.0])[1] - 1 / (1 + np.exp(-4.0))) < 1e-12
    z = np.array([1000.0, 999.0, -5.0], np.float32)
    assert abs(oracle.log_sum_exp(z) - (1000.0 + np.log1p(np.exp(-1.0) + np.exp(-1005.0)))) < 1e-9


def test_confidence_reference_answers():
    assert abs(oracle.confidence([0.5, 0.5])) < 1e-12
    assert abs(oracle.confidence([1.0, 0.0]) - 1.0) < 1e-12
    assert oracle.confidence([1.0]) == 1.0
    assert oracle.argmax([0.1, 0.7, 0.2]) == 1


def test_option_orders_reference_answers():
    assert oracle.option_orders(1, 4) == [[0]]
    assert oracle.option_orders(2, 4) == [[0, 1], [1, 0]]
    o = oracle.option_orders(3, 8)
    assert len(o) == 6 and len({tuple(x) for x in o}) == 6
    assert oracle.option_orders(5, 3) == [[0, 1, 2, 3, 4], [1, 2, 3, 4, 0], [2, 3, 4, 0, 1]]


def test_pointer_identity_is_scaled_dot():
    # readout.rs pointer_head_identity_projection_is_a_dot_product
    eye = np.eye(4, dtype=np.float32)
    z = oracle.pointer_logits(eye, np.zeros(4), eye, np.zeros(4), [1, 0, 0, 0], [[1, 0, 0, 0], [0, 1, 0, 0]])
    assert z[0] > z[1] and abs(z[0] - 0.5) < 1e-6


def test_pointer_closed_forms():
    """readout.rs:30-44 forms a plausible slip breaks: with a zero k map
    every option scores b_k . q / sqrt(dp) whatever its row; q is the decide
    row's map (not an option's); the scale is 1 / sqrt(dp), not 1 / dp."""
    rng = np.random.default_rng(3)
    d, dp = 12, 9
    w_q, w_k = rng.standard_normal((dp, d)), rng.standard_normal((dp, d))
    b_q, b_k = rng.standard_normal(dp), rng.standard_normal(dp)
    decide, opts = rng.standard_normal(d), rng.standard_normal((3, d))
    q = w_q.astype(np.float32) @ decide.astype(np.float32) + b_q.astype(np.float32)
    z0 = oracle.pointer_logits(w_q, b_q, np.zeros((dp, d)), b_k, decide, opts)
    assert np.allclose(z0, float(b_k.astype(np.float32) @ q) / 3.0, rtol=1e-5)
    # swapping the decide row for an option's changes every logit
    z = oracle.pointer_logits(w_q, b_q, w_k, b_k, decide, opts)
    zs = oracle.pointer_logits(w_q, b_q, w_k, b_k, opts[0], opts)
    assert np.all(np.abs(z - zs) > 1e-6)
    # doubling both maps' weights and biases quadruples the logits
    z2 = oracle.pointer_logits(2 * w_q, 2 * b_q, 2 * w_k, 2 * b_k, decide, opts)
    assert np.allclose(z2, 4 * z, rtol=1e-5)


def test_label_readout_picks_label_columns():
    row = np.arange(10, dtype=np.float32)
    logits, probs, mass = oracle.label_readout(row, [7, 2, 9])
    assert logits.tolist() == [7.0, 2.0, 9.0]
    e = np.exp(np.array([7.0, 2.0, 9.0]) - 9.0)
    assert np.allclose(probs, e / e.sum(), atol=1e-12)
    full = np.exp(row.astype(np.float64) - 9.0)
    assert abs(mass - e.sum() / full.sum()) < 1e-9


def test_fold_averages_orders():
    # crates/omg-core/src/engine.rs averaging_orders_cancels_the_letter_pull:
    # label A three logits ahead in both orders -> each option gets 1.5
    out = oracle.fold_mean([[0, 1], [1, 0]], [[3.0, 0.0], [3.0, 0.0]])
    assert out.tolist() == [1.5, 1.5]


# ------------------------------------------- kernel-rounding attention

def test_tiled_attention_is_the_softmax_up_to_f16_probabilities():
    """set_attention_tiles models the flash kernel's rounding: with every
    key in one chunk it differs from the f16-operand forward only by P's
    f16 rounding (relative 2^-11 per probability), on the transformers
    fixtures; with one-tile chunks (every tile a partial, merged by
    weight) it stays within the f16 rounding of the partials of that."""
    for n, cfg, seed, lin, emb, request, hidden in golden_cases():
        ts = list(g.Weights.synth(cfg, seed, lin, emb).tensors())
        ids, pos, seq = flat_request(request)
        f16 = oracle.Model(cfg, ts, gpu_rounding=True).forward(ids, pos, seq)
        whole = oracle.Model(cfg, ts, gpu_rounding=True).set_attention_tiles(32, 1000, 1000).forward(ids, pos, seq)
        split = oracle.Model(cfg, ts, gpu_rounding=True).set_attention_tiles(4, 1, 1).forward(ids, pos, seq)
        assert 0 < rel_diff(whole, f16) < 2e-3, (n, rel_diff(whole, f16))
        assert rel_diff(split, whole) < 2e-3, (n, rel_diff(split, whole))
        assert rel_diff(whole, hidden) < 4e-3


def test_tiled_attention_does_not_depend_on_an_aligned_cache_offset():
    """The property the engine's group alignment relies on: with the
    kernel's whole-power-of-two max, every probability and rescale differs
    by an exact power of two under another running max, so a group's rows
    are bit-equal whether it starts the cache or starts on a key tile after
    another group.  At an offset that is not a multiple of the key tile the
    group's keys share MFMA tiles differently: f32 summation order changes,
    and the f16 rounding of the attention output turns that into
    ~1e-4 changes (why the engine starts every group on a key tile)."""
    cfg = g.config_json(vocab=64, d=64, layers=3, heads=4, kv_heads=1, head_dim=256, ff=96, window=7,
                        sliding=[True, False, True], norm_offset=0.0)
    ts = list(g.Weights.synth(cfg, 5, g.Q4, g.Q8).tensors())
    rng = np.random.default_rng(2)
    prefix, toks = rng.integers(0, 64, 45).tolist(), rng.integers(0, 64, 13).tolist()
    m = oracle.Model(cfg, ts, gpu_rounding=True).set_attention_tiles(32, 1000, 1000)
    alone_ids = np.array(prefix + toks, np.uint32)
    alone_pos = np.arange(len(prefix) + len(toks), dtype=np.int32)
    alone_seq = np.array([0] * len(prefix) + [1] * len(toks), np.int32)
    alone = m.forward(alone_ids, alone_pos, alone_seq)

    def after(lead_len: int) -> np.ndarray:
        # the same group (group bits 1 << 12) after a lead_len-token group 0
        lead = rng.integers(0, 64, lead_len).tolist()
        ids = np.array(lead + prefix + toks, np.uint32)
        pos = np.array(list(range(lead_len)) + list(range(len(prefix) + len(toks))), np.int32)
        seq = np.array([0] * lead_len + [1 << 12] * len(prefix) + [(1 << 12) | 1] * len(toks), np.int32)
        return m.forward(ids, pos, seq)[lead_len:]

    assert np.array_equal(after(32), alone)
    assert np.array_equal(after(64), alone)
    d = rel_diff(after(19), alone)
    assert 0 < d < 5e-4, d
