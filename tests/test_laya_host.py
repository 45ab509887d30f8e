"""The encoder path on the CPU: the oracle's pieces pinned against closed
forms and library routines, its whole pass by the invariants the reference
pass has (sequence isolation, order independence, the local window's exact
reach), and the library's host-side parts (config validation, the tensor
catalogue of laya.rs:252-305, seeded weights) — no GPU calls."""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

import grande_amd as g
import oracle
from grande_amd import laya as ly


def test_erf_within_abramowitz_stegun_bound():
    """laya.rs:1529-1546 / matmul_gated.wgsl:117-124: A&S 7.1.26, |error|
    < 1.5e-7 (plus f32 rounding)."""
    for x in np.linspace(-6, 6, 2001):
        assert abs(oracle.erf(float(x)) - math.erf(float(x))) < 4e-7, x
    assert oracle.erf(0.0) == 0.0


def test_gelu_erf_is_exact_gelu():
    for x in np.linspace(-8, 8, 801):
        exp = 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))
        assert abs(oracle.gelu_erf(float(x)) - exp) < 1e-6 * max(1.0, abs(x)), x


def test_layer_norm_closed_form():
    """layernorm.wgsl: (x - mean) / sqrt(var + eps) * w + b, variance
    around the mean; a dropped bias or an E[x^2] variance fails this."""
    rng = np.random.default_rng(0)
    x = (rng.normal(3.0, 2.0, 768)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 768).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, 768).astype(np.float32)
    xd = x.astype(np.float64)
    exp = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * w + b
    assert np.max(np.abs(oracle.layer_norm(x, w, b, 1e-5) - exp)) < 2e-5
    exp0 = (xd - xd.mean()) / np.sqrt(xd.var() + 1e-5) * w
    assert np.max(np.abs(oracle.layer_norm(x, w, None, 1e-5) - exp0)) < 2e-5


def test_rope_bi_is_a_complex_rotation():
    """rope_bi.wgsl: pairs (d, d + 32) rotate by pos * theta^(-2d/64),
    (a + ib)(cos + i sin); q is scaled after the rotation."""
    rng = np.random.default_rng(1)
    v = rng.normal(0, 1, 64).astype(np.float32)
    for pos, theta in ((0, 1e4), (1, 1e4), (37, 1e4), (255, 160000.0)):
        got = oracle.rope_bi(v, pos, theta, 0.125)
        ang = pos * np.power(float(theta), -np.arange(0, 64, 2) / 64.0)
        z = (v[:32].astype(np.float64) + 1j * v[32:]) * np.exp(1j * ang) * 0.125
        exp = np.concatenate([z.real, z.imag])
        assert np.max(np.abs(got - exp)) < 1e-4 * max(1, pos / 16), (pos, theta)


def tiny(**over) -> str:
    kw = dict(vocab=200, d=64, layers=2, heads=1, ff=96, local_attention=8, head_layers=1, act_costs={"a": 1.0},
              cls=1, sep=2, mask=4, pad=0)
    kw.update(over)
    return ly.laya_config_json(**kw)


def oracle_for(cfg, seed=3, dtype=g.Q8):
    return oracle.Laya(cfg, list(ly.synth_weights(cfg, seed, dtype, dtype).tensors()))


def test_oracle_sequences_are_isolated_and_order_free():
    orc = oracle_for(tiny())
    rng = np.random.default_rng(2)
    seqs = [(rng.integers(5, 200, n).tolist(), [1, n - 2], int(q)) for n, q in ((9, 0), (30, 1), (17, 2))]
    together = orc.hidden(seqs)
    for i, s in enumerate(seqs):
        assert np.array_equal(orc.hidden([s])[0], together[i])
    for a, b in zip(orc.hidden(seqs[::-1]), together[::-1]):
        assert np.array_equal(a, b)


def test_oracle_local_window_reach_is_inclusive():
    """One local layer, no head layers: the [CLS] row (row 0) sees rows
    0..window (|i - j| <= window, attention_bi.wgsl), nothing beyond."""
    cfg = tiny(layers=1, sliding=[True], head_layers=0, type_emb=False, act_costs=None, local_attention=8)
    orc = oracle_for(cfg)
    w = 4
    base = list(range(10, 30))
    ref = orc.hidden([(base, [], 0)])[0][0]
    far = list(base)
    far[w + 1] = 150
    assert np.array_equal(orc.hidden([(far, [], 0)])[0][0], ref)
    near = list(base)
    near[w] = 150
    assert not np.array_equal(orc.hidden([(near, [], 0)])[0][0], ref)
    glob = oracle_for(tiny(layers=1, sliding=[False], head_layers=0, type_emb=False, act_costs=None))
    assert not np.array_equal(glob.hidden([(far, [], 0)])[0][0], glob.hidden([(base, [], 0)])[0][0])


def test_oracle_type_embedding_and_scorer_shapes():
    orc = oracle_for(tiny())
    s = (list(range(5, 25)), [3, 7, 11], 0)
    rows0 = orc.hidden([s])[0]
    rows1 = orc.hidden([(s[0], s[1], 1)])[0]
    assert rows0.shape == (4, 64) and not np.array_equal(rows0, rows1)
    logits, act = orc.score(rows0)
    assert logits.shape == (3,) and np.isfinite(logits).all() and 0.0 < act < 1.0


def test_catalogue_and_seeded_weights():
    cfg = tiny(layers=3, head_layers=2, act_costs={"a": 1.0, "b": 2.0})
    w = ly.synth_weights(cfg, 7, g.Q8, g.Q4)
    ts = {t.name: t for t in w.tensors()}
    # laya.rs:252-305: layer 0 has no attention norm; 3 act outputs (2 costs + 1)
    assert "enc.0.attn_norm" not in ts and "enc.1.attn_norm" in ts
    assert ts["embed"].dtype == g.Q4 and ts["enc.2.wo"].dtype == g.Q8 and ts["enc.2.wo"].shape == (64, 96)
    assert ts["head.1.l1"].shape == (256, 64) and ts["head.1.in_proj_b"].shape == (192,)
    assert ts["act.l1"].shape == (256, 68) and ts["act.l2"].shape == (3, 256)
    assert ts["scorer.l1"].dtype == g.F16 and ts["type_emb"].dtype == g.F16 and ts["enc.0.mlp_norm"].dtype == g.F16
    norm = ts["enc.1.mlp_norm"].to_f32()
    assert np.all(np.abs(norm - 1.0) <= 0.5) and np.all(np.abs(ts["head.0.l2_b"].to_f32()) <= 0.02)
    again = {t.name: t for t in ly.synth_weights(cfg, 7, g.Q8, g.Q4).tensors()}
    assert all(np.array_equal(ts[k].data, again[k].data) for k in ts)
    b = ly.LayaBuilder(cfg)
    assert sorted(b.missing()) == sorted(ts)


@pytest.mark.parametrize("over,msg", [(dict(d=96, heads=2), "head_dim"), (dict(d=2560, heads=40), "2048"),
                                      (dict(head_max_len=600), "head_max_len"), (dict(ff=100), "multiples of 32")])
def test_config_rejections(over, msg):
    with pytest.raises(g.OmgError, match=msg):
        ly.LayaBuilder(tiny(**over))


def test_config_model_type_and_token_ids():
    v = json.loads(tiny())
    v["model_type"] = "bert"
    with pytest.raises(g.OmgError, match="modernbert"):
        ly.LayaBuilder(json.dumps(v))
    v = json.loads(tiny())
    del v["laya_tokens"]["mask_token"]
    with pytest.raises(g.OmgError, match="mask_token"):
        ly.LayaBuilder(json.dumps(v))


def test_exported_directory_round_trip(tmp_path):
    """tools/export_laya.py's layout (config.json with laya_agent,
    manifest.json, *.bin) read back bit-exactly; special ids given by the
    caller replace laya_tokens (the reference resolves them with its
    tokenizer)."""
    cfg = tiny(layers=2, head_layers=1)
    w = ly.synth_weights(cfg, 13, g.Q8, g.Q4)
    g.export_dir(w, tmp_path)
    back = {t.name: t for t in ly.load_dir(tmp_path).tensors()}
    for t in w.tensors():
        b = back[t.name]
        assert (b.dtype, b.shape) == (t.dtype, t.shape)
        assert np.array_equal(b.data, t.data) and np.array_equal(b.scales, t.scales)
    v = json.loads(cfg)
    v["laya_tokens"] = {"cls_token": "[CLS]", "sep_token": "[SEP]", "mask_token": "[MASK]", "pad_token": "[PAD]"}
    (tmp_path / "config.json").write_text(json.dumps(v))
    with pytest.raises(g.OmgError, match="cls_token"):
        ly.load_dir(tmp_path)
    assert len(ly.load_dir(tmp_path, special=(1, 2, 4, 0))) == len(back)


def test_oracle_matches_transformers_modernbert():
    """tests/golden/hf_modernbert.npz (make_hf_modernbert.py): transformers'
    ModernBertModel, torch's TransformerEncoderLayer with the reference's
    unscaled head attention, and the scorer as nn.Sequential, all in
    float64 on the same seeded weights.  The oracle carries the GPU path's
    f16 rounding points, hence 2e-3.  A planted mistake (window 5 instead
    of 4 on the local layers) misses by far more."""
    from pathlib import Path
    z = np.load(Path(__file__).resolve().parent / "golden" / "hf_modernbert.npz")
    seqs = [tuple(s) for s in json.loads(bytes(z["seqs"]).decode())]
    for v in ("enc", "full"):
        cfg = bytes(z[f"{v}_config"]).decode()
        ts = list(ly.synth_weights(cfg, int(z["seed"][0]), g.Q8, g.Q8).tensors())
        orc = oracle.Laya(cfg, ts)
        rows = orc.hidden(seqs)
        exp = z[f"{v}_rows"]
        got = np.concatenate(rows)
        assert np.abs(got - exp).max() / np.abs(exp).max() < 2e-3, v
        logits = np.concatenate([orc.score(r)[0] for r in rows])
        assert np.abs(logits - z[f"{v}_logits"]).max() < 2e-3, v
        wrong = json.loads(cfg)
        wrong["local_attention"] = 10
        bad = np.concatenate(oracle.Laya(json.dumps(wrong), ts).hidden(seqs))
        assert np.abs(bad - exp).max() / np.abs(exp).max() > 1e-2, v
