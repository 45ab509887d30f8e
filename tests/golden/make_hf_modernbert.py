"""Writes tests/golden/hf_modernbert.npz: the encoder path's forward in
float64 by library routines, on the seeded weights of a tiny config, for
pinning the CPU oracle (oracle/laya.c).

  - the encoder: Hugging Face transformers' ModernBertModel (eager
    attention), built from a local config with the weights copied in
    (no download);
  - the decision-head layers: torch.nn.TransformerEncoderLayer (pre-norm,
    ReLU) with the q rows of in_proj (weight and bias) multiplied by
    sqrt(64), which cancels torch's 1/sqrt(head_dim): the reference runs
    these layers' attention unscaled (laya.rs:1346-1350 with
    shaders/attention_bi.wgsl);
  - the scorer: nn.Sequential(LayerNorm, Linear, GELU, Linear) at each
    marker row (laya.rs:1447-1457).

Run once in a container that has transformers:  python tests/golden/make_hf_modernbert.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import grande_amd as g  # noqa: E402
from grande_amd import laya as ly  # noqa: E402

SEED = 21
VARIANTS = {
    # encoder only: final norm output, no type embedding, no head layers
    "enc": dict(head_layers=0, type_emb=False),
    # encoder + type embedding + two decision-head layers + scorer
    "full": dict(head_layers=2, type_emb=True),
}
BASE = dict(vocab=200, d=128, layers=4, heads=2, ff=192, local_attention=8, global_every=3, cls=1, sep=2, mask=4,
            pad=0, act_costs=None)
SEQS = [(23, [3, 11], 0), (40, [5], 1), (9, [2, 6, 7], 2)]


def sequences():
    rng = np.random.default_rng(5)
    out = []
    for n, markers, qtype in SEQS:
        ids = rng.integers(5, BASE["vocab"], n).tolist()
        ids[0], ids[-1] = BASE["cls"], BASE["sep"]
        for m in markers:
            ids[m] = BASE["mask"]
        out.append((ids, markers, qtype))
    return out


def run(variant: str):
    from transformers import ModernBertConfig, ModernBertModel

    kw = dict(BASE, **VARIANTS[variant])
    cfg_text = ly.laya_config_json(**kw)
    w = {t.name: t for t in ly.synth_weights(cfg_text, SEED, g.Q8, g.Q8).tensors()}
    f = {k: torch.from_numpy(t.to_f32().astype(np.float64)) for k, t in w.items()}
    d, L, H = kw["d"], kw["layers"], kw["heads"]
    hc = ModernBertConfig(vocab_size=kw["vocab"], hidden_size=d, intermediate_size=kw["ff"], num_hidden_layers=L,
                          num_attention_heads=H, local_attention=kw["local_attention"],
                          layer_types=["full_attention" if i % kw["global_every"] == 0 else "sliding_attention"
                                       for i in range(L)],
                          rope_parameters={"full_attention": {"rope_type": "default", "rope_theta": 160000.0},
                                           "sliding_attention": {"rope_type": "default", "rope_theta": 10000.0}},
                          norm_eps=1e-5, norm_bias=False, attention_bias=False, mlp_bias=False,
                          hidden_activation="gelu", pad_token_id=0, bos_token_id=1, eos_token_id=2, cls_token_id=1,
                          sep_token_id=2, max_position_embeddings=512)
    hc._attn_implementation = "eager"
    model = ModernBertModel(hc).double().eval()
    sd = {"embeddings.tok_embeddings.weight": f["embed"], "embeddings.norm.weight": f["embed_norm"],
          "final_norm.weight": f["final_norm"]}
    for l in range(L):
        p = f"layers.{l}."
        if l > 0:
            sd[p + "attn_norm.weight"] = f[f"enc.{l}.attn_norm"]
        sd[p + "attn.Wqkv.weight"] = f[f"enc.{l}.qkv"]
        sd[p + "attn.Wo.weight"] = f[f"enc.{l}.o"]
        sd[p + "mlp_norm.weight"] = f[f"enc.{l}.mlp_norm"]
        sd[p + "mlp.Wi.weight"] = torch.cat([f[f"enc.{l}.wi_val"], f[f"enc.{l}.wi_gate"]], 0)
        sd[p + "mlp.Wo.weight"] = f[f"enc.{l}.wo"]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("inv_freq" in m for m in missing), missing

    heads = []
    for h in range(kw["head_layers"]):
        layer = torch.nn.TransformerEncoderLayer(d, H, 4 * d, dropout=0.0, activation="relu", batch_first=True,
                                                 norm_first=True, layer_norm_eps=1e-5).double().eval()
        n = lambda s: f[f"head.{h}.{s}"]  # noqa: E731
        win, bin_ = n("in_proj").clone(), n("in_proj_b").clone()
        win[:d] *= 8.0
        bin_[:d] *= 8.0
        with torch.no_grad():
            layer.self_attn.in_proj_weight.copy_(win)
            layer.self_attn.in_proj_bias.copy_(bin_)
            layer.self_attn.out_proj.weight.copy_(n("out_proj"))
            layer.self_attn.out_proj.bias.copy_(n("out_proj_b"))
            layer.norm1.weight.copy_(n("norm1_w"))
            layer.norm1.bias.copy_(n("norm1_b"))
            layer.norm2.weight.copy_(n("norm2_w"))
            layer.norm2.bias.copy_(n("norm2_b"))
            layer.linear1.weight.copy_(n("l1"))
            layer.linear1.bias.copy_(n("l1_b"))
            layer.linear2.weight.copy_(n("l2"))
            layer.linear2.bias.copy_(n("l2_b"))
        heads.append(layer)
    scorer = torch.nn.Sequential(torch.nn.LayerNorm(d, eps=1e-5), torch.nn.Linear(d, d), torch.nn.GELU(),
                                 torch.nn.Linear(d, 1)).double().eval()
    with torch.no_grad():
        scorer[0].weight.copy_(f["scorer.norm_w"])
        scorer[0].bias.copy_(f["scorer.norm_b"])
        scorer[1].weight.copy_(f["scorer.l1"])
        scorer[1].bias.copy_(f["scorer.l1_b"])
        scorer[3].weight.copy_(f["scorer.l2"])
        scorer[3].bias.copy_(f["scorer.l2_b"])

    rows, logits = [], []
    with torch.no_grad():
        for ids, markers, qtype in sequences():
            x = model(input_ids=torch.tensor([ids])).last_hidden_state
            if kw["type_emb"]:
                x = x + f["type_emb"][qtype]
            for layer in heads:
                x = layer(x)
            r = x[0, [0] + markers]
            rows.append(r.numpy())
            logits.append(scorer(r[1:])[:, 0].numpy())
    return cfg_text, rows, logits


def main() -> None:
    out = {}
    for v in VARIANTS:
        cfg_text, rows, logits = run(v)
        out[f"{v}_config"] = np.frombuffer(cfg_text.encode(), np.uint8)
        out[f"{v}_rows"] = np.concatenate(rows).astype(np.float64)
        out[f"{v}_logits"] = np.concatenate(logits).astype(np.float64)
    out["seed"] = np.array([SEED])
    out["seqs"] = np.frombuffer(json.dumps(sequences()).encode(), np.uint8)
    path = Path(__file__).resolve().parent / "hf_modernbert.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
