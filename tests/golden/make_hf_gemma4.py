"""Writes tests/golden/hf_gemma4.npz: golden hidden rows of the Gemma 4
decision-path forward from Hugging Face transformers' Gemma4TextModel (5.x),
run in float64 on CPU in THIS container (never on the GPU box), on the
seeded weights of crates/omg-wgpu/tests/reference.rs:66-104's Gemma 4
configs (grande_amd.Weights.synth, dequantized exactly), with the
block-causal request mask of make_hf_golden.py.

What it pins in the oracle (oracle/oracle.c): head_dim 512 global layers,
proportional RoPE on a quarter of their dims, the last two layers reading
the K/V of the last earlier layer of their type, unscaled (scale 1) query
products, V RMS-norm without weight, per-layer inputs (table * sqrt(P) plus
the normed projection, over sqrt(2)), the gated per-layer block and the
per-layer output scalar, Gemma 4's (w, not 1 + w) norms.

Gemma4RMSNorm normalises in float32 whatever the model dtype, so the
fixture carries float32-level rounding (rel ~1e-7).

    python tests/golden/make_hf_gemma4.py
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
from tests.golden.make_hf_golden import layout, mask  # noqa: E402

OUT = Path(__file__).resolve().parent / "hf_gemma4.npz"

BASE = dict(vocab=64, d=64, layers=4, head_dim=256, global_head_dim=512, ff=96, double_wide_mlp=True,
            shared_kv_layers=2, window=5, sliding=[True, False, True, False], partial_rotary_global=0.25,
            per_layer_dim=32, softcap=30.0)
CASES = [
    ("gemma4_q8", dict(BASE, heads=4, kv_heads=1), 7, g.Q8, g.Q8,
     [([2, 5, 9, 14, 20, 31, 7, 8, 3, 22], [[11, 12, 13, 14, 15], [30, 31, 32, 33, 34, 35, 36, 37]])]),
    ("gemma4_gqa_q4", dict(BASE, heads=8, kv_heads=2), 11, g.Q4, g.Q8,
     [([2, 5, 9, 14, 20, 31, 7, 8, 3, 22, 4, 6], [[11, 12, 13], [30, 31, 32, 33, 34, 35, 36]]),
      ([2, 3, 4], [[33, 34, 35, 36]])]),
]


def hf_model(cfg: dict, tensors: dict):
    from transformers.models.gemma4 import Gemma4TextConfig, Gemma4TextModel

    L, P = cfg["layers"], cfg["per_layer_dim"]
    hc = Gemma4TextConfig(
        vocab_size=cfg["vocab"], hidden_size=cfg["d"], intermediate_size=cfg["ff"], num_hidden_layers=L,
        num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv_heads"], head_dim=cfg["head_dim"],
        global_head_dim=cfg["global_head_dim"], rms_norm_eps=1e-6, sliding_window=cfg["window"],
        layer_types=["sliding_attention" if s else "full_attention" for s in cfg["sliding"]],
        rope_parameters={"sliding_attention": {"rope_type": "default", "rope_theta": 1e4},
                         "full_attention": {"rope_type": "proportional", "rope_theta": 1e6,
                                            "partial_rotary_factor": cfg["partial_rotary_global"]}},
        hidden_size_per_layer_input=P, vocab_size_per_layer_input=cfg["vocab"],
        num_kv_shared_layers=cfg["shared_kv_layers"], use_double_wide_mlp=cfg["double_wide_mlp"],
        final_logit_softcapping=cfg["softcap"], attention_k_eq_v=False, enable_moe_block=False,
        hidden_activation="gelu_pytorch_tanh", max_position_embeddings=4096,
    )
    hc._attn_implementation = "eager"
    model = Gemma4TextModel(hc).to(torch.float64).eval()
    H, KV = cfg["heads"], cfg["kv_heads"]
    shared0 = L - cfg["shared_kv_layers"]

    def t(name):
        return torch.from_numpy(tensors[name].astype(np.float64))

    sd = {"embed_tokens.weight": t("embed"), "norm.weight": t("final_norm"),
          "embed_tokens_per_layer.weight": t("per_layer_table"),
          "per_layer_model_projection.weight": t("pl_model_proj"),
          "per_layer_projection_norm.weight": t("pl_proj_norm")}
    for l in range(L):
        p, b = f"layers.{l}.", f"blk.{l}."
        hd = cfg["head_dim"] if cfg["sliding"][l] else cfg["global_head_dim"]
        qkv = t(b + "qkv")
        sd[p + "self_attn.q_proj.weight"] = qkv[:H * hd]
        if l < shared0:
            sd[p + "self_attn.k_proj.weight"] = qkv[H * hd:(H + KV) * hd]
            sd[p + "self_attn.v_proj.weight"] = qkv[(H + KV) * hd:]
            sd[p + "self_attn.k_norm.weight"] = t(b + "k_norm")
        sd[p + "self_attn.o_proj.weight"] = t(b + "o")
        sd[p + "self_attn.q_norm.weight"] = t(b + "q_norm")
        sd[p + "mlp.gate_proj.weight"] = t(b + "gate")
        sd[p + "mlp.up_proj.weight"] = t(b + "up")
        sd[p + "mlp.down_proj.weight"] = t(b + "down")
        sd[p + "input_layernorm.weight"] = t(b + "attn_norm")
        sd[p + "post_attention_layernorm.weight"] = t(b + "post_attn_norm")
        sd[p + "pre_feedforward_layernorm.weight"] = t(b + "ffn_norm")
        sd[p + "post_feedforward_layernorm.weight"] = t(b + "post_ffn_norm")
        sd[p + "per_layer_input_gate.weight"] = t(b + "pl_gate")
        sd[p + "per_layer_projection.weight"] = t(b + "pl_proj")
        sd[p + "post_per_layer_input_norm.weight"] = t(b + "pl_norm")
        sd[p + "layer_scalar"] = t(b + "out_scale")
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if "rotary" not in m]
    assert not missing and not unexpected, (missing, unexpected)
    return model


def main() -> None:
    out = {}
    for name, kw, seed, lin, emb, request in CASES:
        cfg_json = g.gemma4_config_json(**kw)
        w = g.Weights.synth(cfg_json, seed, lin, emb)
        tensors = {t.name: t.to_f32() for t in w.tensors()}
        model = hf_model(kw, tensors)
        ids, pos, who = layout(request)
        masks = {"full_attention": mask(pos, who, 0), "sliding_attention": mask(pos, who, kw["window"])}
        with torch.no_grad():
            h = model(input_ids=torch.from_numpy(ids)[None], position_ids=torch.from_numpy(pos)[None],
                      attention_mask=masks).last_hidden_state[0].numpy()
        out[name + "/config"] = np.frombuffer(cfg_json.encode(), np.uint8)
        out[name + "/meta"] = np.array([seed, lin, emb], np.int64)
        out[name + "/request"] = np.frombuffer(json.dumps(request).encode(), np.uint8)
        out[name + "/hidden"] = h.astype(np.float64)
        print(f"{name}: {len(ids)} tokens, |h| max {np.abs(h).max():.3f}")
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
