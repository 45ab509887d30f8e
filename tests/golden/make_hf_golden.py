"""Writes tests/golden/hf_gemma3.npz: golden hidden rows of the decision-path
forward from an implementation independent of both the reference and the
oracle — Hugging Face transformers' Gemma3TextModel (5.x), run in float64
on CPU in THIS container (never on the GPU box), with:

  * the identical seeded weights (grande_amd.Weights.synth, the generator of
    crates/omg-wgpu/tests/reference.rs:106-139), dequantized exactly;
  * a block-causal mask built from the request structure (a token sees the
    same request's prefix and its own branch, causally, and within the
    window on sliding layers), not from sequence ids;
  * positions prefix_len + j for branch tokens (omg-core backend.rs:22-30).

The fixture stores the inputs (config, seed, dtypes, the request) and the
expected final-norm hidden state of every token.  tests/test_oracle.py
checks the oracle against it.

    python tests/golden/make_hf_golden.py
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

OUT = Path(__file__).resolve().parent / "hf_gemma3.npz"

# Cases: (name, config kwargs, seed, linear dtype, embed dtype, request).
# Requests are lists of groups: (prefix, [branch tokens...]).
CASES = [
    ("gemma3_f16", dict(vocab=40, d=64, layers=3, heads=2, kv_heads=1, head_dim=256, ff=96, window=6,
                        sliding=[True, False, True], norm_offset=None),
     7, g.F16, g.F16,
     [([2, 5, 9, 14, 20, 31, 7, 8, 3, 22], [[11, 12, 13, 14, 15], [30, 31, 32, 33, 34, 35, 36, 37]])]),
    ("gguf_q4_gqa", dict(vocab=64, d=64, layers=4, heads=4, kv_heads=2, head_dim=256, ff=96, window=5,
                         sliding=[True, False, True, False], norm_offset=0.0),
     9, g.Q4, g.Q8,
     [([2, 5, 9, 14, 20, 31, 7, 8, 3, 22, 4, 6], [[11, 12, 13], [30, 31, 32, 33, 34, 35, 36]])]),
    ("gguf_q8_groups", dict(vocab=64, d=96, layers=2, heads=4, kv_heads=1, head_dim=256, ff=128, window=4,
                            sliding=[True, False], norm_offset=0.0),
     19, g.Q8, g.Q8,
     [([2, 5, 9, 14, 20], [[11, 12], [30, 31, 32]]), ([2, 3, 4], [[33, 34, 35, 36]])]),
]


def hf_model(cfg: dict, tensors: dict):
    from transformers import Gemma3TextConfig, Gemma3TextModel

    hc = Gemma3TextConfig(
        vocab_size=cfg["vocab"], hidden_size=cfg["d"], intermediate_size=cfg["ff"],
        num_hidden_layers=cfg["layers"], num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv_heads"],
        head_dim=cfg["head_dim"], rms_norm_eps=1e-6, query_pre_attn_scalar=cfg["head_dim"],
        sliding_window=cfg["window"], max_position_embeddings=4096,
        layer_types=["sliding_attention" if s else "full_attention" for s in cfg["sliding"]],
        rope_parameters={"full_attention": {"rope_type": "default", "rope_theta": 1e6},
                         "sliding_attention": {"rope_type": "default", "rope_theta": 1e4}},
        hidden_activation="gelu_pytorch_tanh", attention_bias=False, attention_dropout=0.0,
    )
    hc._attn_implementation = "eager"
    model = Gemma3TextModel(hc).to(torch.float64).eval()
    # HF Gemma 3 norms apply (1 + w); the checkpoint applies (offset + w).
    offset = 1.0 if cfg.get("norm_offset") is None else cfg["norm_offset"]
    H, KV, hd = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]

    def t(name):
        return torch.from_numpy(tensors[name].astype(np.float64))

    def norm(name):
        return t(name) + (offset - 1.0)

    sd = {"embed_tokens.weight": t("embed"), "norm.weight": norm("final_norm")}
    for l in range(cfg["layers"]):
        p, b = f"layers.{l}.", f"blk.{l}."
        qkv = t(b + "qkv")
        sd[p + "self_attn.q_proj.weight"] = qkv[:H * hd]
        sd[p + "self_attn.k_proj.weight"] = qkv[H * hd:(H + KV) * hd]
        sd[p + "self_attn.v_proj.weight"] = qkv[(H + KV) * hd:]
        sd[p + "self_attn.o_proj.weight"] = t(b + "o")
        sd[p + "self_attn.q_norm.weight"] = norm(b + "q_norm")
        sd[p + "self_attn.k_norm.weight"] = norm(b + "k_norm")
        sd[p + "mlp.gate_proj.weight"] = t(b + "gate")
        sd[p + "mlp.up_proj.weight"] = t(b + "up")
        sd[p + "mlp.down_proj.weight"] = t(b + "down")
        sd[p + "input_layernorm.weight"] = norm(b + "attn_norm")
        sd[p + "post_attention_layernorm.weight"] = norm(b + "post_attn_norm")
        sd[p + "pre_feedforward_layernorm.weight"] = norm(b + "ffn_norm")
        sd[p + "post_feedforward_layernorm.weight"] = norm(b + "post_ffn_norm")
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if "rotary" not in m]
    assert not missing and not unexpected, (missing, unexpected)
    return model


def layout(request):
    """Flatten the request: token ids, positions, and for each token its
    (group, branch) with branch -1 for prefix tokens."""
    ids, pos, who = [], [], []
    for gi, (prefix, branches) in enumerate(request):
        for i, tok in enumerate(prefix):
            ids.append(tok), pos.append(i), who.append((gi, -1))
        for bi, toks in enumerate(branches):
            for j, tok in enumerate(toks):
                ids.append(tok), pos.append(len(prefix) + j), who.append((gi, bi))
    return np.array(ids, np.int64), np.array(pos, np.int64), who


def mask(pos, who, window):
    """Additive [T, T] mask: query i may use key j iff same group, j is in the
    group's prefix or in i's own branch, j is not after i, and (window > 0)
    i and j are less than `window` positions apart."""
    T = len(pos)
    m = np.full((T, T), -np.inf)
    for i in range(T):
        for j in range(T):
            same = who[i][0] == who[j][0] and (who[j][1] == -1 or who[j][1] == who[i][1])
            if same and pos[j] <= pos[i] and (window == 0 or pos[i] - pos[j] < window):
                m[i, j] = 0.0
    return torch.from_numpy(m)[None, None]


def main() -> None:
    out = {}
    for name, kw, seed, lin, emb, request in CASES:
        cfg_json = g.config_json(**kw)
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
