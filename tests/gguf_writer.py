"""A GGUF v3 writer for the tests: a Gemma 3 or Gemma 4 checkpoint in
llama.cpp's tensor names and metadata keys (the ones
tools/export_wgpu_gguf.py reads),
written from a host checkpoint of this library (q / k / v split back out of
the fused qkv tensor, Q8_0 / Q4_0 codes and scales interleaved into GGUF
blocks).  There is no gguf package in the image; the format is GGUF v3 as
llama.cpp documents it (header, key/value pairs, tensor infos, 32-byte
aligned data)."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

import grande_amd as g

U32, I32, F32, BOOL, STR, ARR = 4, 5, 6, 7, 8, 9
GG_F32, GG_F16, GG_Q4_0, GG_Q8_0, GG_BF16 = 0, 1, 2, 8, 30


def _s(b: bytearray, text: str) -> None:
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def _kv(b: bytearray, key: str, vtype: int, value) -> None:
    _s(b, key)
    b += struct.pack("<I", vtype)
    if vtype == U32:
        b += struct.pack("<I", value)
    elif vtype == F32:
        b += struct.pack("<f", value)
    elif vtype == STR:
        _s(b, value)
    elif vtype == ARR:
        etype, items = value
        b += struct.pack("<IQ", etype, len(items))
        for it in items:
            if etype == BOOL:
                b += struct.pack("<B", int(it))
            elif etype == STR:
                _s(b, it)
            elif etype == I32:
                b += struct.pack("<i", it)
    else:
        raise ValueError(vtype)


def _blocks(t: g.QTensor, rows=None) -> tuple[int, bytes]:
    """GGUF payload of a QTensor (optionally a row range)."""
    cols = t.shape[-1]
    r0, r1 = rows if rows else (0, t.shape[0] if len(t.shape) == 2 else 1)
    if t.dtype == g.F16:
        v = t.data.view(np.float16).reshape(-1, cols)[r0:r1]
        return GG_F16, v.tobytes()
    per = 32 if t.dtype == g.Q8 else 16
    codes = t.data.reshape(-1, cols // 32, per)[r0:r1]
    scales = t.scales.reshape(-1, cols // 32, 2)[r0:r1]
    return (GG_Q8_0 if t.dtype == g.Q8 else GG_Q4_0), np.concatenate([scales, codes], axis=2).tobytes()


def write_gemma3(path: str | Path, config_text: str, weights: g.Weights, f32_norms: bool = True,
                 bf16: tuple[str, ...] = ()) -> None:
    """`config_text` is the checkpoint's config.json (norm offset 0, as a
    GGUF stores Gemma 3 norms); 1-D tensors are written as f32 (or bf16 for
    the llama.cpp names in `bf16`)."""
    cfg = json.loads(config_text)
    g4 = cfg.get("model_type") == "gemma4_text"
    arch = "gemma4" if g4 else "gemma3"
    ts = {t.name: t for t in weights.tensors()}
    L, d, H, KV = cfg["num_hidden_layers"], cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    types = cfg.get("layer_types")
    swa = [t == "sliding_attention" for t in types] if types else \
        [(i + 1) % cfg.get("_sliding_window_pattern", 6) != 0 for i in range(L)]
    hd_swa = cfg["head_dim"]
    hd_full = cfg.get("global_head_dim", hd_swa)
    shared = cfg.get("num_kv_shared_layers", 0)
    pl = cfg.get("hidden_size_per_layer_input", 0)
    ffs = [ts[f"blk.{l}.gate"].shape[0] for l in range(L)]
    tensors: list[tuple[str, list[int], int, bytes]] = []

    def add(name, t: g.QTensor, shape, rows=None):
        if len(t.shape) == 1:
            v = t.data.view(np.float16).astype(np.float32)
            if name in bf16:
                u = v.view(np.uint32)
                tensors.append((name, shape, GG_BF16, (u >> 16).astype(np.uint16).tobytes()))
            elif f32_norms:
                tensors.append((name, shape, GG_F32, v.tobytes()))
            else:
                tensors.append((name, shape, GG_F16, t.data.tobytes()))
            return
        kind, payload = _blocks(t, rows)
        tensors.append((name, shape, kind, payload))

    add("token_embd.weight", ts["embed"], ts["embed"].shape)
    add("output_norm.weight", ts["final_norm"], [d])
    if pl:
        add("per_layer_model_proj.weight", ts["pl_model_proj"], [pl * L, d])
        add("per_layer_proj_norm.weight", ts["pl_proj_norm"], [pl])
        add("per_layer_token_embd.weight", ts["per_layer_table"], list(ts["per_layer_table"].shape))
    if g4:
        # partial RoPE of the global layers: 1.0 for rotated pairs, 1e30 for the rest
        rot = cfg["rope_parameters"]["full_attention"].get("partial_rotary_factor", 1.0)
        f = np.full(hd_full // 2, 1e30, np.float32)
        f[: int(rot * hd_full) // 2] = 1.0
        tensors.append(("rope_freqs.weight", [hd_full // 2], GG_F32, f.tobytes()))
    for l in range(L):
        b = f"blk.{l}."
        hd = hd_swa if swa[l] else hd_full
        own = l < L - shared
        add(b + "attn_norm.weight", ts[b + "attn_norm"], [d])
        qkv = ts[b + "qkv"]
        add(b + "attn_q.weight", qkv, [H * hd, d], (0, H * hd))
        if own:
            add(b + "attn_k.weight", qkv, [KV * hd, d], (H * hd, (H + KV) * hd))
            add(b + "attn_v.weight", qkv, [KV * hd, d], ((H + KV) * hd, (H + 2 * KV) * hd))
        add(b + "attn_q_norm.weight", ts[b + "q_norm"], [hd])
        if own:
            add(b + "attn_k_norm.weight", ts[b + "k_norm"], [hd])
        add(b + "attn_output.weight", ts[b + "o"], [d, H * hd])
        add(b + "post_attention_norm.weight", ts[b + "post_attn_norm"], [d])
        add(b + "ffn_norm.weight", ts[b + "ffn_norm"], [d])
        ff = ts[b + "gate"].shape[0]
        add(b + "ffn_gate.weight", ts[b + "gate"], [ff, d])
        add(b + "ffn_up.weight", ts[b + "up"], [ff, d])
        add(b + "ffn_down.weight", ts[b + "down"], [d, ff])
        add(b + "post_ffw_norm.weight", ts[b + "post_ffn_norm"], [d])
        if pl:
            add(b + "inp_gate.weight", ts[b + "pl_gate"], [pl, d])
            add(b + "proj.weight", ts[b + "pl_proj"], [d, pl])
            add(b + "post_norm.weight", ts[b + "pl_norm"], [d])
            add(b + "layer_output_scale.weight", ts[b + "out_scale"], [1])

    head = bytearray(b"GGUF") + struct.pack("<I", 3)
    kvs = bytearray()
    n_kv = 0

    def kv(key, vtype, value):
        nonlocal n_kv
        _kv(kvs, key, vtype, value)
        n_kv += 1

    a = arch + "."
    kv("general.architecture", STR, arch)
    kv("general.alignment", U32, 32)
    kv(a + "block_count", U32, L)
    kv(a + "embedding_length", U32, d)
    kv(a + "attention.head_count", U32, H)
    kv(a + "attention.head_count_kv", U32, KV)
    kv(a + "attention.key_length", U32, hd_full)
    if g4:
        kv(a + "attention.key_length_swa", U32, hd_swa)
        kv(a + "feed_forward_length", ARR, (I32, ffs))
    else:
        kv(a + "feed_forward_length", U32, cfg["intermediate_size"])
    kv(a + "attention.sliding_window", U32, cfg["sliding_window"])
    kv(a + "attention.sliding_window_pattern", ARR, (BOOL, swa))
    kv(a + "attention.layer_norm_rms_epsilon", F32, cfg.get("rms_norm_eps", 1e-6))
    if g4:
        rp = cfg["rope_parameters"]
        kv(a + "rope.freq_base", F32, rp["full_attention"]["rope_theta"])
        kv(a + "rope.freq_base_swa", F32, rp["sliding_attention"]["rope_theta"])
        kv(a + "attention.shared_kv_layers", U32, shared)
        kv(a + "embedding_length_per_layer_input", U32, pl)
        kv(a + "final_logit_softcapping", F32, cfg.get("final_logit_softcapping", 0.0))
    else:
        kv(a + "rope.freq_base", F32, cfg.get("rope_theta", 1e6))
        kv(a + "rope.freq_base_swa", F32, cfg.get("rope_local_base_freq", 1e4))
        kv(a + "attention.query_pre_attn_scalar", U32, int(cfg.get("query_pre_attn_scalar", hd_swa)))
    kv("tokenizer.ggml.bos_token_id", U32, cfg.get("bos_token_id", 2))
    kv("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(8)]))
    infos = bytearray()
    offsets, off = [], 0
    for name, shape, kind, payload in tensors:
        off = (off + 31) // 32 * 32
        offsets.append(off)
        _s(infos, name)
        infos += struct.pack("<I", len(shape))
        for dim in reversed(shape):
            infos += struct.pack("<Q", dim)
        infos += struct.pack("<IQ", kind, off)
        off += len(payload)
    head += struct.pack("<QQ", len(tensors), n_kv)
    out = head + kvs + infos
    out += b"\0" * ((-len(out)) % 32)
    data = bytearray(off)
    for (name, shape, kind, payload), o in zip(tensors, offsets):
        data[o:o + len(payload)] = payload
    Path(path).write_bytes(bytes(out + data))
