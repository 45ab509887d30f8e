"""Checkpoint descriptions and host tensors (crates/omg-wgpu/src/model.rs).

`config_json(...)` writes the HF-style config.json that Config::from_json
reads (model.rs:66-210); `BASELINE_CONFIGS` holds the shapes of the
benchmark configurations; `Weights` is a host checkpoint in the reference's
QTensor encoding (seeded per tests/reference.rs:106-139, or read from an
exported directory); `export_dir` writes the exported-directory layout of
tools/export_wgpu_gguf.py that `Engine.open_dir` loads.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import _lib as L

F16, Q8, Q4 = L.DTYPE_F16, L.DTYPE_Q8, L.DTYPE_Q4
DTYPE_NAMES = {F16: "f16", Q8: "q8", Q4: "q4"}


def config_json(*, vocab: int, d: int, layers: int, heads: int, kv_heads: int, head_dim: int, ff: int,
                window: int, sliding: list[bool] | None = None, pattern: int = 6, eps: float = 1e-6,
                theta_global: float = 1e6, theta_local: float = 1e4, query_pre_attn_scalar: float | None = None,
                norm_offset: float | None = 0.0, bos: int = 2) -> str:
    """A Gemma 3 text config.  `sliding` lists the layer types explicitly;
    otherwise every `pattern`-th layer is global (model.rs:83-93).
    norm_offset 0 is a GGUF-derived export (the +1 folded into the norm
    weights, tools/export_wgpu_gguf.py:171-172); None keeps Gemma 3's 1."""
    cfg: dict = {
        "model_type": "gemma3_text",
        "vocab_size": vocab,
        "hidden_size": d,
        "num_hidden_layers": layers,
        "num_attention_heads": heads,
        "num_key_value_heads": kv_heads,
        "head_dim": head_dim,
        "intermediate_size": ff,
        "sliding_window": window,
        "rms_norm_eps": eps,
        "rope_theta": theta_global,
        "rope_local_base_freq": theta_local,
        "query_pre_attn_scalar": float(query_pre_attn_scalar if query_pre_attn_scalar is not None else head_dim),
        "bos_token_id": bos,
    }
    if sliding is not None:
        cfg["layer_types"] = ["sliding_attention" if s else "full_attention" for s in sliding]
    else:
        cfg["_sliding_window_pattern"] = pattern
    if norm_offset is not None:
        cfg["omg_norm_offset"] = norm_offset
    return json.dumps(cfg)


def gemma4_config_json(*, vocab: int, d: int, layers: int, heads: int, kv_heads: int, head_dim: int = 256,
                       global_head_dim: int = 512, ff: int | list[int], window: int, sliding: list[bool],
                       shared_kv_layers: int = 0, double_wide_mlp: bool = False, partial_rotary_global: float = 0.25,
                       per_layer_dim: int = 0, softcap: float = 0.0, eps: float = 1e-6, theta_global: float = 1e6,
                       theta_local: float = 1e4, bos: int = 2) -> str:
    """A Gemma 4 text config (model.rs:95-210): global layers with their own
    head_dim and partial RoPE, K/V shared by the last `shared_kv_layers`
    layers, V normed, per-layer inputs of width `per_layer_dim`, norm
    offset 0."""
    cfg: dict = {
        "model_type": "gemma4_text",
        "vocab_size": vocab,
        "hidden_size": d,
        "num_hidden_layers": layers,
        "num_attention_heads": heads,
        "num_key_value_heads": kv_heads,
        "head_dim": head_dim,
        "global_head_dim": global_head_dim,
        "intermediate_size": ff,
        "use_double_wide_mlp": double_wide_mlp,
        "num_kv_shared_layers": shared_kv_layers,
        "sliding_window": window,
        "layer_types": ["sliding_attention" if s else "full_attention" for s in sliding],
        "rope_parameters": {
            "full_attention": {"rope_theta": theta_global, "partial_rotary_factor": partial_rotary_global},
            "sliding_attention": {"rope_theta": theta_local},
        },
        "hidden_size_per_layer_input": per_layer_dim,
        "final_logit_softcapping": softcap,
        "rms_norm_eps": eps,
        "bos_token_id": bos,
    }
    return json.dumps(cfg)


# Gemma-3-shaped decoders with the vocabulary pruned
# to 25,000 rows.
GEMMA3_270M = dict(vocab=25_000, d=640, layers=18, heads=4, kv_heads=1, head_dim=256, ff=2048, window=512)
GEMMA3_1B = dict(vocab=25_000, d=1152, layers=26, heads=4, kv_heads=1, head_dim=256, ff=6912, window=512)
GEMMA3_4B = dict(vocab=25_000, d=2560, layers=34, heads=8, kv_heads=4, head_dim=256, ff=10240, window=1024)

BASELINE_CONFIGS = {
    # config 1: 270M Q8_0, 90-token state + 5 branches of 24
    "c1": dict(model=GEMMA3_270M, dtype=Q8, state=90, branches=5, branch_tokens=24),
    # config 2 (the metric's): 270M Q4_0, 2,000-token state + 12 branches of 32
    "c2": dict(model=GEMMA3_270M, dtype=Q4, state=2000, branches=12, branch_tokens=32),
    # config 3: 1B Q4_0, 500 / 2,000-token states + 12 branches of 32
    "c3": dict(model=GEMMA3_1B, dtype=Q4, state=2000, branches=12, branch_tokens=32),
    # config 5: 4B Q4_0, 8,000-token state + 208 branches of 40
    "c5": dict(model=GEMMA3_4B, dtype=Q4, state=8000, branches=208, branch_tokens=40),
}

# The reference's published Gemma 4 figures (docs/comparison.md:92,116):
# E2B Q4_0, vocabulary pruned, 12 questions over a 2,000-token state, 2,663
# tokens in all.  Shape as the E2B checkpoint's config: 35 layers of d 1,536,
# 8 query heads over 1 K/V head, head_dim 256 (sliding, window 512) / 512
# (global, every 5th layer, RoPE on a quarter), ff 6,144 (12,288 on the 20
# layers that share K/V), per-layer inputs of 256, softcap 30; the pruned
# vocabulary taken as 25,000 rows like the other configs.
GEMMA4_E2B = dict(vocab=25_000, d=1536, layers=35, heads=8, kv_heads=1, head_dim=256, global_head_dim=512, ff=6144,
                  double_wide_mlp=True, shared_kv_layers=20, window=512,
                  sliding=[(i + 1) % 5 != 0 for i in range(35)], partial_rotary_global=0.25, per_layer_dim=256,
                  softcap=30.0)
GEMMA4_CONFIGS = {
    "e2b": dict(model=GEMMA4_E2B, dtype=Q4, state=2000, branch_tokens=[56] * 3 + [55] * 9,
                published_ms={"cold": 8100.0, "warm": 2030.0}),
}

# The 26 label tokens read at each branch's answer position: option letters
# A..Z (omg-core readout.rs:11-15) mapped to fixed ids of the synthetic vocab.
LABEL_IDS = list(range(256, 256 + 26))


@dataclass
class QTensor:
    """model.rs:375-383: payload bytes + f16 block scales (Q8 / Q4)."""

    name: str
    dtype: int
    shape: tuple
    data: np.ndarray    # uint8
    scales: np.ndarray  # uint8

    def to_f32(self) -> np.ndarray:
        """Dequantized values (model.rs:507-529), row-major."""
        if self.dtype == F16:
            return self.data.view(np.float16).astype(np.float32).reshape(self.shape)
        d = self.scales.view(np.float16).astype(np.float32)
        if self.dtype == Q8:
            q = self.data.view(np.int8).astype(np.float32).reshape(-1, 32)
            return (q * d[:, None]).reshape(self.shape)
        b = self.data.reshape(-1, 16)
        q = np.concatenate([b & 0xF, b >> 4], axis=1).astype(np.float32)
        return ((q - 8.0) * d[:, None]).reshape(self.shape)


def quantize(dtype: int, values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """QTensor::quantize_q8 / quantize_q4 (model.rs:408-466) via the library."""
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    data = np.zeros(v.size if dtype == Q8 else v.size // 2, np.uint8)
    scales = np.zeros(v.size // 32 * 2, np.uint8)
    L.check(L.lib().omg_quantize(dtype, v.ctypes.data_as(C.POINTER(C.c_float)), v.size,
                                 data.ctypes.data_as(C.POINTER(C.c_uint8)),
                                 scales.ctypes.data_as(C.POINTER(C.c_uint8))))
    return data, scales


class Weights:
    """A host checkpoint held by the library (omg_weights)."""

    def __init__(self, handle, config: str):
        self._h = handle
        self.config = config

    @classmethod
    def synth(cls, config: str, seed: int, linear: int, embed: int) -> "Weights":
        h = L.handle(L.lib().omg_synth(config.encode(), seed, linear, embed))
        return cls(h, config)

    @classmethod
    def load_dir(cls, path: str | Path) -> "Weights":
        h = L.handle(L.lib().omg_load_dir(str(path).encode()))
        return cls(h, (Path(path) / "config.json").read_text())

    @classmethod
    def load_gguf(cls, path: str | Path) -> "Weights":
        """A llama.cpp GGUF's tensors in the catalogue's names (omg_load_gguf);
        `config` is None (Engine.open_gguf builds the engine from the file)."""
        return cls(L.handle(L.lib().omg_load_gguf(str(path).encode())), None)

    def __del__(self):
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_weights_free(self._h)
            self._h = None

    def __len__(self) -> int:
        return int(L.lib().omg_weights_count(self._h))

    def tensors(self):
        """QTensors in catalogue order (model.rs:277-314), as numpy copies."""
        for i in range(len(self)):
            name, dtype, ndim = C.c_char_p(), C.c_int(), C.c_size_t()
            shape = (C.c_int64 * 4)()
            data, scales = C.c_void_p(), C.c_void_p()
            nb, ns = C.c_size_t(), C.c_size_t()
            L.check(L.lib().omg_weights_get(self._h, i, C.byref(name), C.byref(dtype), shape, C.byref(ndim),
                                            C.byref(data), C.byref(nb), C.byref(scales), C.byref(ns)))
            d = np.ctypeslib.as_array(C.cast(data, C.POINTER(C.c_uint8)), (nb.value,)).copy() if nb.value else \
                np.zeros(0, np.uint8)
            s = np.ctypeslib.as_array(C.cast(scales, C.POINTER(C.c_uint8)), (ns.value,)).copy() if ns.value else \
                np.zeros(0, np.uint8)
            yield QTensor(name.value.decode(), dtype.value, tuple(shape[k] for k in range(ndim.value)), d, s)


def export_dir(weights: Weights, path: str | Path) -> None:
    """Write the exported-directory layout (tools/export_wgpu_gguf.py:43-95):
    config.json, one .bin per file group (scales run, then codes, 4-byte
    aligned), manifest.json; a Gemma 4 per-layer token table goes to
    per_layer_table.bin under the manifest's own per_layer_table entry
    (model.rs:744-750)."""
    out = Path(path)
    out.mkdir(parents=True, exist_ok=True)
    (out / "config.json").write_text(weights.config)
    groups: dict[str, list[QTensor]] = {}
    for t in weights.tensors():
        key = t.name.split(".")[0] + "." + t.name.split(".")[1] if t.name.startswith("blk.") else \
            ("per_layer_table" if t.name == "per_layer_table" else "embed")
        groups.setdefault(key, []).append(t)
    files = []
    for key, ts in groups.items():
        fname = f"{key}.bin"
        entries, off = [], 0
        with open(out / fname, "wb") as f:
            def put(b: bytes) -> tuple[int, int]:
                nonlocal off
                start = off
                f.write(b)
                off += len(b)
                while off % 4:
                    f.write(b"\0")
                    off += 1
                return start, len(b)
            for t in ts:
                e = {"name": t.name, "dtype": DTYPE_NAMES[t.dtype], "shape": list(t.shape)}
                if t.dtype != F16:
                    e["scales_offset"], e["scales_nbytes"] = put(t.scales.tobytes())
                e["offset"], e["nbytes"] = put(t.data.tobytes())
                entries.append(e)
        files.append({"path": fname, "tensors": entries})
    man: dict = {"files": [f for f in files if f["path"] != "per_layer_table.bin"]}
    for f in files:
        if f["path"] == "per_layer_table.bin":
            man["per_layer_table"] = dict(f["tensors"][0], path=f["path"])
    (out / "manifest.json").write_text(json.dumps(man, indent=1))
