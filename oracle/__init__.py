"""CPU oracle: a restatement of the reference's decision-path forward.

TEST INFRASTRUCTURE ONLY.  Nothing in grande_amd/ imports this package;
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do,
and only as the checker or the timed CPU baseline.  See oracle.h for the
reference lines each function restates, and tests/test_oracle.py for how
each one is pinned.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"
F16, Q8, Q4 = 0, 1, 2
MAX_LAYERS = 64


def build() -> None:
    """Compile the oracle (oracle/Makefile) into oracle/_build."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _has_avx512() -> bool:
    try:
        return "avx512f" in Path("/proc/cpuinfo").read_text()
    except OSError:
        return False


class orc_config(C.Structure):
    _fields_ = [("vocab", C.c_int32), ("d", C.c_int32), ("layers", C.c_int32), ("heads", C.c_int32),
                ("kv_heads", C.c_int32), ("head_dim", C.c_int32 * MAX_LAYERS), ("ff", C.c_int32 * MAX_LAYERS),
                ("sliding", C.c_int32 * MAX_LAYERS), ("kv_source", C.c_int32 * MAX_LAYERS),
                ("rope_dims", C.c_int32 * MAX_LAYERS), ("eps", C.c_float), ("window", C.c_int32),
                ("theta_global", C.c_float), ("theta_local", C.c_float), ("query_scale", C.c_float),
                ("norm_offset", C.c_float), ("v_norm", C.c_int32), ("softcap", C.c_float), ("bos", C.c_int32),
                ("per_layer_dim", C.c_int32)]


class orc_laya_config(C.Structure):
    _fields_ = [("vocab", C.c_int32), ("d", C.c_int32), ("layers", C.c_int32), ("heads", C.c_int32),
                ("ff", C.c_int32), ("window", C.c_int32), ("head_layers", C.c_int32), ("type_emb", C.c_int32),
                ("act_hidden", C.c_int32), ("act_out", C.c_int32), ("sliding", C.c_int32 * MAX_LAYERS),
                ("theta_global", C.c_float), ("theta_local", C.c_float), ("eps", C.c_float)]


class orc_branch(C.Structure):
    _fields_ = [("tokens", C.POINTER(C.c_uint32)), ("ntokens", C.c_int64), ("want", C.POINTER(C.c_int64)),
                ("nwant", C.c_int64)]


class orc_group(C.Structure):
    _fields_ = [("prefix", C.POINTER(C.c_uint32)), ("prefix_len", C.c_int64), ("branches", C.POINTER(orc_branch)),
                ("nbranches", C.c_int64)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        path = BUILD / ("liboracle_v4.so" if _has_avx512() else "liboracle_v3.so")
        if not path.exists():
            build()
        L = C.CDLL(str(path))
        P = C.c_void_p
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_rng_next": (C.c_float, [C.POINTER(C.c_uint64)]),
            "orc_rng_values": (None, [C.POINTER(C.c_uint64), C.POINTER(C.c_float), C.c_size_t, C.c_float]),
            "orc_quantize_q8": (C.c_int, [P, C.c_size_t, P, P]),
            "orc_quantize_q4": (C.c_int, [P, C.c_size_t, P, P]),
            "orc_get": (C.c_float, [C.c_int, P, P, C.c_size_t]),
            "orc_model_new": (P, [C.POINTER(orc_config), C.c_int]),
            "orc_model_free": (None, [P]),
            "orc_model_set_attention_tiles": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_float]),
            "orc_model_set": (C.c_int, [P, C.c_char_p, C.c_int, C.c_int64, C.c_int64, P, P]),
            "orc_model_missing": (C.c_int, [P, C.c_char_p, C.c_size_t]),
            "orc_forward": (C.c_int, [P, P, P, P, C.c_int64, P]),
            "orc_logits": (C.c_int, [P, P, C.c_int64, P]),
            "orc_pack": (C.c_int, [C.POINTER(orc_group), C.c_int64, C.c_int64, C.c_int, P, P, P, P,
                                   C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
            "orc_state_key": (C.c_uint64, [C.c_char_p, P, C.c_int64]),
            "orc_state_rows": (None, [C.c_int, C.c_int64, C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
            "orc_softmax": (None, [P, C.c_int64, C.c_float, P]),
            "orc_log_sum_exp": (C.c_double, [P, C.c_int64]),
            "orc_confidence": (C.c_double, [P, C.c_int64]),
            "orc_argmax": (C.c_int64, [P, C.c_int64]),
            "orc_option_orders": (C.c_int64, [C.c_int64, C.c_int64, P]),
            "orc_label_readout": (None, [P, C.c_int64, P, C.c_int64, C.c_float, P, P, C.POINTER(C.c_double)]),
            "orc_pointer_logits": (None, [C.c_int64, C.c_int64, P, P, P, P, P, P, C.c_int64, P]),
            "orc_fold_mean": (None, [C.c_int64, C.c_int64, P, P, C.c_float, P]),
            "orc_laya_new": (P, [C.POINTER(orc_laya_config)]),
            "orc_laya_free": (None, [P]),
            "orc_laya_set": (C.c_int, [P, C.c_char_p, C.c_int, C.c_int64, C.c_int64, P, P]),
            "orc_laya_missing": (C.c_int, [P, C.c_char_p, C.c_size_t]),
            "orc_laya_hidden": (C.c_int, [P, P, P, P, C.c_int64, P, C.c_int64, P]),
            "orc_laya_score": (None, [P, P, C.c_int64, P, P]),
            "orc_layer_norm": (None, [P, C.c_int64, P, P, C.c_float, P]),
            "orc_erf": (C.c_float, [C.c_float]),
            "orc_gelu_erf": (C.c_float, [C.c_float]),
            "orc_rope_bi": (None, [P, C.c_int32, C.c_float, C.c_float]),
            "orc_linear": (None, [P, C.c_int64, C.c_int64, P, C.c_int64, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data


# ------------------------------------------------------------- scalars

def f32_to_f16(x: float) -> int:
    return int(lib().orc_f32_to_f16(C.c_float(x)))


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(h))


def rng_values(seed: int, n: int, scale: float = 1.0) -> tuple[np.ndarray, int]:
    """n values of the reference.rs:17-28 xorshift from state `seed`; returns
    (values, next state)."""
    s = C.c_uint64(seed)
    out = np.zeros(n, np.float32)
    lib().orc_rng_values(C.byref(s), out.ctypes.data_as(C.POINTER(C.c_float)), n, scale)
    return out, s.value


def quantize(dtype: int, values: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    v = np.ascontiguousarray(values, np.float32).ravel()
    data = np.zeros(v.size if dtype == Q8 else v.size // 2, np.uint8)
    scales = np.zeros(v.size // 32 * 2, np.uint8)
    fn = lib().orc_quantize_q8 if dtype == Q8 else lib().orc_quantize_q4
    if fn(_ptr(v), v.size, _ptr(data), _ptr(scales)) != 0:
        raise ValueError("oracle quantize: length must be a multiple of 32")
    return data, scales


def get(dtype: int, data: np.ndarray, scales: np.ndarray, n: int) -> np.ndarray:
    return np.array([lib().orc_get(dtype, _ptr(data), _ptr(scales) if scales.size else None, i) for i in range(n)],
                    np.float32)


# --------------------------------------------------------------- model

def config_from_json(text: str) -> orc_config:
    """model.rs:66-210: Gemma 3 text configs, and Gemma 4 (global layers
    with their own head_dim and partial RoPE, K/V shared by the last
    num_kv_shared_layers from the last earlier layer of their type, V
    normed, per-layer inputs)."""
    v = json.loads(text)
    v = v.get("text_config", v)
    L = int(v["num_hidden_layers"])
    gemma4 = v.get("model_type", "gemma3_text") in ("gemma4_text", "gemma4")
    if "layer_types" in v:
        sliding = [t == "sliding_attention" for t in v["layer_types"]]
    else:
        k = int(v.get("_sliding_window_pattern", 6))
        sliding = [True if k == 0 else (i + 1) % k != 0 for i in range(L)]
    rope = v.get("rope_parameters", {})
    hd_local = int(v["head_dim"])
    hd_global = int(v.get("global_head_dim", hd_local))
    rot_local = float(rope.get("sliding_attention", {}).get("partial_rotary_factor", 1.0))
    rot_global = float(rope.get("full_attention", {}).get("partial_rotary_factor", 1.0))
    shared = int(v.get("num_kv_shared_layers", 0))
    first_shared = L - shared
    ff = v["intermediate_size"]
    if isinstance(ff, list):
        ff = [int(x) for x in ff]
    else:
        dbl = bool(v.get("use_double_wide_mlp", False))
        ff = [2 * int(ff) if dbl and i >= first_shared else int(ff) for i in range(L)]
    c = orc_config()
    c.vocab, c.d, c.layers = int(v["vocab_size"]), int(v["hidden_size"]), L
    c.heads, c.kv_heads = int(v["num_attention_heads"]), int(v["num_key_value_heads"])
    for i in range(L):
        hd = hd_local if sliding[i] else hd_global
        src = i
        if i >= first_shared:
            src = next(j for j in range(first_shared - 1, -1, -1) if sliding[j] == sliding[i])
        c.head_dim[i], c.ff[i], c.sliding[i], c.kv_source[i] = hd, ff[i], int(sliding[i]), src
        c.rope_dims[i] = int(hd * (rot_local if sliding[i] else rot_global))
    c.eps = float(v.get("rms_norm_eps", 1e-6))
    c.window = int(v.get("sliding_window", 512))
    c.theta_global = float(rope.get("full_attention", {}).get("rope_theta", v.get("rope_theta", 1e6)))
    c.theta_local = float(rope.get("sliding_attention", {}).get("rope_theta", v.get("rope_local_base_freq", 1e4)))
    if gemma4:
        c.query_scale, c.v_norm = 1.0, 1
        c.norm_offset = float(v.get("omg_norm_offset", 0.0))
    else:
        c.query_scale = float(np.float32(v.get("query_pre_attn_scalar", hd_local)) ** np.float32(-0.5))
        c.v_norm = 0
        c.norm_offset = float(v.get("omg_norm_offset", 1.0))
    c.softcap, c.bos = float(v.get("final_logit_softcapping", 0.0) or 0.0), int(v.get("bos_token_id", 2))
    c.per_layer_dim = int(v.get("hidden_size_per_layer_input", 0))
    return c


class Model:
    """orc_model: dequantized weights + the reference CPU forward."""

    def __init__(self, config_text: str, tensors, gpu_rounding: bool = False):
        self.cfg = config_from_json(config_text)
        self._h = lib().orc_model_new(C.byref(self.cfg), int(gpu_rounding))
        if not self._h:
            raise ValueError("oracle: bad config")
        for t in tensors:
            rows, cols = (t.shape[0], t.shape[1]) if len(t.shape) == 2 else (1, t.shape[0])
            rc = lib().orc_model_set(self._h, t.name.encode(), t.dtype, rows, cols, _ptr(t.data),
                                     _ptr(t.scales) if t.scales.size else None)
            if rc != 0:
                raise ValueError(f"oracle: cannot set {t.name}")
        buf = C.create_string_buffer(1 << 16)
        if lib().orc_model_missing(self._h, buf, len(buf)):
            raise ValueError("oracle: missing " + buf.value.decode())

    def set_attention_tiles(self, key_tile: int, chunk_sliding: int, chunk_global: int, tau: float = 8.0) -> "Model":
        """Model the f16 flash kernel's attention rounding (P to f16 against a
        lazily moved max, f16 chunk partials merged by weight) instead of
        the reference's f32 softmax; key_tile 0 switches it off."""
        if lib().orc_model_set_attention_tiles(self._h, key_tile, chunk_sliding, chunk_global, tau) != 0:
            raise ValueError("oracle: bad attention tiling")
        return self

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_free(self._h)
            self._h = None

    def forward(self, ids, pos, seq) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.uint32)
        pos = np.ascontiguousarray(pos, np.int32)
        seq = np.ascontiguousarray(seq, np.int32)
        out = np.zeros((ids.size, self.cfg.d), np.float32)
        rc = lib().orc_forward(self._h, _ptr(ids), _ptr(pos), _ptr(seq), ids.size, _ptr(out))
        if rc != 0:
            raise ValueError(f"oracle forward failed ({rc})")
        return out

    def logits(self, rows: np.ndarray) -> np.ndarray:
        rows = np.ascontiguousarray(rows, np.float32)
        out = np.zeros((rows.shape[0], self.cfg.vocab), np.float32)
        lib().orc_logits(self._h, _ptr(rows), rows.shape[0], _ptr(out))
        return out


def pack_single(prefix, branches) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """tests/reference.rs:368-378 pack(): one group, seq 0 for the prefix and
    b + 1 for branch b; returns (ids, pos, seq)."""
    ids, pos, seq = list(prefix), list(range(len(prefix))), [0] * len(prefix)
    for bi, b in enumerate(branches):
        for j, t in enumerate(b.tokens):
            ids.append(t)
            pos.append(len(prefix) + j)
            seq.append(bi + 1)
    return np.array(ids, np.uint32), np.array(pos, np.int32), np.array(seq, np.int32)


def pack(groups, first: int = 0, resident: bool = False):
    """engine.rs:1512-1571 restated in C (orc_pack): (ids, meta[n,4], wanted[r,4])."""
    keep = []
    arr = (orc_group * len(groups))()
    total = rows = 0
    for gi, g in enumerate(groups):
        p = np.ascontiguousarray(g.prefix, np.uint32)
        br = (orc_branch * max(1, len(g.branches)))()
        for bi, b in enumerate(g.branches):
            t = np.ascontiguousarray(b.tokens, np.uint32)
            w = np.ascontiguousarray(b.want, np.int64)
            keep += [t, w]
            br[bi].tokens = t.ctypes.data_as(C.POINTER(C.c_uint32))
            br[bi].ntokens = t.size
            br[bi].want = w.ctypes.data_as(C.POINTER(C.c_int64))
            br[bi].nwant = w.size
            total += t.size
            rows += w.size
        keep += [p, br]
        total += p.size
        arr[gi].prefix = p.ctypes.data_as(C.POINTER(C.c_uint32))
        arr[gi].prefix_len = p.size
        arr[gi].branches = br
        arr[gi].nbranches = len(g.branches)
    ids = np.zeros(max(total, 1), np.uint32)
    meta = np.zeros((max(total, 1), 4), np.int32)
    wanted = np.zeros((max(rows, 1), 4), np.int64)
    decoded = np.zeros((max(len(groups), 1), 2), np.int64)
    n_ids, n_w, n_d = C.c_int64(), C.c_int64(), C.c_int64()
    rc = lib().orc_pack(arr, len(groups), first, int(resident), _ptr(ids), _ptr(meta), _ptr(wanted), _ptr(decoded),
                        C.byref(n_ids), C.byref(n_w), C.byref(n_d))
    if rc != 0:
        raise ValueError(f"oracle pack failed ({rc})")
    return ids[:n_ids.value], meta[:n_ids.value], wanted[:n_w.value], decoded[:n_d.value]


# --------------------------------------------------------------- state

def state_key(model_id: str, prefix) -> int:
    p = np.ascontiguousarray(prefix, np.uint32)
    return int(lib().orc_state_key(model_id.encode(), _ptr(p) if p.size else None, p.size))


def state_rows(sliding: bool, window: int, p: int) -> tuple[int, int]:
    r0, r1 = C.c_int64(), C.c_int64()
    lib().orc_state_rows(int(sliding), window, p, C.byref(r0), C.byref(r1))
    return r0.value, r1.value


# ------------------------------------------------------------- readout

def softmax(z, temperature: float = 1.0) -> np.ndarray:
    z = np.ascontiguousarray(z, np.float32)
    out = np.zeros(z.size, np.float64)
    lib().orc_softmax(_ptr(z), z.size, temperature, _ptr(out))
    return out


def log_sum_exp(z) -> float:
    z = np.ascontiguousarray(z, np.float32)
    return float(lib().orc_log_sum_exp(_ptr(z), z.size))


def confidence(p) -> float:
    p = np.ascontiguousarray(p, np.float64)
    return float(lib().orc_confidence(_ptr(p), p.size))


def argmax(p) -> int:
    p = np.ascontiguousarray(p, np.float64)
    return int(lib().orc_argmax(_ptr(p), p.size))


def option_orders(k: int, n: int) -> list[list[int]]:
    out = np.zeros(max(1, 2 * k * k), np.int64)
    cnt = lib().orc_option_orders(k, n, _ptr(out))
    return [list(map(int, out[r * k:(r + 1) * k])) for r in range(cnt)]


def label_readout(row, label_ids, temperature: float = 1.0):
    """readout.rs:124-146: (label logits, probs, candidate mass)."""
    row = np.ascontiguousarray(row, np.float32)
    lab = np.ascontiguousarray(label_ids, np.uint32)
    logits = np.zeros(lab.size, np.float32)
    probs = np.zeros(lab.size, np.float64)
    mass = C.c_double()
    lib().orc_label_readout(_ptr(row), row.size, _ptr(lab), lab.size, temperature, _ptr(logits), _ptr(probs),
                            C.byref(mass))
    return logits, probs, mass.value


def pointer_logits(w_q, b_q, w_k, b_k, decide, opts) -> np.ndarray:
    w_q, b_q, w_k, b_k, decide, opts = (np.ascontiguousarray(a, np.float32) for a in (w_q, b_q, w_k, b_k, decide, opts))
    dp, d = w_q.shape
    out = np.zeros(opts.shape[0], np.float32)
    lib().orc_pointer_logits(d, dp, _ptr(w_q), _ptr(b_q), _ptr(w_k), _ptr(b_k), _ptr(decide), _ptr(opts),
                             opts.shape[0], _ptr(out))
    return out


def fold_mean(orders, logits, excluded: float = -1e4) -> np.ndarray:
    orders = np.ascontiguousarray(orders, np.int64)
    logits = np.ascontiguousarray(logits, np.float32)
    nruns, k = orders.shape
    out = np.zeros(k, np.float32)
    lib().orc_fold_mean(k, nruns, _ptr(orders), _ptr(logits), excluded, _ptr(out))
    return out


# ------------------------------------------------- bidirectional encoder

def laya_config_from_json(text: str) -> orc_laya_config:
    """The encoder config.json fields laya.rs:88-206 reads (the agent config
    under laya_agent)."""
    v = json.loads(text)
    a = v.get("laya_agent", {})
    L = int(v["num_hidden_layers"])
    if "layer_types" in v:
        sliding = [t == "sliding_attention" for t in v["layer_types"]]
    else:
        every = int(v.get("global_attn_every_n_layers", 3))
        sliding = [every != 0 and i % every != 0 for i in range(L)]
    c = orc_laya_config()
    c.vocab, c.d, c.layers = int(v["vocab_size"]), int(v["hidden_size"]), L
    c.heads, c.ff = int(v["num_attention_heads"]), int(v["intermediate_size"])
    c.window = int(v.get("local_attention", 128)) // 2
    c.head_layers = int(a.get("head_layers", 2))
    c.type_emb = int(bool(a.get("type_emb", True)))
    c.act_hidden = 256
    c.act_out = 0 if a.get("act_head") is False else (len(a.get("act_costs", {})) + 1 if "act_costs" in a else 0)
    for i in range(L):
        c.sliding[i] = int(sliding[i])
    rope = v.get("rope_parameters", {})
    c.theta_global = float(rope.get("full_attention", {}).get("rope_theta", v.get("global_rope_theta", 160000.0)))
    c.theta_local = float(rope.get("sliding_attention", {}).get("rope_theta", v.get("local_rope_theta", 10000.0)))
    c.eps = float(v.get("norm_eps", v.get("layer_norm_eps", 1e-5)))
    return c


class Laya:
    """orc_laya: the encoder path's CPU restatement (laya.c)."""

    def __init__(self, config_text: str, tensors):
        self.cfg = laya_config_from_json(config_text)
        self._h = lib().orc_laya_new(C.byref(self.cfg))
        if not self._h:
            raise ValueError("oracle: bad encoder config")
        for t in tensors:
            rows, cols = (t.shape[0], t.shape[1]) if len(t.shape) == 2 else (1, t.shape[0])
            rc = lib().orc_laya_set(self._h, t.name.encode(), t.dtype, rows, cols, _ptr(t.data),
                                    _ptr(t.scales) if t.scales.size else None)
            if rc != 0:
                raise ValueError(f"oracle: cannot set {t.name}")
        buf = C.create_string_buffer(1 << 16)
        if lib().orc_laya_missing(self._h, buf, len(buf)):
            raise ValueError("oracle: missing " + buf.value.decode())

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_laya_free(self._h)
            self._h = None

    def hidden(self, seqs) -> list[np.ndarray]:
        """Per sequence (ids, markers, qtype): the [CLS] row then each
        marker's row, as LayaEngine::hidden returns them."""
        ids, meta, qt, rows = pack_laya(seqs)
        out = np.zeros((rows.size, self.cfg.d), np.float32)
        rc = lib().orc_laya_hidden(self._h, _ptr(ids), _ptr(meta), _ptr(qt), ids.size, _ptr(rows), rows.size,
                                   _ptr(out))
        if rc != 0:
            raise ValueError(f"oracle encoder pass failed ({rc})")
        res, at = [], 0
        for s in seqs:
            n = 1 + len(s[1])
            res.append(out[at:at + n])
            at += n
        return res

    def score(self, rows: np.ndarray) -> tuple[np.ndarray, float]:
        rows = np.ascontiguousarray(rows, np.float32)
        k = rows.shape[0] - 1
        logits = np.zeros(k, np.float32)
        act = C.c_float(0.0)
        lib().orc_laya_score(self._h, _ptr(rows), k, _ptr(logits), C.byref(act))
        return logits, float(act.value)


def pack_laya(seqs):
    """laya.rs:1165-1187: sequences back to back; meta = (position, sequence,
    first row, last row + 1); rows read back = each sequence's first token,
    then its markers."""
    ids, meta, qt, rows = [], [], [], []
    for si, (tok, markers, qtype) in enumerate(seqs):
        start = len(ids)
        for i, t in enumerate(tok):
            ids.append(t)
            qt.append(qtype)
            meta += [i, si, start, start + len(tok)]
        rows.append(start)
        rows += [start + m for m in markers]
    return (np.array(ids, np.uint32), np.array(meta, np.int32), np.array(qt, np.int32), np.array(rows, np.int64))


def layer_norm(x, w, b=None, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    y = np.zeros_like(x)
    lib().orc_layer_norm(_ptr(x), x.size, _ptr(w), None if bb is None else _ptr(bb), eps, _ptr(y))
    return y


def erf(x: float) -> float:
    return float(lib().orc_erf(C.c_float(x)))


def gelu_erf(x: float) -> float:
    return float(lib().orc_gelu_erf(C.c_float(x)))


def rope_bi(v, pos: int, theta: float, scale: float = 1.0) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().orc_rope_bi(_ptr(v), pos, theta, scale)
    return v
