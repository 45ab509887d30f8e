"""The bidirectional encoder path (crates/omg-wgpu/src/laya.rs): Laya's
mmBERT / ModernBERT encoder with its decision head, on the gfx950 kernels
behind include/omg_hip.h.

`laya_config_json(...)` writes the exported directory's config.json
(the encoder config with the agent config under "laya_agent" and the
special token ids under "laya_tokens", laya.rs:312-323); `LayaBuilder` /
`LayaEngine` mirror the reference's types of the same names; `Sequence` and
`Output` are laya.rs:468-488's.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass, field
from typing import Sequence as Seq

import numpy as np

from . import _lib as L
from .model import Q8, QTensor, Weights

QTYPES = ("choice", "score", "noul")  # laya.rs:43-45


def laya_config_json(*, vocab: int, d: int, layers: int, heads: int, ff: int, local_attention: int = 128,
                     global_every: int = 3, sliding: list[bool] | None = None, eps: float = 1e-5,
                     theta_global: float = 160000.0, theta_local: float = 10000.0, head_layers: int = 2,
                     type_emb: bool = True, act_costs: dict | None = None, max_len: int = 512,
                     head_max_len: int = 192, temperature=(1.0, 1.0, 1.0), temperature_by_options: dict | None = None,
                     cls: int = 1, sep: int = 2, mask: int = 4, pad: int = 0) -> str:
    cfg: dict = {
        "model_type": "modernbert",
        "vocab_size": vocab,
        "hidden_size": d,
        "num_hidden_layers": layers,
        "num_attention_heads": heads,
        "intermediate_size": ff,
        "local_attention": local_attention,
        "global_attn_every_n_layers": global_every,
        "global_rope_theta": theta_global,
        "local_rope_theta": theta_local,
        "norm_eps": eps,
        "hidden_activation": "gelu",
        "laya_agent": {
            "head_layers": head_layers,
            "type_emb": type_emb,
            "max_len": max_len,
            "head_max_len": head_max_len,
            "temperature": list(temperature),
        },
        "laya_tokens": {"cls_token": cls, "sep_token": sep, "mask_token": mask, "pad_token": pad},
    }
    if sliding is not None:
        cfg["layer_types"] = ["sliding_attention" if s else "full_attention" for s in sliding]
    if act_costs is not None:
        cfg["laya_agent"]["act_costs"] = act_costs
    else:
        cfg["laya_agent"]["act_head"] = False
    if temperature_by_options:
        cfg["laya_agent"]["temperature_by_options"] = temperature_by_options
    return json.dumps(cfg)


# mmBERT-base-shaped encoder, Q8_0, 56,000-token
# vocabulary; 64 requests x 3 questions of 256 tokens, one [MASK] each.
MMBERT_BASE = dict(vocab=56_000, d=768, layers=22, heads=12, ff=1152, local_attention=128, global_every=3)
C4 = dict(model=MMBERT_BASE, dtype=Q8, requests=64, questions=3, seq_len=256)


@dataclass
class Sequence:
    """One question (laya.rs:468-476): token ids, the index of each option's
    [MASK], the question type (0 choice, 1 score, 2 noul)."""
    ids: list[int]
    markers: list[int]
    qtype: int = 0


@dataclass
class Output:
    """laya.rs:478-488: the scorer's raw logit per option and the act
    head's probability (None without an act head)."""
    logits: np.ndarray
    act_probability: float | None = None


def synth_weights(config: str, seed: int, linear: int, embed: int) -> Weights:
    """Seeded weights for an encoder config (omg_laya_synth)."""
    h = L.handle(L.lib().omg_laya_synth(config.encode(), seed, linear, embed))
    return Weights(h, config)


def _special(special):
    if special is None:
        return None
    arr = (C.c_uint32 * 4)(*special)
    return arr


def load_dir(path, special=None) -> Weights:
    """An exported directory's tensors (omg_laya_load_dir); `special` =
    (cls, sep, mask, pad) ids replaces the config's laya_tokens."""
    from pathlib import Path
    h = L.handle(L.lib().omg_laya_load_dir(str(path).encode(), _special(special)))
    return Weights(h, (Path(path) / "config.json").read_text())


class _CSeqs:
    def __init__(self, seqs: Seq[Sequence]):
        self.keep = []
        self.arr = (L.omg_laya_seq * max(1, len(seqs)))()
        for i, s in enumerate(seqs):
            ids = np.ascontiguousarray(s.ids, np.uint32)
            mk = np.ascontiguousarray(s.markers, np.uint32)
            self.keep += [ids, mk]
            self.arr[i].ids = ids.ctypes.data_as(C.POINTER(C.c_uint32))
            self.arr[i].nids = ids.size
            self.arr[i].markers = mk.ctypes.data_as(C.POINTER(C.c_uint32))
            self.arr[i].nmarkers = mk.size
            self.arr[i].qtype = int(s.qtype)
        self.n = len(seqs)


class LayaBuilder:
    """laya.rs:611-1083."""

    def __init__(self, config: str):
        self._h = L.handle(L.lib().omg_laya_builder_new(config.encode()))

    def __del__(self):
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_laya_builder_free(self._h)
            self._h = None

    def push(self, t: QTensor) -> None:
        shape = (C.c_int64 * len(t.shape))(*t.shape)
        L.check(L.lib().omg_laya_builder_push(self._h, t.name.encode(), t.dtype, shape, len(t.shape),
                                              t.data.ctypes.data, t.data.size,
                                              t.scales.ctypes.data if t.scales.size else None, t.scales.size))

    def push_weights(self, w: Weights) -> None:
        L.check(L.lib().omg_laya_builder_push_weights(self._h, w._h))

    def missing(self) -> list[str]:
        buf = C.create_string_buffer(1 << 16)
        L.lib().omg_laya_builder_missing(self._h, buf, len(buf))
        return [s for s in buf.value.decode().split("\n") if s]

    def finish(self, capacity: int, max_rows: int) -> "LayaEngine":
        h, self._h = self._h, None
        return LayaEngine(L.handle(L.lib().omg_laya_builder_finish(h, capacity, max_rows)))


class LayaEngine:
    """laya.rs:1086-1494."""

    def __init__(self, handle):
        self._h = handle
        cfg = L.omg_laya_config_t()
        L.check(L.lib().omg_laya_config(self._h, C.byref(cfg)))
        self.d, self.capacity, self.max_rows = cfg.d, cfg.capacity, cfg.max_rows
        self.act_out = cfg.act_out
        self.cls, self.sep, self.mask = cfg.cls, cfg.sep, cfg.mask

    @classmethod
    def open_dir(cls, path, capacity: int, max_rows: int, special=None) -> "LayaEngine":
        """LayaBackend::load of an exported directory (omg_laya_open_dir)."""
        return cls(L.handle(L.lib().omg_laya_open_dir(str(path).encode(), _special(special), capacity, max_rows)))

    @classmethod
    def new(cls, weights: Weights, capacity: int, max_rows: int) -> "LayaEngine":
        b = LayaBuilder(weights.config)
        b.push_weights(weights)
        return b.finish(capacity, max_rows)

    def close(self) -> None:
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_laya_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def warmup(self) -> None:
        L.check(L.lib().omg_laya_warmup(self._h))

    def hidden(self, seqs: Seq[Sequence]) -> list[np.ndarray]:
        """Per sequence: the [CLS] row then each marker's row (laya.rs:1138)."""
        cs = _CSeqs(seqs)
        rows = sum(1 + len(s.markers) for s in seqs)
        out = np.zeros((rows, self.d), np.float32)
        L.check(L.lib().omg_laya_hidden(self._h, cs.arr, cs.n, out.ctypes.data_as(C.POINTER(C.c_float)), out.size))
        res, at = [], 0
        for s in seqs:
            n = 1 + len(s.markers)
            res.append(out[at:at + n])
            at += n
        return res

    def evaluate(self, seqs: Seq[Sequence]) -> list[Output]:
        """Scorer logits per option and the act probability (laya.rs:1435)."""
        cs = _CSeqs(seqs)
        nlog = sum(len(s.markers) for s in seqs)
        logits = np.zeros(max(1, nlog), np.float32)
        act = np.zeros(max(1, len(seqs)), np.float32)
        L.check(L.lib().omg_laya_evaluate(self._h, cs.arr, cs.n, logits.ctypes.data_as(C.POINTER(C.c_float)), nlog,
                                          act.ctypes.data_as(C.POINTER(C.c_float)), len(seqs)))
        out, at = [], 0
        for i, s in enumerate(seqs):
            k = len(s.markers)
            out.append(Output(logits[at:at + k].copy(), None if np.isnan(act[i]) else float(act[i])))
            at += k
        return out

    def temperature_for(self, qtype: int, k: int) -> float:
        t = C.c_float(0.0)
        L.check(L.lib().omg_laya_temperature(self._h, qtype, k, C.byref(t)))
        return float(t.value)

    def probabilities(self, qtype: int, logits: np.ndarray) -> np.ndarray:
        """laya.rs:1487-1493: softmax of logits / the calibration temperature."""
        t = max(self.temperature_for(qtype, len(logits)), 1e-3)
        z = np.asarray(logits, np.float32) / np.float32(t)
        e = np.exp(z - z.max())
        return (e / e.sum()).astype(np.float64)

    # measurement surface
    def prepare(self, seqs: Seq[Sequence]) -> None:
        self._prepared = _CSeqs(seqs)
        L.check(L.lib().omg_laya_prepare(self._h, self._prepared.arr, self._prepared.n))

    def launch(self) -> None:
        L.check(L.lib().omg_laya_launch(self._h))

    def sync(self) -> None:
        L.check(L.lib().omg_laya_sync(self._h))

    def profile(self, on: bool) -> None:
        L.check(L.lib().omg_laya_profile(self._h, int(on)))

    def full_last_layer(self, on: bool) -> None:
        """Run the last head layer for every row (on) instead of the read-out
        rows only (the default); the returned rows are the same bits."""
        L.check(L.lib().omg_laya_set_full_last_layer(self._h, int(on)))

    def profile_report(self) -> dict[str, tuple[int, float]]:
        n = L.lib().omg_laya_profile_report(self._h, None, 0)
        buf = C.create_string_buffer(n + 1)
        L.lib().omg_laya_profile_report(self._h, buf, len(buf))
        out = {}
        for line in buf.value.decode().splitlines():
            name, cnt, ms = line.split()
            out[name] = (int(cnt), float(ms))
        return out
