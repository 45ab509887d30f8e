"""Host-side mirror of the reference's engine surface over the C ABI.

Names and meaning follow omg-core's backend contract
(crates/omg-core/src/backend.rs:9-167: Token ids, Want, BranchTokens,
BranchOutput, Group, GroupOutput, PrefixSource) and omg_wgpu's engine
(crates/omg-wgpu/src/engine.rs: EngineBuilder::{new, push, missing,
finish}, Engine::{evaluate, evaluate_groups, warmup, set_state_cache,
save_state, restore_state, is_resident, prefix_source, evict_resident},
SavedState::{to_bytes, from_bytes}).  Errors are OmgError with the
library's message, where the reference returns anyhow errors.
"""
from __future__ import annotations

import ctypes as C
import itertools
import enum
from dataclasses import dataclass, field
from pathlib import Path
from typing import Sequence

import numpy as np

from . import _lib as L
from .model import QTensor, Weights


class Want(enum.IntEnum):
    """backend.rs:14-20, plus LABELS: logits of given label ids only, and
    LABELS_LSE: those logits then the log-sum-exp of the full row (the
    inputs of readout.rs:124-146's Readout::distribution)."""

    LOGITS = L.WANT_LOGITS
    HIDDEN = L.WANT_HIDDEN
    LABELS = L.WANT_LABELS
    LABELS_LSE = L.WANT_LABELS_LSE


class PrefixSource(enum.IntEnum):
    """backend.rs:92-104."""

    NONE = L.SRC_NONE
    RESIDENT = L.SRC_RESIDENT
    RAM = L.SRC_RAM
    DISK = L.SRC_DISK
    DECODED = L.SRC_DECODED


class Role(enum.IntEnum):
    """readout.rs Mark, for the pointer readout: a wanted row that is not
    scored (Mark::Last), an option's `</opt>` row (Mark::OptEnd) or the
    `<decide>` row (Mark::Decide)."""

    NONE = L.ROLE_NONE
    OPT = L.ROLE_OPT
    DECIDE = L.ROLE_DECIDE


@dataclass
class PointerHead:
    """readout.rs:17-44 PointerHead: two affine maps d -> dp (weights
    row-major [dp, d], biases [dp]), option logits k_i . q / sqrt(dp) with
    q = W_q h_decide + b_q and k_i = W_k h_i + b_k."""

    w_q: np.ndarray
    b_q: np.ndarray
    w_k: np.ndarray
    b_k: np.ndarray

    def __post_init__(self) -> None:
        # The library copies dp x d and dp floats from each array: the four
        # shapes must agree before any pointer is passed.
        self.w_q, self.b_q, self.w_k, self.b_k = (np.ascontiguousarray(x, np.float32)
                                                  for x in (self.w_q, self.b_q, self.w_k, self.b_k))
        if self.w_q.ndim != 2 or self.w_q.shape != self.w_k.shape:
            raise ValueError(f"pointer head: weight shapes {self.w_q.shape} / {self.w_k.shape}")
        dp = self.w_q.shape[0]
        if self.b_q.shape != (dp,) or self.b_k.shape != (dp,):
            raise ValueError(f"pointer head: bias shapes {self.b_q.shape} / {self.b_k.shape}, expected ({dp},)")

    @property
    def dp(self) -> int:
        return int(self.w_q.shape[0])

    @property
    def d(self) -> int:
        return int(self.w_q.shape[1])

    @classmethod
    def load(cls, src: "str | Path | bytes") -> "PointerHead":
        """readout.rs:208-345: `head.safetensors` with q.weight [dp, d],
        q.bias [dp], k.weight, k.bias in F32, F16 or BF16."""
        data = src if isinstance(src, (bytes, bytearray)) else Path(src).read_bytes()
        if len(data) < 8:
            raise ValueError("head.safetensors: too short")
        n = int.from_bytes(data[:8], "little")
        if 8 + n > len(data):
            raise ValueError("head.safetensors: header")
        import json

        header = json.loads(data[8:8 + n])
        base = 8 + n

        def tensor(name: str) -> np.ndarray:
            t = header.get(name)
            if t is None:
                raise ValueError(f"head.safetensors: missing tensor {name}")
            lo, hi = (int(v) for v in t["data_offsets"])
            shape = [int(v) for v in t["shape"]]
            if not 0 <= lo <= hi <= len(data) - base:
                raise ValueError(f"head.safetensors: {name} data out of range")
            raw = np.frombuffer(data[base + lo:base + hi], np.uint8)
            kind = t["dtype"]
            if kind == "F32":
                v = raw.view("<f4").astype(np.float32)
            elif kind == "F16":
                v = raw.view("<f2").astype(np.float32)
            elif kind == "BF16":
                v = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
            else:
                raise ValueError(f"head.safetensors: {name} dtype {kind}")
            if v.size != int(np.prod(shape)):
                raise ValueError(f"head.safetensors: {name} size")
            return v.reshape(shape)

        w_q, b_q, w_k, b_k = (tensor(x) for x in ("q.weight", "q.bias", "k.weight", "k.bias"))
        try:
            return cls(w_q, b_q, w_k, b_k)
        except ValueError as e:
            raise ValueError(f"head.safetensors: {e}") from None


@dataclass
class BranchTokens:
    """backend.rs:22-30: branch tokens + ascending wanted indices."""

    tokens: Sequence[int]
    want: Sequence[int]


@dataclass
class BranchOutput:
    """backend.rs:32-36: rows in `want` order."""

    rows: list = field(default_factory=list)


@dataclass
class Group:
    """backend.rs:38-45 / engine.rs:26-38."""

    prefix: Sequence[int]
    branches: Sequence[BranchTokens]


@dataclass
class GroupOutput:
    """backend.rs:62-68."""

    branches: list
    prefix_source: PrefixSource


def _u32(xs) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(xs, dtype=np.int64).astype(np.uint32))


class _CGroups:
    """C views of a list of Groups; keeps the backing arrays alive.  Each
    group's branch tokens form one array and its wanted rows another; every
    omg_branch points into them by address (one conversion per group rather
    than two per branch)."""

    def __init__(self, groups: Sequence[Group]):
        self.keep = []
        self.arr = (L.omg_group * max(1, len(groups)))()
        self.n = len(groups)
        for gi, g in enumerate(groups):
            p = _u32(g.prefix)
            nb = len(g.branches)
            br = (L.omg_branch * max(1, nb))()
            nt = [len(b.tokens) for b in g.branches]
            nw = [len(b.want) for b in g.branches]
            t = _u32_joined([b.tokens for b in g.branches], sum(nt))
            w = _u32_joined([b.want for b in g.branches], sum(nw))
            ta, wa = _addr(t), _addr(w)
            for bi in range(nb):
                c = br[bi]
                c.tokens, c.ntokens, c.want, c.nwant = ta, nt[bi], wa, nw[bi]
                ta += 4 * nt[bi]
                wa += 4 * nw[bi]
            self.keep += [p, t, w, br]
            a = self.arr[gi]
            a.prefix, a.prefix_len, a.branches, a.nbranches = _addr(p), p.size, br, nb


def _u32_joined(seqs: Sequence, total: int) -> np.ndarray:
    """The sequences one after another as uint32 (as _u32 converts each)."""
    if total == 0:
        return np.zeros(1, np.uint32)
    if all(isinstance(x, np.ndarray) for x in seqs):
        return _u32(np.concatenate([np.asarray(x, dtype=np.int64).ravel() for x in seqs]))
    return np.fromiter(itertools.chain.from_iterable(seqs), np.int64, total).astype(np.uint32)


def _addr(a: np.ndarray) -> int:
    return a.__array_interface__["data"][0]


class EngineBuilder:
    """engine.rs:763-1335."""

    def __init__(self, config: str):
        self._h = L.handle(L.lib().omg_builder_new(config.encode()))
        self.config = config

    def __del__(self):
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_builder_free(self._h)
            self._h = None

    def push(self, t: QTensor) -> None:
        shape = (C.c_int64 * len(t.shape))(*t.shape)
        L.check(L.lib().omg_builder_push(self._h, t.name.encode(), t.dtype, shape, len(t.shape),
                                         t.data.ctypes.data, t.data.size, t.scales.ctypes.data if t.scales.size else None,
                                         t.scales.size))

    def push_weights(self, w: Weights) -> None:
        L.check(L.lib().omg_builder_push_weights(self._h, w._h))

    def missing(self) -> list[str]:
        buf = C.create_string_buffer(1 << 16)
        L.lib().omg_builder_missing(self._h, buf, len(buf))
        return [s for s in buf.value.decode().split("\n") if s]

    def finish(self, capacity: int, max_rows: int) -> "Engine":
        h, self._h = self._h, None
        return Engine(L.handle(L.lib().omg_builder_finish(h, capacity, max_rows)))


class Engine:
    """engine.rs:449-2182 over libomg_hip.so."""

    def __init__(self, handle):
        self._h = handle
        c = L.omg_config_t()
        L.check(L.lib().omg_config(self._h, C.byref(c)))
        self.vocab, self.d, self.layers = c.vocab, c.d, c.layers
        self.capacity, self.max_rows, self.bos = c.capacity, c.max_rows, c.bos

    @classmethod
    def new(cls, weights: Weights, capacity: int, max_rows: int) -> "Engine":
        """engine.rs:1341-1351."""
        b = EngineBuilder(weights.config)
        b.push_weights(weights)
        return b.finish(capacity, max_rows)

    @classmethod
    def open_dir(cls, path: str | Path, capacity: int, max_rows: int) -> "Engine":
        """backend.rs:28-71 (an exported directory)."""
        return cls(L.handle(L.lib().omg_open_dir(str(path).encode(), capacity, max_rows)))

    @classmethod
    def open_gguf(cls, path: str | Path, capacity: int, max_rows: int) -> "Engine":
        """A llama.cpp GGUF file read directly (omg_open_gguf)."""
        return cls(L.handle(L.lib().omg_open_gguf(str(path).encode(), capacity, max_rows)))

    def close(self) -> None:
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_close(self._h)
            self._h = None

    __del__ = close

    def warmup(self) -> None:
        L.check(L.lib().omg_warmup(self._h))

    def evaluate_groups(self, groups: Sequence[Group], want: Want, labels: Sequence[int] | None = None
                        ) -> list[GroupOutput]:
        cg = _CGroups(groups)
        lab = _u32(labels if labels is not None else [])
        width = {Want.HIDDEN: self.d, Want.LOGITS: self.vocab, Want.LABELS: lab.size,
                 Want.LABELS_LSE: lab.size + 1}[Want(want)]
        rows = sum(len(b.want) for g in groups for b in g.branches)
        out = np.empty((max(rows, 1), max(width, 1)), np.float32)  # every returned row is written
        src = (C.c_int * max(1, len(groups)))()
        L.check(L.lib().omg_evaluate_groups(self._h, cg.arr, cg.n, int(want),
                                            lab.ctypes.data_as(C.POINTER(C.c_uint32)), lab.size,
                                            out.ctypes.data_as(C.POINTER(C.c_float)), out.size, src))
        res, r = [], 0
        for gi, g in enumerate(groups):
            bo = []
            for b in g.branches:
                bo.append(BranchOutput(rows=[out[r + s, :width].copy() for s in range(len(b.want))]))
                r += len(b.want)
            res.append(GroupOutput(branches=bo, prefix_source=PrefixSource(src[gi])))
        return res

    def set_pointer_head(self, head: "PointerHead | None") -> None:
        """The head omg_evaluate_pointer scores with (None clears it)."""
        if head is None:
            L.check(L.lib().omg_set_pointer_head(self._h, 0, 0, None, None, None, None))
            return
        head.__post_init__()  # fields may have been reassigned since construction
        ts = [head.w_q, head.b_q, head.w_k, head.b_k]
        ptr = [x.ctypes.data_as(C.POINTER(C.c_float)) for x in ts]
        L.check(L.lib().omg_set_pointer_head(self._h, head.d, head.dp, *ptr))

    def evaluate_pointer(self, groups: Sequence[Group], roles: Sequence[Sequence[Sequence[int]]]
                         ) -> list[list[np.ndarray]]:
        """readout.rs:149-173 on the device: per group, per branch, the
        option logits of the rows marked Role.OPT (in want order) against
        the branch's Role.DECIDE row.  roles[g][b] has one Role per wanted
        row of branch b of group g."""
        cg = _CGroups(groups)
        flat = np.array([r for gr in roles for br in gr for r in br], np.uint8)
        k = sum(1 for gr in roles for br in gr for r in br if r == Role.OPT)
        out = np.zeros(max(k, 1), np.float32)
        written = C.c_size_t(0)
        src = (C.c_int * max(1, len(groups)))()
        L.check(L.lib().omg_evaluate_pointer(self._h, cg.arr, cg.n, flat.ctypes.data_as(C.POINTER(C.c_uint8)),
                                             flat.size, out.ctypes.data_as(C.POINTER(C.c_float)), out.size,
                                             C.byref(written), src))
        res, i = [], 0
        for gr in roles:
            gout = []
            for br in gr:
                n = sum(1 for r in br if r == Role.OPT)
                gout.append(out[i:i + n].copy())
                i += n
            res.append(gout)
        return res

    def evaluate(self, prefix: Sequence[int], branches: Sequence[BranchTokens], want: Want,
                 labels: Sequence[int] | None = None) -> list[BranchOutput]:
        """engine.rs:1386-1396."""
        return self.evaluate_groups([Group(prefix, branches)], want, labels)[0].branches

    def prefix_source(self) -> PrefixSource:
        return PrefixSource(L.lib().omg_prefix_source(self._h))

    def is_resident(self, prefix: Sequence[int]) -> bool:
        p = _u32(prefix)
        return bool(L.lib().omg_is_resident(self._h, p.ctypes.data_as(C.POINTER(C.c_uint32)), p.size))

    def evict_resident(self) -> None:
        L.lib().omg_evict_resident(self._h)

    def set_state_cache(self, nbytes: int, directory: str | Path | None, model_id: str) -> None:
        L.check(L.lib().omg_set_state_cache(self._h, nbytes, str(directory).encode() if directory else None,
                                            model_id.encode()))

    def save_state(self, prefix: Sequence[int], model_id: str) -> bytes:
        """Engine::save_state + SavedState::to_bytes: GRWS1 bytes."""
        p = _u32(prefix)
        ptr, n = C.POINTER(C.c_uint8)(), C.c_size_t()
        L.check(L.lib().omg_save_state(self._h, p.ctypes.data_as(C.POINTER(C.c_uint32)), p.size, model_id.encode(),
                                       C.byref(ptr), C.byref(n)))
        try:
            return C.string_at(ptr, n.value)
        finally:
            L.lib().omg_free_bytes(ptr)

    def restore_state(self, data: bytes, model_id: str) -> None:
        buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
        L.check(L.lib().omg_restore_state(self._h, buf, len(data), model_id.encode()))

    # ---- measurement surface ----
    def prepare(self, groups: Sequence[Group], want: Want, labels: Sequence[int] | None = None,
                first_resident: bool = False) -> None:
        cg = _CGroups(groups)
        lab = _u32(labels if labels is not None else [])
        L.check(L.lib().omg_pass_prepare(self._h, cg.arr, cg.n, int(want), lab.ctypes.data_as(C.POINTER(C.c_uint32)),
                                         lab.size, int(first_resident)))

    def launch(self) -> None:
        L.check(L.lib().omg_pass_launch(self._h))

    def graph(self, on: bool) -> None:
        """Replay the prepared pass as one captured HIP graph."""
        L.check(L.lib().omg_pass_graph(self._h, int(on)))

    def read_prepared(self, max_floats: int) -> np.ndarray:
        """The prepared pass's rows (wanted order) after its launches."""
        out = np.zeros(max(max_floats, 1), np.float32)
        n = C.c_size_t()
        L.check(L.lib().omg_pass_read(self._h, out.ctypes.data_as(C.POINTER(C.c_float)), out.size, C.byref(n)))
        return out[:n.value]

    def sync(self) -> None:
        L.check(L.lib().omg_sync(self._h))

    def profile(self, on: bool) -> None:
        L.check(L.lib().omg_profile(self._h, int(on)))

    def full_last_layer(self, on: bool) -> None:
        """Run every layer for every row (on) instead of, the default, the
        read-out rows only from the last layer that writes K/V past its
        attention on; the returned rows are the same bits."""
        L.check(L.lib().omg_set_full_last_layer(self._h, int(on)))

    def profile_report(self) -> dict[str, tuple[int, float]]:
        """kernel name -> (launches, total ms) since profiling was switched on."""
        buf = C.create_string_buffer(1 << 16)
        L.lib().omg_profile_report(self._h, buf, len(buf))
        out = {}
        for line in buf.value.decode().splitlines():
            name, n, ms = line.split()
            out[name] = (int(n), float(ms))
        return out


def pack(groups: Sequence[Group], first: int = 0, resident: bool = False, align: int = 1, rows: int = 0):
    """engine.rs:1512-1571 through omg_pack: (ids, meta[n,4], wanted[r,4]);
    align > 1: the engine's layout with later groups on multiples of
    `align` cache rows (when that fits in `rows`)."""
    cg = _CGroups(groups)
    total = sum(len(g.prefix) + sum(len(b.tokens) for b in g.branches) for g in groups)
    total += max(0, align - 1) * len(groups)
    nwant = sum(len(b.want) for g in groups for b in g.branches)
    ids = np.zeros(max(total, 1), np.uint32)
    meta = np.zeros((max(total, 1), 4), np.int32)
    wanted = np.zeros((max(nwant, 1), 4), np.int64)
    n_ids, n_w = C.c_size_t(ids.size), C.c_size_t(wanted.shape[0])
    L.check(L.lib().omg_pack(cg.arr, cg.n, first, int(resident), align, rows, ids.ctypes.data_as(C.POINTER(C.c_uint32)),
                             meta.ctypes.data_as(C.POINTER(C.c_int32)), wanted.ctypes.data_as(C.POINTER(C.c_int64)),
                             C.byref(n_ids), C.byref(n_w)))
    return ids[:n_ids.value], meta[:n_ids.value], wanted[:n_w.value]


def state_key(model_id: str, prefix: Sequence[int]) -> int:
    p = _u32(prefix)
    return int(L.lib().omg_state_key(model_id.encode(), p.ctypes.data_as(C.POINTER(C.c_uint32)), p.size))


def state_check(data: bytes, model_id: str) -> tuple[int, int]:
    """SavedState::from_bytes without an engine: (prefix length, layers)."""
    buf = (C.c_uint8 * max(1, len(data))).from_buffer_copy(data if data else b"\0")
    pl, nl = C.c_size_t(), C.c_size_t()
    L.check(L.lib().omg_state_check(buf, len(data), model_id.encode(), C.byref(pl), C.byref(nl)))
    return pl.value, nl.value


class DeviceWeight:
    """A weight uploaded in the device layout, for the kernel-level tests."""

    def __init__(self, t: QTensor):
        rows, cols = t.shape
        self._h = L.handle(L.lib().omg_weight_upload(t.dtype, rows, cols, t.data.ctypes.data,
                                                     t.scales.ctypes.data if t.scales.size else None))
        self.rows, self.cols = rows, cols

    def __del__(self):
        lib = getattr(L, "_lib", None)
        if lib is not None and getattr(self, "_h", None):
            lib.omg_weight_free(self._h)
            self._h = None

    def gemm(self, x_ptr: int, ldx: int, m: int, y_ptr: int, ldy: int, stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_gemm(self._h, x_ptr, ldx, m, y_ptr, ldy, stream))

    def gemm_geglu(self, up: "DeviceWeight", x_ptr: int, ldx: int, m: int, act_ptr: int, ldact: int,
                   stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_gemm_geglu(self._h, up._h, x_ptr, ldx, m, act_ptr, ldact, stream))

    def label_readout(self, rows_ptr: int, nrows: int, labels_ptr: int, nlabels: int, softcap: float, out_ptr: int,
                      stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_label_readout(self._h, rows_ptr, nrows, labels_ptr, nlabels, softcap, out_ptr, stream))

    def label_readout_noalloc(self, rows_ptr: int, nrows: int, labels_ptr: int, nlabels: int, softcap: float,
                              out_ptr: int, stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_label_readout_noalloc(self._h, rows_ptr, nrows, labels_ptr, nlabels, softcap, out_ptr,
                                                      stream))

    def embed_norm(self, ids_ptr: int, t: int, scale: float, w_ptr: int, eps: float, x_ptr: int, hn_ptr: int,
                   stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_embed_norm(self._h, ids_ptr, t, scale, w_ptr, eps, x_ptr, hn_ptr, stream))

    def gemm_geglu_erf(self, up: "DeviceWeight", x_ptr: int, ldx: int, m: int, act_ptr: int, ldact: int,
                       stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_gemm_geglu_erf(self._h, up._h, x_ptr, ldx, m, act_ptr, ldact, stream))

    def gemm_bias_relu(self, x_ptr: int, ldx: int, m: int, bias_ptr: int, y_ptr: int, ldy: int,
                       stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_gemm_bias_relu(self._h, x_ptr, ldx, m, bias_ptr, y_ptr, ldy, stream))

    def qkv_heads(self, x_ptr: int, ldx: int, m: int, bias_ptr: int | None, rope_ptr: int | None,
                  meta_ptr: int | None, qscale: float, tpad: int, q_ptr: int, k_ptr: int, vt_ptr: int,
                  stream: int | None = None) -> None:
        L.check(L.lib().omg_dev_qkv_heads(self._h, x_ptr, ldx, m, bias_ptr, rope_ptr, meta_ptr, qscale, tpad, q_ptr,
                                          k_ptr, vt_ptr, stream))


def attention_bi(q_ptr: int, k_ptr: int, vt_ptr: int, meta_ptr: int, heads: int, t: int, tpad: int, window: int,
                 out_ptr: int, stream: int | None = None) -> None:
    """The encoder path's attention kernel on device pointers."""
    L.check(L.lib().omg_dev_attention_bi(q_ptr, k_ptr, vt_ptr, meta_ptr, heads, t, tpad, window, out_ptr, stream))
