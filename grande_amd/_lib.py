"""ctypes binding of include/omg_hip.h (libomg_hip.so, built in-tree by
grande_amd/build.py).  Loading fails loudly when the library is missing:
there is no fallback path."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libomg_hip.so"

OK = 0
E_INVALID, E_CAPACITY, E_DEVICE, E_STATE, E_IO, E_MISSING = -1, -2, -3, -4, -5, -6
DTYPE_F16, DTYPE_Q8, DTYPE_Q4 = 0, 1, 2
WANT_LOGITS, WANT_HIDDEN, WANT_LABELS, WANT_LABELS_LSE = 0, 1, 2, 3
SRC_NONE, SRC_RESIDENT, SRC_RAM, SRC_DISK, SRC_DECODED = 0, 1, 2, 3, 4
ROLE_NONE, ROLE_OPT, ROLE_DECIDE = 0, 1, 2


class OmgError(RuntimeError):
    """A non-zero status from the C ABI, with omg_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


# The uint32 pointers are declared void* here (same ABI): the wrapper sets
# them from array addresses, which is much cheaper than typed pointers.
class omg_branch(C.Structure):
    _fields_ = [("tokens", C.c_void_p), ("ntokens", C.c_size_t),
                ("want", C.c_void_p), ("nwant", C.c_size_t)]


class omg_group(C.Structure):
    _fields_ = [("prefix", C.c_void_p), ("prefix_len", C.c_size_t),
                ("branches", C.POINTER(omg_branch)), ("nbranches", C.c_size_t)]


class omg_config_t(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("d", C.c_uint32), ("layers", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("bos", C.c_uint32),
                ("capacity", C.c_uint64), ("max_rows", C.c_uint64)]


class omg_laya_seq(C.Structure):
    _fields_ = [("ids", C.POINTER(C.c_uint32)), ("nids", C.c_size_t), ("markers", C.POINTER(C.c_uint32)),
                ("nmarkers", C.c_size_t), ("qtype", C.c_int)]


class omg_laya_config_t(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("d", C.c_uint32), ("layers", C.c_uint32), ("heads", C.c_uint32),
                ("ff", C.c_uint32), ("head_layers", C.c_uint32), ("act_out", C.c_uint32), ("max_len", C.c_uint32),
                ("cls", C.c_uint32), ("sep", C.c_uint32), ("mask", C.c_uint32), ("pad", C.c_uint32),
                ("capacity", C.c_uint64), ("max_rows", C.c_uint64)]


_P = C.c_void_p
_SIGS = {
    "omg_last_error": (C.c_char_p, []),
    "omg_builder_new": (_P, [C.c_char_p]),
    "omg_builder_push": (C.c_int, [_P, C.c_char_p, C.c_int, C.POINTER(C.c_int64), C.c_size_t, _P, C.c_size_t, _P,
                                   C.c_size_t]),
    "omg_synth": (_P, [C.c_char_p, C.c_uint64, C.c_int, C.c_int]),
    "omg_load_dir": (_P, [C.c_char_p]),
    "omg_load_gguf": (_P, [C.c_char_p]),
    "omg_open_gguf": (_P, [C.c_char_p, C.c_size_t, C.c_size_t]),
    "omg_weights_count": (C.c_size_t, [_P]),
    "omg_weights_get": (C.c_int, [_P, C.c_size_t, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int64),
                                  C.POINTER(C.c_size_t), C.POINTER(_P), C.POINTER(C.c_size_t), C.POINTER(_P),
                                  C.POINTER(C.c_size_t)]),
    "omg_weights_free": (None, [_P]),
    "omg_builder_push_weights": (C.c_int, [_P, _P]),
    "omg_builder_missing": (C.c_size_t, [_P, C.c_char_p, C.c_size_t]),
    "omg_builder_finish": (_P, [_P, C.c_size_t, C.c_size_t]),
    "omg_builder_free": (None, [_P]),
    "omg_open_dir": (_P, [C.c_char_p, C.c_size_t, C.c_size_t]),
    "omg_close": (None, [_P]),
    "omg_config": (C.c_int, [_P, C.POINTER(omg_config_t)]),
    "omg_warmup": (C.c_int, [_P]),
    "omg_evaluate_groups": (C.c_int, [_P, C.POINTER(omg_group), C.c_size_t, C.c_int, C.POINTER(C.c_uint32),
                                      C.c_size_t, C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_int)]),
    "omg_set_pointer_head": (C.c_int, [_P, C.c_size_t, C.c_size_t, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                       C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "omg_evaluate_pointer": (C.c_int, [_P, C.POINTER(omg_group), C.c_size_t, C.POINTER(C.c_uint8), C.c_size_t,
                                       C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_size_t), C.POINTER(C.c_int)]),
    "omg_evaluate": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(omg_branch), C.c_size_t, C.c_int,
                               C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(C.c_float), C.c_size_t]),
    "omg_prefix_source": (C.c_int, [_P]),
    "omg_is_resident": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_size_t]),
    "omg_evict_resident": (None, [_P]),
    "omg_set_state_cache": (C.c_int, [_P, C.c_size_t, C.c_char_p, C.c_char_p]),
    "omg_save_state": (C.c_int, [_P, C.POINTER(C.c_uint32), C.c_size_t, C.c_char_p, C.POINTER(C.POINTER(C.c_uint8)),
                                 C.POINTER(C.c_size_t)]),
    "omg_restore_state": (C.c_int, [_P, C.POINTER(C.c_uint8), C.c_size_t, C.c_char_p]),
    "omg_free_bytes": (None, [C.POINTER(C.c_uint8)]),
    "omg_quantize": (C.c_int, [C.c_int, C.POINTER(C.c_float), C.c_size_t, C.POINTER(C.c_uint8),
                               C.POINTER(C.c_uint8)]),
    "omg_pack": (C.c_int, [C.POINTER(omg_group), C.c_size_t, C.c_size_t, C.c_int, C.c_size_t, C.c_size_t,
                           C.POINTER(C.c_uint32),
                           C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_size_t),
                           C.POINTER(C.c_size_t)]),
    "omg_state_key": (C.c_uint64, [C.c_char_p, C.POINTER(C.c_uint32), C.c_size_t]),
    "omg_state_check": (C.c_int, [C.POINTER(C.c_uint8), C.c_size_t, C.c_char_p, C.POINTER(C.c_size_t),
                                  C.POINTER(C.c_size_t)]),
    "omg_pass_prepare": (C.c_int, [_P, C.POINTER(omg_group), C.c_size_t, C.c_int, C.POINTER(C.c_uint32),
                                   C.c_size_t, C.c_int]),
    "omg_pass_launch": (C.c_int, [_P]),
    "omg_pass_graph": (C.c_int, [_P, C.c_int]),
    "omg_pass_read": (C.c_int, [_P, _P, C.c_size_t, C.POINTER(C.c_size_t)]),
    "omg_sync": (C.c_int, [_P]),
    "omg_profile": (C.c_int, [_P, C.c_int]),
    "omg_set_full_last_layer": (C.c_int, [_P, C.c_int]),
    "omg_profile_report": (C.c_size_t, [_P, C.c_char_p, C.c_size_t]),
    "omg_weight_upload": (_P, [C.c_int, C.c_int64, C.c_int64, _P, _P]),
    "omg_weight_free": (None, [_P]),
    "omg_dev_gemm": (C.c_int, [_P, _P, C.c_int64, C.c_int64, _P, C.c_int64, _P]),
    "omg_dev_gemm_geglu": (C.c_int, [_P, _P, _P, C.c_int64, C.c_int64, _P, C.c_int64, _P]),
    "omg_dev_embed_norm": (C.c_int, [_P, _P, C.c_int64, C.c_float, _P, C.c_float, _P, _P, _P]),
    "omg_dev_label_readout": (C.c_int, [_P, _P, C.c_int64, _P, C.c_int64, C.c_float, _P, _P]),
    "omg_dev_label_readout_noalloc": (C.c_int, [_P, _P, C.c_int64, _P, C.c_int64, C.c_float, _P, _P]),
    "omg_dev_gemm_geglu_erf": (C.c_int, [_P, _P, _P, C.c_int64, C.c_int64, _P, C.c_int64, _P]),
    "omg_dev_gemm_bias_relu": (C.c_int, [_P, _P, C.c_int64, C.c_int64, _P, _P, C.c_int64, _P]),
    "omg_dev_qkv_heads": (C.c_int, [_P, _P, C.c_int64, C.c_int64, _P, _P, _P, C.c_float, C.c_int64, _P, _P, _P,
                                    _P]),
    "omg_dev_attention_bi": (C.c_int, [_P, _P, _P, _P, C.c_int, C.c_int64, C.c_int64, C.c_int, _P, _P]),
    "omg_laya_builder_new": (_P, [C.c_char_p]),
    "omg_laya_builder_push": (C.c_int, [_P, C.c_char_p, C.c_int, C.POINTER(C.c_int64), C.c_size_t, _P, C.c_size_t,
                                        _P, C.c_size_t]),
    "omg_laya_builder_push_weights": (C.c_int, [_P, _P]),
    "omg_laya_builder_missing": (C.c_size_t, [_P, C.c_char_p, C.c_size_t]),
    "omg_laya_builder_finish": (_P, [_P, C.c_size_t, C.c_size_t]),
    "omg_laya_builder_free": (None, [_P]),
    "omg_laya_synth": (_P, [C.c_char_p, C.c_uint64, C.c_int, C.c_int]),
    "omg_laya_close": (None, [_P]),
    "omg_laya_open_dir": (_P, [C.c_char_p, _P, C.c_size_t, C.c_size_t]),
    "omg_laya_load_dir": (_P, [C.c_char_p, _P]),
    "omg_laya_config": (C.c_int, [_P, C.POINTER(omg_laya_config_t)]),
    "omg_laya_warmup": (C.c_int, [_P]),
    "omg_laya_hidden": (C.c_int, [_P, C.POINTER(omg_laya_seq), C.c_size_t, C.POINTER(C.c_float), C.c_size_t]),
    "omg_laya_evaluate": (C.c_int, [_P, C.POINTER(omg_laya_seq), C.c_size_t, C.POINTER(C.c_float), C.c_size_t,
                                    C.POINTER(C.c_float), C.c_size_t]),
    "omg_laya_temperature": (C.c_int, [_P, C.c_int, C.c_size_t, C.POINTER(C.c_float)]),
    "omg_laya_prepare": (C.c_int, [_P, C.POINTER(omg_laya_seq), C.c_size_t]),
    "omg_laya_launch": (C.c_int, [_P]),
    "omg_laya_sync": (C.c_int, [_P]),
    "omg_laya_profile": (C.c_int, [_P, C.c_int]),
    "omg_laya_set_full_last_layer": (C.c_int, [_P, C.c_int]),
    "omg_laya_profile_report": (C.c_size_t, [_P, C.c_char_p, C.c_size_t]),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m grande_amd.build`")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().omg_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(code: int) -> None:
    if code != OK:
        raise OmgError(code, last_error())


def handle(ptr):
    if not ptr:
        raise OmgError(E_INVALID, last_error())
    return ptr
