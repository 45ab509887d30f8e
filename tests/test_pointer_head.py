"""The pointer head's file reader (readout.rs:208-345): head.safetensors
tensors q.weight [dp, d], q.bias, k.weight, k.bias in F32, F16 or BF16,
written here with the safetensors package, and its refusals."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

import grande_amd as g

st = pytest.importorskip("safetensors.numpy")


def arrays(rng, d=6, dp=4):
    return {"q.weight": rng.standard_normal((dp, d)), "q.bias": rng.standard_normal(dp),
            "k.weight": rng.standard_normal((dp, d)), "k.bias": rng.standard_normal(dp)}


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_head_loads_f32_and_f16(tmp_path, dtype):
    t = {k: v.astype(dtype) for k, v in arrays(np.random.default_rng(1)).items()}
    path = tmp_path / "head.safetensors"
    st.save_file(t, str(path))
    h = g.PointerHead.load(path)
    assert (h.d, h.dp) == (6, 4)
    for got, name in ((h.w_q, "q.weight"), (h.b_q, "q.bias"), (h.w_k, "k.weight"), (h.b_k, "k.bias")):
        assert got.dtype == np.float32 and np.array_equal(got, t[name].astype(np.float32))
    assert g.PointerHead.load(path.read_bytes()).w_q.tobytes() == h.w_q.tobytes()


def bf16_file(t: dict, drop: str | None = None, shape_of: dict | None = None) -> bytes:
    """A safetensors file of BF16 tensors (the upper halves of the f32 bits)."""
    header, blobs, off = {}, [], 0
    for name, v in t.items():
        if name == drop:
            continue
        raw = (v.astype(np.float32).view(np.uint32) >> 16).astype("<u2").tobytes()
        shape = (shape_of or {}).get(name, list(v.shape))
        header[name] = {"dtype": "BF16", "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def test_head_loads_bf16():
    t = arrays(np.random.default_rng(2))
    h = g.PointerHead.load(bf16_file(t))
    exp = (t["q.weight"].astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
    assert np.array_equal(h.w_q, exp)


def test_head_refusals():
    t = arrays(np.random.default_rng(3))
    with pytest.raises(ValueError, match="too short"):
        g.PointerHead.load(b"\\x01")
    with pytest.raises(ValueError, match="missing tensor k.bias"):
        g.PointerHead.load(bf16_file(t, drop="k.bias"))
    bad = dict(t, **{"k.weight": np.zeros((4, 5))})
    with pytest.raises(ValueError, match="weight shapes"):
        g.PointerHead.load(bf16_file(bad))
    bad = dict(t, **{"q.bias": np.zeros(3)})
    with pytest.raises(ValueError, match="bias shape"):
        g.PointerHead.load(bf16_file(bad))


def test_head_shapes_are_checked_on_construction():
    """A head built from arrays directly is held to the file reader's shape
    rules before any pointer reaches the library: W_q and W_k [dp, d], both
    biases [dp]."""
    rng = np.random.default_rng(3)
    a = arrays(rng)
    ok = g.PointerHead(a["q.weight"], a["q.bias"], a["k.weight"], a["k.bias"])
    assert (ok.d, ok.dp) == (6, 4) and ok.w_q.dtype == np.float32 and ok.w_q.flags.c_contiguous
    bad = [
        (a["q.weight"], a["q.bias"], a["k.weight"][:, :5], a["k.bias"]),  # W_k narrower
        (a["q.weight"], a["q.bias"], a["k.weight"][:3], a["k.bias"]),     # W_k shorter
        (a["q.weight"], a["q.bias"][:3], a["k.weight"], a["k.bias"]),     # b_q short
        (a["q.weight"], a["q.bias"], a["k.weight"], np.zeros(5)),        # b_k long
        (a["q.weight"].ravel(), a["q.bias"], a["k.weight"].ravel(), a["k.bias"]),  # not 2-D
    ]
    for args in bad:
        with pytest.raises(ValueError, match="pointer head"):
            g.PointerHead(*args)
