"""Kernel-level parity on the GPU through the C ABI: the MFMA GEMM and the
gated GeGLU GEMM against a CPU GEMM with the same f16 rounding points, on
the odd shapes of the reference's kernel tests
(crates/omg-wgpu/tests/matmul.rs:201-290, relative tolerance 2e-3) and on
the 270M configuration's shapes; the embedding gather bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DTYPES = [g.F16, g.Q8, g.Q4]


def weight(rng: np.random.Generator, n: int, k: int, dtype: int, name: str = "w") -> tuple[g.QTensor, np.ndarray]:
    """[n, k] weight in `dtype` and its dequantized values rounded to f16 —
    the kernel's rounding point (matmul.rs:178-199)."""
    v = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    if dtype == g.F16:
        t = g.QTensor(name, g.F16, (n, k), v.astype(np.float16).view(np.uint8).ravel().copy(), np.zeros(0, np.uint8))
    else:
        data, scales = oracle.quantize(dtype, v)
        t = g.QTensor(name, dtype, (n, k), data, scales)
    return t, t.to_f32().astype(np.float16).astype(np.float32)


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(23, 96, 64), (130, 200, 96), (64, 128, 32), (1, 640, 2048),
                                   (384, 1536, 640), (2384, 640, 2048), (257, 1152, 1152),
                                   (600, 1536, 4096), (1000, 640, 4128), (700, 1152, 1024), (1100, 1536, 640)])
def test_gemm_matches_cpu(m, n, k, dtype):
    rng = np.random.default_rng(m * n * k + dtype)
    x = (rng.uniform(-1, 1, (m, k)) * 4).astype(np.float16)
    t, wd = weight(rng, n, k, dtype)
    w = g.DeviceWeight(t)
    xd = dev(x)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    w.gemm(xd.data_ptr(), k, m, y.data_ptr(), n)
    torch.cuda.synchronize()
    exp = x.astype(np.float32) @ wd.T
    got = y.cpu().numpy()
    worst = float(np.max(np.abs(got - exp) / np.maximum(np.abs(exp), 1.0)))
    assert worst < 2e-3, f"gemm {dtype} {m}x{n}x{k}: max rel diff {worst}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(23, 96, 64), (70, 100, 160), (384, 2048, 640), (2384, 2048, 640),
                                   (600, 256, 1184), (130, 8192, 96), (600, 8192, 96),
                                   (1, 96, 640), (40, 100, 1184), (64, 320, 2560)])
def test_gated_matches_cpu(m, n, k, dtype):
    rng = np.random.default_rng(7 * m * n * k + dtype)
    x = rng.uniform(-1, 1, (m, k)).astype(np.float16)
    tg, gd = weight(rng, n, k, dtype, "gate")
    tu, ud = weight(rng, n, k, dtype, "up")
    wg, wu = g.DeviceWeight(tg), g.DeviceWeight(tu)
    xd = dev(x)
    act = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    wg.gemm_geglu(wu, xd.data_ptr(), k, m, act.data_ptr(), n)
    torch.cuda.synchronize()
    xf = x.astype(np.float32)
    exp = gelu(xf @ gd.T) * (xf @ ud.T)
    got = act.cpu().numpy().astype(np.float32)
    worst = float(np.max(np.abs(got - exp) / np.maximum(np.abs(exp), 1.0)))
    assert worst < 2e-3, f"gated {dtype} {m}x{n}x{k}: max rel diff {worst}"


def test_gemm_rows_are_independent_of_m():
    """A row's result does not depend on how many rows share the launch (no
    split-K, fixed k order): the basis of the bit-equal resident-prefix and
    isolation invariants."""
    rng = np.random.default_rng(5)
    n, k = 640, 2048
    t, _ = weight(rng, n, k, g.Q4)
    w = g.DeviceWeight(t)
    x = rng.uniform(-2, 2, (2384, k)).astype(np.float16)
    outs = []
    for m in (2384, 384, 17, 1):
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        xd = dev(x[:m])  # held until the launch has run
        w.gemm(xd.data_ptr(), k, m, y.data_ptr(), n)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
    for o in outs[1:]:
        assert np.array_equal(o, outs[0][:o.shape[0]])


@pytest.mark.parametrize("k", [640, 2560])
def test_gated_rows_are_independent_of_m(k):
    """The gated product's rows are the same bits whichever tile shape the
    launch's M selects (96-row tiles for long passes, 32-row tiles with a
    deeper ring for short ones, gate and up on paired waves for branch-sized
    ones): the basis of the bit-equal warm and isolated rows through the
    feed-forward."""
    rng = np.random.default_rng(11 + k)
    n = 512
    tg, _ = weight(rng, n, k, g.Q4, "gate")
    tu, _ = weight(rng, n, k, g.Q4, "up")
    wg, wu = g.DeviceWeight(tg), g.DeviceWeight(tu)
    x = rng.uniform(-1, 1, (2384, k)).astype(np.float16)
    outs = []
    for m in (2384, 513, 384, 64, 40, 1):
        act = torch.zeros((m, n), dtype=torch.float16, device="cuda")
        xd = dev(x[:m])  # held until the launch has run
        wg.gemm_geglu(wu, xd.data_ptr(), k, m, act.data_ptr(), n)
        torch.cuda.synchronize()
        outs.append(act.cpu().numpy())
    for o in outs[1:]:
        assert np.array_equal(o, outs[0][:o.shape[0]])


@pytest.mark.parametrize("dtype", DTYPES)
def test_embed_gather_bit_exact(dtype):
    """embed.wgsl:15-48 = reference.rs:182-189: x = deq(E[id]) * sqrt(d),
    bit-exact; the fused first norm within f16 rounding."""
    rng = np.random.default_rng(11 + dtype)
    vocab, d = 300, 640
    t, _ = weight(rng, vocab, d, dtype, "embed")
    w = g.DeviceWeight(t)
    ids = rng.integers(0, vocab, 97).astype(np.uint32)
    norm_w = (1.0 + rng.uniform(-0.5, 0.5, d)).astype(np.float32)
    scale = np.float32(np.sqrt(np.float32(d)))
    x = torch.zeros((ids.size, d), dtype=torch.float32, device="cuda")
    hn = torch.zeros((ids.size, d), dtype=torch.float16, device="cuda")
    idd, wd = dev(ids.view(np.int32)), dev(norm_w)
    w.embed_norm(idd.data_ptr(), ids.size, float(scale), wd.data_ptr(), 1e-6, x.data_ptr(), hn.data_ptr())
    torch.cuda.synchronize()
    deq = t.to_f32()  # exact dequantization, f32
    exp = (deq[ids] * scale).astype(np.float32)
    got = x.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), "embedding gather is not bit-exact"
    ms = (exp.astype(np.float64) ** 2).mean(axis=1, keepdims=True)
    exp_h = exp / np.sqrt(ms + 1e-6) * norm_w
    assert np.max(np.abs(hn.cpu().numpy().astype(np.float32) - exp_h)) < 1e-2 * np.max(np.abs(exp_h))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("vocab,d,nrows,softcap", [(25000, 640, 12, 0.0), (1000, 64, 1, 30.0), (4097, 1152, 37, 0.0)])
def test_label_readout_matches_cpu(vocab, d, nrows, softcap, dtype):
    """logits = rows . deq(E)^T in f32 (softcap applied), then the label
    columns and log_sum_exp of the whole row (readout.rs:124-146,
    math.rs:13-17), against float64 on the dequantized weights: label
    logits within 1e-4 of the row scale, log-sum-exp within 1e-5."""
    rng = np.random.default_rng(vocab + d + nrows + dtype)
    t, _ = weight(rng, vocab, d, dtype, "embed")
    e = t.to_f32().astype(np.float64)
    rows = rng.uniform(-1, 1, (nrows, d)).astype(np.float32)
    labels = rng.choice(vocab, 26, replace=False).astype(np.uint32)
    w = g.DeviceWeight(t)
    out = torch.zeros((nrows, 27), dtype=torch.float32, device="cuda")
    lab = dev(labels.view(np.int32))
    rd = dev(rows)
    w.label_readout(rd.data_ptr(), nrows, lab.data_ptr(), 26, softcap, out.data_ptr())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    z = rows.astype(np.float64) @ e.T
    if softcap > 0:
        z = softcap * np.tanh(z / softcap)
    m = z.max(1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(1, keepdims=True)))[:, 0]
    scale = np.maximum(np.abs(z).max(1), 1.0)
    assert np.max(np.abs(got[:, :26] - z[:, labels]) / scale[:, None]) < 1e-4
    assert np.max(np.abs(got[:, 26] - lse) / np.maximum(np.abs(lse), 1.0)) < 1e-5


def test_label_readout_odd_shapes_and_out_of_vocab_labels():
    """Widths that are not multiples of 4 (every row of the logits starts
    off the 16-byte grid) and an odd rows x vocab product (the partials sit
    past an odd count of floats) give the same label logits and log-sum-exp
    as an aligned shape's rows; a label id past the vocabulary reads
    nothing and gives NaN in its column only."""
    rng = np.random.default_rng(77)
    vocab, d, nrows = 1001, 64, 3
    t, _ = weight(rng, vocab, d, g.Q8, "embed")
    e = t.to_f32().astype(np.float64)
    rows = rng.uniform(-1, 1, (nrows, d)).astype(np.float32)
    labels = np.array([0, 5, vocab - 1, vocab, 77, 0xFFFFFFFF], np.uint32)
    w = g.DeviceWeight(t)
    out = torch.zeros((nrows, labels.size + 1), dtype=torch.float32, device="cuda")
    rd, lab = dev(rows), dev(labels.view(np.int32))  # held until the launch has run
    w.label_readout(rd.data_ptr(), nrows, lab.data_ptr(), labels.size, 0.0, out.data_ptr())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    z = rows.astype(np.float64) @ e.T
    m = z.max(1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(1, keepdims=True)))[:, 0]
    ok = labels < vocab
    assert np.isnan(got[:, :-1][:, ~ok]).all()
    assert np.max(np.abs(got[:, :-1][:, ok] - z[:, labels[ok]])) < 1e-4 * max(1.0, np.abs(z).max())
    assert np.max(np.abs(got[:, -1] - lse) / np.maximum(np.abs(lse), 1.0)) < 1e-5
