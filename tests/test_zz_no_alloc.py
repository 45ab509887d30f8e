"""omg_dev_label_readout_noalloc against omg_dev_label_readout through the C
ABI: the same rows, bit for bit, on two calls in a row (the second with
fewer rows and a smaller vocabulary, so the first call's contents are
still in the shared scratch), and the scratch limit refused cleanly."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def case(rng, vocab: int, d: int, nrows: int, dtype: int):
    v = rng.uniform(-1, 1, (vocab, d)).astype(np.float32)
    data, scales = oracle.quantize(dtype, v)
    w = g.DeviceWeight(g.QTensor("embed", dtype, (vocab, d), data, scales))
    rows = torch.from_numpy(rng.uniform(-1, 1, (nrows, d)).astype(np.float32)).cuda()
    labels = torch.from_numpy(rng.choice(vocab, 26, replace=False).astype(np.int32)).cuda()
    return w, rows, labels


def readout(w, rows, labels, nrows: int, softcap: float, noalloc: bool) -> np.ndarray:
    out = torch.full((nrows, 27), float("nan"), dtype=torch.float32, device="cuda")
    f = w.label_readout_noalloc if noalloc else w.label_readout
    f(rows.data_ptr(), nrows, labels.data_ptr(), 26, softcap, out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_readout_matches_allocating_readout():
    rng = np.random.default_rng(42)
    for vocab, d, nrows, softcap in ((25000, 640, 40, 0.0), (3000, 256, 5, 30.0)):
        w, rows, labels = case(rng, vocab, d, nrows, g.Q4)
        ref = readout(w, rows, labels, nrows, softcap, noalloc=False)
        got = readout(w, rows, labels, nrows, softcap, noalloc=True)
        assert np.isfinite(got).all()
        assert np.array_equal(got, ref), f"vocab {vocab}, {nrows} rows"


def test_noalloc_readout_refuses_beyond_its_scratch():
    rng = np.random.default_rng(3)
    w, rows, labels = case(rng, 70000, 64, 64, g.Q8)
    with pytest.raises(g.OmgError, match="scratch"):
        readout(w, rows, labels, 64, 0.0, noalloc=True)
