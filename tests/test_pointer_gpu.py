"""Readout::Pointer on the device (omg_evaluate_pointer) against the oracle's
restatement of PointerHead::logits (readout.rs:30-44, pinned in
test_oracle.py): on the engine's own hidden rows of the same request within
f32 summation order, and on the plain f32 oracle forward within the
reference's bar (2e-2 after softmax, identical argmax).  Multi-group
requests, decide rows anywhere in a branch, unscored rows, and the refusals
of readout.rs:149-173."""
from __future__ import annotations

import numpy as np
import pytest

import grande_amd as g
import oracle
from tests.common import build, gemma3_tiny, gemma4_tiny, oracle_rows
from grande_amd import BranchTokens, Group, OmgError, PointerHead, Role, Want

pytestmark = pytest.mark.gpu
O, D, N = Role.OPT, Role.DECIDE, Role.NONE


def head(rng, d, dp=24) -> PointerHead:
    s = 1.0 / np.sqrt(d)
    return PointerHead((rng.standard_normal((dp, d)) * s).astype(np.float32), rng.standard_normal(dp).astype(np.float32),
                       (rng.standard_normal((dp, d)) * s).astype(np.float32), rng.standard_normal(dp).astype(np.float32))


def request(rng, vocab):
    tok = lambda n: rng.integers(0, vocab, n).tolist()  # noqa: E731
    groups = [Group(tok(21), [BranchTokens(tok(8), [2, 4, 6, 7]), BranchTokens(tok(6), [1, 3, 5]),
                              BranchTokens(tok(7), [0, 2, 6])]),
              Group(tok(15), [BranchTokens(tok(5), [1, 2, 3, 4])])]
    roles = [[[O, O, O, D], [O, N, D], [D, O, O]], [[O, O, D, N]]]
    return groups, roles


def expected(hd: PointerHead, rows_of, roles):
    out = []
    for gi, gr in enumerate(roles):
        go = []
        for bi, br in enumerate(gr):
            rows = rows_of(gi, bi)
            decide = rows[[i for i, r in enumerate(br) if r == D][0]]
            opts = np.stack([rows[i] for i, r in enumerate(br) if r == O])
            go.append(oracle.pointer_logits(hd.w_q, hd.b_q, hd.w_k, hd.b_k, decide, opts))
        out.append(go)
    return out


@pytest.mark.parametrize("family", ["gemma3", "gemma4"])
def test_pointer_matches_oracle_on_the_engines_rows_and_the_f32_forward(family):
    rng = np.random.default_rng(5)
    cfg = gemma3_tiny() if family == "gemma3" else gemma4_tiny()
    eng, plain, _, w = build(cfg, 7, g.Q8, g.F16)
    hd = head(rng, 64)
    eng.set_pointer_head(hd)
    groups, roles = request(rng, 40)
    got = eng.evaluate_pointer(groups, roles)
    hidden = eng.evaluate_groups(groups, Want.HIDDEN)
    same = expected(hd, lambda gi, bi: hidden[gi].branches[bi].rows, roles)
    for ga, gb in zip(got, same):
        for a, b in zip(ga, gb):
            assert a.shape == b.shape
            assert np.max(np.abs(a - b)) <= 1e-5 * max(1.0, float(np.max(np.abs(b)))), (a, b)
    ref = [oracle_rows(plain, gr.prefix, gr.branches) for gr in groups]
    f32 = expected(hd, lambda gi, bi: ref[gi][bi], roles)
    worst = 0.0
    for ga, gb in zip(got, f32):
        for a, b in zip(ga, gb):
            pa, pb = oracle.softmax(a), oracle.softmax(b)
            worst = max(worst, float(np.max(np.abs(pa - pb))))
            assert int(np.argmax(pa)) == int(np.argmax(pb))
    assert worst <= 2e-2, worst


def test_pointer_is_the_same_on_a_resident_prefix():
    rng = np.random.default_rng(6)
    eng, _, _, _ = build(gemma3_tiny(), 8, g.Q4, g.F16, oracle_models=False)
    eng.set_pointer_head(head(rng, 64, dp=16))
    groups, roles = request(rng, 40)
    cold = eng.evaluate_pointer(groups[:1], roles[:1])
    warm = eng.evaluate_pointer(groups[:1], roles[:1])
    assert eng.prefix_source() == g.PrefixSource.RESIDENT
    for a, b in zip(cold[0], warm[0]):
        assert np.array_equal(a, b)


def test_pointer_refusals_leave_the_engine_usable():
    rng = np.random.default_rng(9)
    eng, _, _, _ = build(gemma3_tiny(), 9, g.F16, g.F16, oracle_models=False)
    groups, roles = request(rng, 40)
    with pytest.raises(OmgError, match="without a pointer head"):
        eng.evaluate_pointer(groups, roles)
    bad = head(rng, 32)
    with pytest.raises(OmgError, match="input width"):
        eng.set_pointer_head(bad)
    eng.set_pointer_head(head(rng, 64))
    with pytest.raises(OmgError, match="no decide row"):
        eng.evaluate_pointer(groups, [[[O, O, O, O], [O, N, D], [D, O, O]], [[O, O, D, N]]])
    with pytest.raises(OmgError, match="more than one decide row"):
        eng.evaluate_pointer(groups, [[[O, O, D, D], [O, N, D], [D, O, O]], [[O, O, D, N]]])
    with pytest.raises(OmgError, match="roles for"):
        eng.evaluate_pointer(groups, [[[O, O, O, D], [O, D], [D, O, O]], [[O, O, D, N]]])
    ok = eng.evaluate_pointer(groups, roles)
    assert [len(x) for gr in ok for x in gr] == [3, 1, 2, 2]
    eng.set_pointer_head(None)
    with pytest.raises(OmgError, match="without a pointer head"):
        eng.evaluate_pointer(groups, roles)
