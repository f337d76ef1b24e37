"""GPU parity of the sampling-side decode ops against the CPU oracle (and the
reference's golden vectors): gh_topk_select ids and values bit-exact
(value descending, lower index first on ties), gh_apply_rep_penalties
bit-exact, including repeated / out-of-range history ids and the limits."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def gpu_topk(gh, lg, K):
    dl = gh.Buf.from_array(np.ascontiguousarray(lg, np.float32))
    dv, di = gh.Buf.zeros(K, np.float32), gh.Buf.zeros(K, np.int32)
    gh.call("gh_topk_select", dl.p, len(lg), K, dv.p, di.p)
    return dv.numpy(), di.numpy(np.int32)


def orc_topk(lg, K):
    vals, ids = np.zeros(K, np.float32), np.zeros(K, np.int32)
    lg = np.ascontiguousarray(lg, np.float32)
    assert O.oracle().orc_topk_select(O.P(lg), len(lg), K, O.P(vals), O.P(ids)) == 0
    return vals, ids


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_topk_golden(gh, tag):
    g = golden("sampling")
    v, i = gpu_topk(gh, g[f"tk{tag}_x"], int(g[f"tk{tag}_k"]))
    assert np.array_equal(i, g[f"tk{tag}_ids"])
    assert np.array_equal(bits(v), bits(g[f"tk{tag}_vals"]))


@pytest.mark.parametrize("V,K", [(1, 1), (63, 7), (4096, 40), (4097, 128), (100352, 50), (262144, 128),
                                 (262144, 1), (131071, 100)])
def test_topk_parity(gh, V, K):
    lg = O.rng_normal(80 + K, V, 0, 3)
    lg[::7] = np.round(lg[::7])  # many exact ties
    v, i = gpu_topk(gh, lg, K)
    rv, ri = orc_topk(lg, K)
    assert np.array_equal(i, ri)
    assert np.array_equal(bits(v), bits(rv))


def test_topk_infinities_and_signed_zero(gh):
    lg = np.zeros(5000, np.float32)
    lg[[10, 4000]] = -0.0
    lg[[20, 30]] = np.inf
    lg[[40, 4500]] = -np.inf
    v, i = gpu_topk(gh, lg, 128)
    rv, ri = orc_topk(lg, 128)
    assert np.array_equal(i, ri) and np.array_equal(bits(v), bits(rv))
    assert list(i[:3]) == [20, 30, 0]  # +inf first, then the zeros (+0 and -0 equal) by index
    v, i = gpu_topk(gh, lg, 1)
    assert i[0] == 20


def test_topk_nan_ranks_last(gh):
    lg = O.rng_normal(90, 100)
    lg[[5, 17]] = np.nan
    v, i = gpu_topk(gh, lg, 100)
    assert list(i[-2:]) == [5, 17]
    fin = np.delete(lg, [5, 17])
    _, ri = orc_topk(fin, 98)
    ids = np.delete(np.arange(100), [5, 17])
    assert np.array_equal(i[:98], ids[ri])


def test_topk_limits(gh):
    lg = gh.Buf.from_array(np.zeros(300000, np.float32))
    dv, di = gh.Buf.zeros(200, np.float32), gh.Buf.zeros(200, np.int32)
    for V, K, msg in [(1000, 0, "K out of range"), (1000, 129, "K out of range"), (10, 20, "vocab too small"),
                      (262145, 5, "exceeds maximum")]:
        with pytest.raises(gh.GHError, match=msg):
            gh.call("gh_topk_select", lg.p, V, K, dv.p, di.p)


def gpu_pen(gh, lg, hist, rep, freq, pres):
    dl = gh.Buf.from_array(np.ascontiguousarray(lg, np.float32))
    h = np.ascontiguousarray(hist, np.int32)
    gh.call("gh_apply_rep_penalties", dl.p, len(lg), h.ctypes.data_as(C.c_void_p), len(h), gh.fl(rep), gh.fl(freq),
            gh.fl(pres))
    return dl.numpy()


def orc_pen(lg, hist, rep, freq, pres):
    o = np.ascontiguousarray(lg, np.float32).copy()
    h = np.ascontiguousarray(hist, np.int32)
    O.oracle().orc_apply_rep_penalties(O.P(o), len(o), O.P(h), len(h), O.f(rep), O.f(freq), O.f(pres))
    return o


@pytest.mark.parametrize("tag", ["a", "b", "c", "d", "e"])
def test_penalties_golden(gh, tag):
    g = golden("sampling")
    rep, freq, pres = [float(v) for v in g[f"rp{tag}_p"]]
    o = gpu_pen(gh, g[f"rp{tag}_x"], g["rp_hist"], rep, freq, pres)
    assert np.array_equal(bits(o), bits(g[f"rp{tag}_out"]))


@pytest.mark.parametrize("V,n", [(4096, 2048), (100352, 2048), (50000, 200000), (7, 1)])
def test_penalties_parity_and_reuse(gh, V, n):
    hist = O.rng_below(91, n, V + 10) - 5  # some ids out of range on both sides
    lg = O.rng_normal(92, V, 0, 2)
    for rep, freq, pres in [(1.2, 0.1, 0.3), (0.8, 0.0, 0.0), (1.0, 0.5, 0.0)]:
        assert np.array_equal(bits(gpu_pen(gh, lg, hist, rep, freq, pres)), bits(orc_pen(lg, hist, rep, freq, pres)))
    # the count table is left clean: a second history sees only its own counts
    h2 = np.array([3, 3], np.int32)
    assert np.array_equal(bits(gpu_pen(gh, lg, h2, 1.0, 1.0, 0.0)), bits(orc_pen(lg, h2, 1.0, 1.0, 0.0)))
