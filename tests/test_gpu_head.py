"""GPU parity of the fused decode tail (final rmsnorm + tied fp16 lm head +
greedy id, gh_lm_head_greedy_dev) and of gh_argmax_token against the CPU
oracle: logits within 1e-3 (fp32 accumulate), ids exact under the reference's
rule (first finite maximum, lowest index on ties, serial fallback when nothing
is finite), including ties, +-0 and non-finite logits."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import close

pytestmark = pytest.mark.gpu

TOL = 1e-3
EPS = 1e-5


def _head(gh, x, nw, tab16, d, V):
    dx, dn, dt = gh.Buf.from_array(x), gh.Buf.from_array(nw), gh.Buf.from_array(tab16)
    lg = gh.Buf.zeros(V, np.float32)
    tok = gh.Buf.zeros(1, np.int32)
    gh.call("gh_lm_head_greedy_dev", dx.p, dn.p, gh.fl(EPS), dt.p, lg.p, d, V, tok.p)
    gh.sync()
    return lg.numpy(), int(tok.numpy(np.int32)[0])


def _oracle_logits(x, nw, tab16, d, V):
    xn = np.zeros(d, np.float32)
    O.oracle().orc_rmsnorm_forward(O.P(x), O.P(nw), O.P(xn), None, C.c_int64(1), d, C.c_float(EPS))
    y = np.zeros(V, np.float32)
    O.oracle().orc_linear_forward_fp16(O.P(xn), O.P(tab16), O.P(y), 1, d, V)
    return y


def _argmax(l):
    l = np.ascontiguousarray(l, np.float32)
    return int(O.oracle().orc_argmax_token(O.P(l), len(l)))


@pytest.mark.parametrize("d,V", [(512, 4096), (256, 1000), (1536, 4099), (2048, 517), (8, 3)])
def test_head_greedy_parity(gh, d, V):
    x = O.rng_normal(60, d)
    nw = O.rng_normal(61, d, 1.0, 0.1)
    tab = O.f32_to_f16(O.rng_normal(62, V * d, 0, 0.02))
    lg, tok = _head(gh, x, nw, tab, d, V)
    ref = _oracle_logits(x, nw, tab, d, V)
    assert close(lg, ref, TOL)
    assert tok == _argmax(lg)
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 1e-3:
        assert tok == _argmax(ref)


def test_head_greedy_ties_and_zero(gh):
    d, V = 512, 4096
    x = O.rng_normal(63, d)
    nw = np.ones(d, np.float32)
    tab = O.f32_to_f16(O.rng_normal(64, V * d, 0, 0.02)).reshape(V, d)
    # three identical rows aligned with x: the same (largest) logit, lowest index wins
    big = O.f32_to_f16(np.sign(x).astype(np.float32) * 0.5)
    for r in (3001, 300, 2047):
        tab[r] = big
    lg, tok = _head(gh, x, nw, tab.ravel(), d, V)
    assert lg[300] == lg[3001] == lg[2047] == lg.max()
    assert tok == 300
    # x = 0: every logit is +-0, so row 0 wins
    lg, tok = _head(gh, np.zeros(d, np.float32), nw, tab.ravel(), d, V)
    assert np.all(lg == 0) and tok == 0


def _inf_rows(V, d, kinds):
    """Rows giving logit +inf ('p'), -inf ('n'), NaN ('q') or a finite value ('f') for x > 0."""
    tab = np.full((V, d), O.f32_to_f16(np.array([0.01], np.float32))[0], np.uint16)
    pinf, ninf = np.uint16(0x7C00), np.uint16(0xFC00)
    for i, k in enumerate(kinds):
        if k == "p":
            tab[i, 5] = pinf
        elif k == "n":
            tab[i, 5] = ninf
        elif k == "q":
            tab[i, 5], tab[i, 6] = pinf, ninf
    return tab.ravel()


@pytest.mark.parametrize("kinds,expect", [
    ("nqqpqpq", 3),      # nothing finite, l[0] = -inf: the first +inf
    ("qppppnn", 0),      # nothing finite, l[0] = NaN: 0
    ("pnnpqnq", 0),      # nothing finite, l[0] = +inf: 0
    ("nnqnnqn", 0),      # no +inf at all: 0
    ("pqfnpfq", 2),      # a finite value beats +inf (first finite maximum)
])
def test_head_greedy_non_finite(gh, kinds, expect):
    d = 64
    V = len(kinds)
    x = np.abs(O.rng_normal(65, d)) + 0.1
    nw = np.ones(d, np.float32)
    lg, tok = _head(gh, x, nw, _inf_rows(V, d, kinds), d, V)
    assert _argmax(lg) == expect
    assert tok == expect


def test_argmax_token_rule(gh):
    cases = [
        O.rng_normal(66, 4096),
        np.array([1.0, 3.0, 3.0, -2.0, 3.0], np.float32),
        np.array([-0.0, 0.0, -0.0], np.float32),
        np.array([np.nan, 1.0, np.inf, 1.0], np.float32),
        np.array([-np.inf, np.nan, np.inf, np.inf], np.float32),
        np.array([np.nan, np.inf], np.float32),
    ]
    for l in cases:
        out = np.zeros(1, np.int32)
        dl = gh.Buf.from_array(l)
        gh.call("gh_argmax_token", dl.p, len(l), out.ctypes.data_as(C.c_void_p))
        assert int(out[0]) == _argmax(l), l
