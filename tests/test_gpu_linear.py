"""GPU parity of the quantized linear path against the CPU oracle:
bit-exact block decode, GEMV within 1e-3 (fp32 accumulate), MFMA GEMM
within 2e-2 (bf16 operands). Normwise relative error max|d|/max|ref|."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import close

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
GEMM_TOL = 2e-2


def _w(kind, N, K, seed=2):
    return O.quantize(kind, O.rng_normal(seed, N * K, 0, 0.02))


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_dequant_bit_exact(gh, kind):
    n = 256 * 97
    x = O.rng_normal(5, n, 0, 1)
    x[300] = np.nan  # a zeroed block
    q = O.quantize(kind, x)
    dq = gh.Buf.from_array(q)
    out = gh.Buf.zeros(n, np.float32)
    gh.call("gh_dequantize_f32", dq.p, kind, gh.i64(n), out.p)
    got = out.numpy()
    ref = O.dequantize(kind, q, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    p = C.c_void_p()
    gh.call("gh_quant_materialize", dq.p, kind, gh.i64(n), 3, C.byref(p))
    h = np.empty(n, np.uint16)
    gh.call("gh_device_copy", h.ctypes.data_as(C.c_void_p), 0, p, 1, C.c_size_t(n * 2))
    assert np.array_equal(h, O.materialize(kind, q, n))


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("M,K,N", [(1, 256, 24), (3, 512, 2192), (8, 1024, 512), (2, 256, 4608), (1, 4096, 1000)])
def test_gemv_parity(gh, kind, M, K, N):
    w = _w(kind, N, K)
    x = O.rng_normal(7, M * K)
    y = gh.Buf.zeros(M * N, np.float32)
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
    ref = O.linear_q(x, w, M, K, N, kind)
    assert close(y.numpy().reshape(M, N), ref, GEMV_TOL)


@pytest.mark.parametrize("kind", [2, 3])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 14336), (8, 4096, 14336), (1, 14336, 4096)])
def test_gemv_c2_full(gh, kind, M, K, N):
    """benchmark configuration c2 at full size."""
    w = _w(kind, N, K)
    x = O.rng_normal(8, M * K)
    y = gh.Buf.zeros(M * N, np.float32)
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
    ref = O.linear_q(x, w, M, K, N, kind)
    assert close(y.numpy().reshape(M, N), ref, GEMV_TOL)


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("M,K,N", [(9, 256, 40), (128, 512, 256), (300, 1024, 200), (33, 1024, 130), (256, 512, 2192), (64, 256, 70),
                                   (250, 1024, 1100), (200, 256, 1100), (128, 512, 2320)])
def test_gemm_parity(gh, kind, M, K, N):
    w = _w(kind, N, K)
    x = O.rng_normal(9, M * K)
    y = gh.Buf.zeros(M * N, np.float32)
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
    ref = O.linear_q(x, w, M, K, N, kind)
    assert close(y.numpy().reshape(M, N), ref, GEMM_TOL)


@pytest.mark.parametrize("kind", [2, 3])
def test_gemm_c2_full_rows_match_gemv(gh, kind):
    """M=2048 prefill GEMM at full size: sampled rows against the (pinned)
    GEMV of the same rows, and a few rows against the oracle directly."""
    M, K, N = 2048, 4096, 14336
    w = _w(kind, N, K)
    x = O.rng_normal(10, M * K)
    dw, dx = gh.Buf.from_array(w), gh.Buf.from_array(x)
    y = gh.Buf.zeros(M * N, np.float32)
    gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
    Y = y.numpy().reshape(M, N)
    rows = np.array([0, 1, 127, 128, 1000, 2046, 2047, 513], np.int64)
    xs = np.ascontiguousarray(x.reshape(M, K)[rows])
    ys = gh.Buf.zeros(8 * N, np.float32)
    dxs = gh.Buf.from_array(xs)
    gh.call("gh_linear_forward_q4", dxs.p, dw.p, ys.p, 8, K, N, kind)
    assert close(Y[rows], ys.numpy().reshape(8, N), GEMM_TOL)
    ref = O.linear_q(np.ascontiguousarray(xs[:2]), w, 2, K, N, kind)
    assert close(Y[rows[:2]], ref, GEMM_TOL)


def test_fp16_and_f32_linear(gh):
    M, K, N = 2, 512, 4096
    wf = O.rng_normal(11, N * K, 0, 0.02)
    wh = O.f32_to_f16(wf)
    x = O.rng_normal(12, M * K)
    y = gh.Buf.zeros(M * N, np.float32)
    dx, dwh, dwf = gh.Buf.from_array(x), gh.Buf.from_array(wh), gh.Buf.from_array(wf)
    gh.call("gh_linear_forward_fp16", dx.p, dwh.p, y.p, M, K, N)
    ref = np.empty(M * N, np.float32)
    O.oracle().orc_linear_forward_fp16(O.P(x), O.P(wh), O.P(ref), M, K, N)
    assert close(y.numpy(), ref, GEMV_TOL)
    gh.call("gh_linear_forward_f32", dx.p, dwf.p, y.p, M, K, N)
    O.oracle().orc_linear_forward_f32(O.P(x), O.P(wf), O.P(ref), M, K, N)
    assert close(y.numpy(), ref, GEMV_TOL)
    Mg = 64
    xg = O.rng_normal(13, Mg * K)
    yg = gh.Buf.zeros(Mg * N, np.float32)
    dxg = gh.Buf.from_array(xg)
    gh.call("gh_linear_forward_fp16", dxg.p, dwh.p, yg.p, Mg, K, N)
    refg = np.empty(Mg * N, np.float32)
    O.oracle().orc_linear_forward_fp16(O.P(xg), O.P(wh), O.P(refg), Mg, K, N)
    assert close(yg.numpy(), refg, GEMM_TOL)


@pytest.mark.parametrize("kind", [2, 3])
@pytest.mark.parametrize("K,N", [(256, 37), (3072, 530), (16384, 300)])
def test_small_m_gemv_every_m(gh, kind, K, N):
    """Every token count of the small-M path (1..8) at one, many and the
    maximum number of super-blocks (the last case runs in token groups),
    ragged N (tiles of 16 rows)."""
    w = _w(kind, N, K, seed=21)
    dw = gh.Buf.from_array(w)
    for M in range(1, 9):
        x = O.rng_normal(22 + M, M * K)
        dx = gh.Buf.from_array(x)
        y = gh.Buf.zeros(M * N, np.float32)
        gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
        ref = O.linear_q(x, w, M, K, N, kind)
        assert close(y.numpy().reshape(M, N), ref, GEMV_TOL), f"M={M}"


@pytest.mark.parametrize("kind", [2, 3])
def test_small_m_gemv_activation_range(gh, kind):
    """Activations spanning 1e-4..1e3 in magnitude per token: the split of
    each activation into two fp16 parts keeps the fp32-level accuracy."""
    M, K, N = 3, 2048, 64
    w = _w(kind, N, K, seed=31)
    x = O.rng_normal(32, M * K).reshape(M, K)
    x[0] *= 1e3
    x[1] *= 1e-4
    x[2, ::7] *= 50.0
    x = np.ascontiguousarray(x.reshape(-1), np.float32)
    dw, dx = gh.Buf.from_array(w), gh.Buf.from_array(x)
    y = gh.Buf.zeros(M * N, np.float32)
    gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind)
    ref = O.linear_q(x, w, M, K, N, kind).reshape(M, N)
    got = y.numpy().reshape(M, N)
    for t in range(M):
        assert close(got[t], ref[t], GEMV_TOL), f"token {t}"
