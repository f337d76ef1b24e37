"""Direct GPU parity of the standalone elementwise entry points of the C ABI
against the CPU oracle (itself pinned bit-exactly to the compiled reference's
ops by tests/golden/elementwise.npz):

  rmsnorm_forward (core/ops.h:134, core/math_cpu.cpp:299-316),
  swiglu_forward (core/ops.h:156, core/math_cpu.cpp:522-529),
  add / add_inplace / scale_inplace / zero / copy (core/ops.h:121-127,
  core/math_cpu.cpp:173-214), embedding_forward_half (core/ops.h:111,
  core/math_cpu.cpp:227-241), convert_f32_to_f16 / f16_to_f32
  (core/ops.h:82-83, core/dtype.h:61-126).

Pure data movement and single-rounding ops are bit-exact; RMSNorm's double
sum of squares is reduced in a different order than the serial CPU loop, so
its statistic may differ in the last bit of the double (tolerance 1e-6
elementwise), and SiLU calls the device expf (tolerance 1e-6 elementwise)."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def elem_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-30))) if a.size else 0.0


def test_rmsnorm_golden_inputs(gh):
    g = golden("elementwise")
    x, w = g["rms_x"], g["rms_w"]
    rows, dim = 5, 96
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    out, rr = gh.Buf.zeros(rows * dim, np.float32), gh.Buf.zeros(rows, np.float32)
    gh.call("gh_rmsnorm_forward", dx.p, dw.p, out.p, rr.p, gh.i64(rows), dim, gh.fl(1e-5))
    assert elem_rel(out.numpy(), g["rms_out"]) <= 1e-6
    assert elem_rel(rr.numpy(), g["rms_rrms"]) <= 1e-6


@pytest.mark.parametrize("rows,dim,with_rrms", [(1, 512, True), (7, 1536, True), (33, 4096, False), (3, 100, True)])
def test_rmsnorm_vs_oracle(gh, rows, dim, with_rrms):
    x = O.rng_normal(500 + rows, rows * dim, 0.3, 2.0)
    w = O.rng_normal(600 + dim, dim, 1.0, 0.2)
    ro = np.zeros(rows * dim, np.float32)
    rr = np.zeros(rows, np.float32)
    O.oracle().orc_rmsnorm_forward(O.P(x), O.P(w), O.P(ro), O.P(rr), C.c_int64(rows), dim, O.f(1e-5))
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    out = gh.Buf.zeros(rows * dim, np.float32)
    drr = gh.Buf.zeros(rows, np.float32) if with_rrms else None
    gh.call("gh_rmsnorm_forward", dx.p, dw.p, out.p, drr.p if drr else None, gh.i64(rows), dim, gh.fl(1e-5))
    assert elem_rel(out.numpy(), ro) <= 1e-6
    if with_rrms:
        assert elem_rel(drr.numpy(), rr) <= 1e-6


def test_rmsnorm_zero_row(gh):
    """An all-zero row: inv = 1/sqrt(eps), output zero (finite statistic)."""
    dim = 256
    x = np.zeros(dim, np.float32)
    w = np.ones(dim, np.float32)
    ro, rr = np.zeros(dim, np.float32), np.zeros(1, np.float32)
    O.oracle().orc_rmsnorm_forward(O.P(x), O.P(w), O.P(ro), O.P(rr), C.c_int64(1), dim, O.f(1e-5))
    dx, dw = gh.Buf.from_array(x), gh.Buf.from_array(w)
    out, drr = gh.Buf.zeros(dim, np.float32), gh.Buf.zeros(1, np.float32)
    gh.call("gh_rmsnorm_forward", dx.p, dw.p, out.p, drr.p, gh.i64(1), dim, gh.fl(1e-5))
    assert np.array_equal(out.numpy(), ro)
    assert elem_rel(drr.numpy(), rr) <= 1e-6


def test_swiglu_golden_inputs(gh):
    g = golden("elementwise")
    dg, du = gh.Buf.from_array(g["sw_g"]), gh.Buf.from_array(g["sw_u"])
    out = gh.Buf.zeros(1000, np.float32)
    gh.call("gh_swiglu_forward", dg.p, du.p, out.p, gh.i64(1000))
    assert elem_rel(out.numpy(), g["sw_out"]) <= 1e-6


@pytest.mark.parametrize("n", [1, 777, 1 << 20])
def test_swiglu_vs_oracle(gh, n):
    gv = O.rng_normal(700 + n % 97, n, 0.0, 4.0)
    gv[: min(n, 4)] = [-100.0, 100.0, 0.0, -0.0][: min(n, 4)]  # saturated and zero gates
    u = O.rng_normal(800 + n % 89, n)
    ro = np.zeros(n, np.float32)
    O.oracle().orc_swiglu_forward(O.P(gv), O.P(u), O.P(ro), C.c_int64(n))
    dg, du = gh.Buf.from_array(gv), gh.Buf.from_array(u)
    out = gh.Buf.zeros(n, np.float32)
    gh.call("gh_swiglu_forward", dg.p, du.p, out.p, gh.i64(n))
    got = out.numpy()
    assert elem_rel(got, ro) <= 1e-6
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("n", [1, 1000, 3 << 18])
def test_add_scale_zero_copy(gh, n):
    """add (core/math_cpu.cpp:173-178), add_inplace, scale_inplace, zero and
    copy: one IEEE operation per element, so bit-exact against numpy fp32."""
    a = O.rng_normal(900, n)
    b = O.rng_normal(901, n)
    da, db = gh.Buf.from_array(a), gh.Buf.from_array(b)
    out = gh.Buf.zeros(n, np.float32)
    gh.call("gh_add", da.p, db.p, out.p, gh.i64(n))
    assert np.array_equal(bits(out.numpy()), bits(a + b))
    gh.call("gh_add_inplace", da.p, db.p, gh.i64(n))
    assert np.array_equal(bits(da.numpy()), bits(a + b))
    gh.call("gh_scale_inplace", da.p, gh.fl(0.3), gh.i64(n))
    assert np.array_equal(bits(da.numpy()), bits((a + b) * np.float32(0.3)))
    gh.call("gh_copy", out.p, db.p, gh.i64(n))
    assert np.array_equal(bits(out.numpy()), bits(b))
    gh.call("gh_zero", out.p, gh.i64(n))
    assert not np.any(out.numpy())


def test_elementwise_empty_and_null(gh):
    """n = 0 is a no-op; a null pointer is rejected with the reference's message."""
    lib = gh.load()
    gh.call("gh_zero", None, gh.i64(0))
    gh.call("gh_add", None, None, None, gh.i64(0))
    assert lib.gh_zero(None, gh.i64(4)) == 1
    assert b"ops::zero on null pointer" in lib.gh_last_error()
    assert lib.gh_copy(None, None, gh.i64(4)) == 1


def test_embedding_golden_inputs(gh):
    g = golden("elementwise")
    ids, tab = g["emb_ids"], g["emb_table"]
    dids, dtab = gh.Buf.from_array(ids), gh.Buf.from_array(tab)
    out = gh.Buf.zeros(240, np.float32)
    gh.call("gh_embedding_forward_half", dids.p, dtab.p, out.p, gh.i64(6), 40, 100)
    assert np.array_equal(bits(out.numpy()), bits(g["emb_out"]))


def test_embedding_vs_oracle_out_of_range(gh):
    """c1 table (4096 x 512 fp16); ids include -1, V and a huge value: those
    rows are zero (core/math_cpu.cpp:233-236)."""
    V, dim = 4096, 512
    tab = O.f32_to_f16(O.rng_normal(1000, V * dim, 0, 0.02))
    ids = np.concatenate([O.rng_below(1001, 60, V), np.array([-1, V, 1 << 30, 0], np.int32)]).astype(np.int32)
    ro = np.zeros(len(ids) * dim, np.float32)
    O.oracle().orc_embedding_forward_half(O.P(ids), O.P(tab), O.P(ro), C.c_int64(len(ids)), dim, V)
    dids, dtab = gh.Buf.from_array(ids), gh.Buf.from_array(tab)
    out = gh.Buf.zeros(len(ids) * dim, np.float32)
    gh.call("gh_embedding_forward_half", dids.p, dtab.p, out.p, gh.i64(len(ids)), dim, V)
    got = out.numpy()
    assert np.array_equal(bits(got), bits(ro))
    assert not np.any(got.reshape(len(ids), dim)[60:63])


def test_convert_f16_round_trip(gh):
    """f32 -> f16 (RNE, core/dtype.h:61-87) and back, bit-exact against the
    golden-pinned oracle conversions, including specials and subnormals."""
    x = np.concatenate([O.rng_normal(1100, 4096, 0, 30.0),
                        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 1e-8, -6e-8, 5.96e-8, 2.0 ** -25,
                                  3.0 * 2.0 ** -26], np.float32)]).astype(np.float32)
    ref16 = O.f32_to_f16(x)
    dx = gh.Buf.from_array(x)
    h = gh.Buf.zeros(x.size, np.uint16)
    gh.call("gh_convert_f32_to_f16", dx.p, h.p, gh.i64(x.size))
    got16 = h.numpy()
    assert np.array_equal(got16, ref16)
    back = gh.Buf.zeros(x.size, np.float32)
    gh.call("gh_convert_f16_to_f32", h.p, back.p, gh.i64(x.size))
    assert np.array_equal(bits(back.numpy()), bits(O.f16_to_f32(ref16)))


def test_argmax_token_host(gh):
    """argmax_token to a host int against the oracle (golden-pinned ties)."""
    g = golden("elementwise")
    out = C.c_int32()
    for x in (g["am_x"], g["am_ties"]):
        d = gh.Buf.from_array(x)
        gh.call("gh_argmax_token", d.p, x.size, C.byref(out))
        assert out.value == O.oracle().orc_argmax_token(O.P(x), x.size)
