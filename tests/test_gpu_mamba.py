"""GPU parity of the Mamba-2 layer: the chunked SSD scan (bf16 MFMA operands,
normwise rel-err 2e-2) against the oracle's sequential recurrence, the full
layer against the reference's golden output, and the fused single-token
state update (fp32, 1e-3) against the oracle's host decode path."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import close, golden

pytestmark = pytest.mark.gpu


def scan_case(T, H, P, N, seed):
    xs = O.rng_normal(seed, T * H * P)
    Bm = O.rng_normal(seed + 1, T * N) / np.float32(np.sqrt(N))
    Cm = O.rng_normal(seed + 2, T * N) / np.float32(np.sqrt(N))
    raw = O.rng_normal(seed + 3, T * H, -2.0, 0.5)
    dt = np.log1p(np.exp(raw.astype(np.float64))).astype(np.float32)
    A = -np.exp(O.rng_uniform(seed + 4, H, np.log(1.0), np.log(16.0)))
    D = np.ones(H, np.float32)
    s0 = O.rng_normal(seed + 5, H * P * N, 0, 0.1)
    return [np.ascontiguousarray(a, np.float32) for a in (xs, Bm, Cm, dt, A, D, s0)]


def gpu_scan(gh, case, T, H, P, N, chunk=256):
    xs, Bm, Cm, dt, A, D, s0 = case
    bufs = [gh.Buf.from_array(a) for a in (xs, Bm, Cm, dt, A, D)]
    st = gh.Buf.from_array(s0)
    y = gh.Buf.zeros(T * H * P, np.float32)
    gh.call("gh_ssd_scan", *[b.p for b in bufs], st.p, y.p, T, H, P, N, chunk)
    return y.numpy(), st.numpy()


def oracle_scan(case, T, H, P, N):
    xs, Bm, Cm, dt, A, D, s0 = case
    st = s0.copy()
    y = np.zeros(T * H * P, np.float32)
    O.oracle().orc_ssd_scan_sequential(O.P(xs), O.P(Bm), O.P(Cm), O.P(dt), O.P(A), O.P(D), O.P(st), O.P(y), T, H, P, N)
    return y, st


@pytest.mark.parametrize("T,H,N,chunk", [(1, 2, 64, 256), (100, 3, 64, 64), (300, 4, 128, 256), (513, 2, 128, 128),
                                         (1000, 3, 64, 128), (2048, 5, 128, 256)])
def test_ssd_scan_small(gh, T, H, N, chunk):
    case = scan_case(T, H, 64, N, 10 + T)
    y, st = gpu_scan(gh, case, T, H, 64, N, chunk)
    ry, rst = oracle_scan(case, T, H, 64, N)
    assert close(y, ry, 2e-2)
    assert close(st, rst, 2e-2)


def test_ssd_scan_c3(gh):
    """benchmark configuration c3 scan at full size: T=4096, 48 heads x 64, d_state 128, chunk 256."""
    T, H, P, N = 4096, 48, 64, 128
    case = scan_case(T, H, P, N, 3)
    y, st = gpu_scan(gh, case, T, H, P, N)
    ry, rst = oracle_scan(case, T, H, P, N)
    assert close(y, ry, 2e-2)
    assert close(st, rst, 2e-2)


def test_ssd_chunk_invariance(gh):
    """The chunk length does not change the result (up to rounding)."""
    T, H, P, N = 512, 2, 64, 64
    case = scan_case(T, H, P, N, 77)
    y64, s64 = gpu_scan(gh, case, T, H, P, N, 64)
    y256, s256 = gpu_scan(gh, case, T, H, P, N, 256)
    assert close(y64, y256, 2e-2) and close(s64, s256, 2e-2)


def test_ssd_known_answers(gh):
    """dt = 0: y = D x and the state is unchanged; A -> 0 (no decay): the state
    is the plain sum of dt B x^T."""
    T, H, P, N = 70, 2, 64, 64
    xs, Bm, Cm, dt, A, D, s0 = scan_case(T, H, P, N, 5)
    y, st = gpu_scan(gh, [xs, Bm, Cm, np.zeros_like(dt), A, D, s0], T, H, P, N)
    expect = xs.reshape(T, H, P) + np.einsum("tn,hpn->thp", Cm.reshape(T, N), s0.reshape(H, P, N))
    assert close(y, expect.ravel(), 2e-2)
    assert np.allclose(st, s0, atol=1e-6)
    z = np.zeros(H * P * N, np.float32)
    y, st = gpu_scan(gh, [xs, Bm, Cm, dt, np.zeros_like(A), D, z], T, H, P, N)
    ref = np.einsum("th,thp,tn->hpn", dt.reshape(T, H), xs.reshape(T, H, P), Bm.reshape(T, N))
    assert close(st, ref.ravel(), 2e-2)


def mamba_args(g, kind):
    names = ["x", "w_in", "conv_w", "conv_b", "dt_bias", "a_log", "D", "norm_w", "w_out"]
    return [g[f"k{kind}_{n}"] for n in names]


@pytest.mark.parametrize("kind", [2, 0])
def test_mamba_forward_golden(gh, kind):
    g = golden("mamba")
    B, T, d, di, conv_dim, nh, dh, ds, k = [int(v) for v in g["shape"]]
    bufs = [gh.Buf.from_array(a) for a in mamba_args(g, kind)]
    st = gh.Buf.from_array(g[f"k{kind}_state_in"])
    out = gh.Buf.zeros(B * T * d, np.float32)
    gh.call("gh_mamba2_forward_half", *[b.p for b in bufs], st.p, out.p, B, T, d, di, conv_dim, nh, dh, ds, k,
            gh.fl(1e-5), kind)
    assert close(out.numpy(), g[f"k{kind}_out"], 2e-2)
    assert close(st.numpy(), g[f"k{kind}_state_out"], 2e-2)


def layer_case(d, di, nh, ds, k, kind, seed):
    conv_dim = di + 2 * ds
    proj = di + conv_dim + nh
    w_in = O.quantize(kind, O.rng_normal(seed, proj * d, 0, 0.02))
    w_out = O.quantize(kind, O.rng_normal(seed + 1, d * di, 0, 0.02))
    conv_w = O.rng_normal(seed + 2, conv_dim * k, 0, 0.3)
    conv_b = O.rng_normal(seed + 3, conv_dim, 0, 0.1)
    dt_bias = np.zeros(nh, np.float32)
    a_log = O.rng_uniform(seed + 4, nh, 0.0, np.log(16.0))
    D = np.ones(nh, np.float32)
    norm_w = np.ones(di, np.float32)
    return [w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out], conv_dim


def test_mamba_forward_c3_vs_oracle(gh):
    """benchmark configuration c3 layer (d 1536, d_inner 3072, 48x64, d_state 128, Q4_K)
    at T=256 against the oracle's sequential layer."""
    d, di, nh, dh, ds, k, T, kind = 1536, 3072, 48, 64, 128, 4, 256, 3
    w, conv_dim = layer_case(d, di, nh, ds, k, kind, 30)
    x = O.rng_normal(3, T * d)
    st0 = np.zeros(nh * dh * ds, np.float32)
    bufs = [gh.Buf.from_array(a) for a in [x] + w]
    st = gh.Buf.from_array(st0)
    out = gh.Buf.zeros(T * d, np.float32)
    gh.call("gh_mamba2_forward_half", *[b.p for b in bufs], st.p, out.p, 1, T, d, di, conv_dim, nh, dh, ds, k,
            gh.fl(1e-5), kind)
    ref = np.zeros(T * d, np.float32)
    rst = st0.copy()
    assert O.oracle().orc_mamba2_forward_q(O.P(x), *[O.P(a) for a in w[:-1]], O.P(w[-1]), O.P(rst), O.P(ref), 1, T,
                                           d, di, conv_dim, nh, dh, ds, k, O.f(1e-5), kind) == 0
    assert close(out.numpy(), ref, 2e-2)
    assert close(st.numpy(), rst, 2e-2)


@pytest.mark.parametrize("shape", ["c1", "c3"])
def test_mamba_step_vs_oracle(gh, shape):
    """The fused single-token update against the host decode path, 12 steps."""
    if shape == "c1":
        d, di, nh, dh, ds, k, kind = 512, 1024, 16, 64, 64, 4, 2
    else:
        d, di, nh, dh, ds, k, kind = 1536, 3072, 48, 64, 128, 4, 3
    w, conv_dim = layer_case(d, di, nh, ds, k, kind, 40)
    bufs = [gh.Buf.from_array(a) for a in w]
    conv = np.zeros(conv_dim * (k - 1), np.float32)
    ssm = O.rng_normal(41, nh * dh * ds, 0, 0.1)
    dconv, dssm = gh.Buf.from_array(conv), gh.Buf.from_array(ssm)
    rconv, rssm = conv.copy(), ssm.copy()
    out = gh.Buf.zeros(d, np.float32)
    for step in range(12):
        x = O.rng_normal(100 + step, d)
        dx = gh.Buf.from_array(x)
        gh.call("gh_mamba2_step_half", dx.p, *[b.p for b in bufs], dconv.p, dssm.p, out.p, d, di, conv_dim, nh, dh,
                ds, k, gh.fl(1e-5), kind)
        ref = np.zeros(d, np.float32)
        assert O.oracle().orc_mamba2_step_q(O.P(x), *[O.P(a) for a in w], O.P(rconv), O.P(rssm), O.P(ref), d, di,
                                            conv_dim, nh, dh, ds, k, O.f(1e-5), kind) == 0
        assert close(out.numpy(), ref, 1e-3), step
    assert close(dssm.numpy(), rssm, 1e-3)
    assert close(dconv.numpy(), rconv, 1e-3)  # the window holds raw in_proj outputs (GEMV rounding)


def test_mamba_prefill_equals_steps(gh):
    """T tokens through the chunked forward == T single-token steps from zero
    state (the window starts at zero in both), c1 shapes."""
    d, di, nh, dh, ds, k, kind, T = 512, 1024, 16, 64, 64, 4, 2, 40
    w, conv_dim = layer_case(d, di, nh, ds, k, kind, 50)
    bufs = [gh.Buf.from_array(a) for a in w]
    x = O.rng_normal(51, T * d)
    dx = gh.Buf.from_array(x)
    st = gh.Buf.zeros(nh * dh * ds, np.float32)
    out = gh.Buf.zeros(T * d, np.float32)
    gh.call("gh_mamba2_forward_half", dx.p, *[b.p for b in bufs], st.p, out.p, 1, T, d, di, conv_dim, nh, dh, ds, k,
            gh.fl(1e-5), kind)
    dconv = gh.Buf.zeros(conv_dim * (k - 1), np.float32)
    dssm = gh.Buf.zeros(nh * dh * ds, np.float32)
    o1 = gh.Buf.zeros(d, np.float32)
    outs = []
    for t in range(T):
        xt = gh.Buf.from_array(np.ascontiguousarray(x[t * d:(t + 1) * d]))
        gh.call("gh_mamba2_step_half", xt.p, *[b.p for b in bufs], dconv.p, dssm.p, o1.p, d, di, conv_dim, nh, dh,
                ds, k, gh.fl(1e-5), kind)
        outs.append(o1.numpy())
    assert close(out.numpy(), np.concatenate(outs), 2e-2)
    assert close(st.numpy(), dssm.numpy(), 2e-2)


def test_mamba_c3_prompt_then_512_steps(gh):
    """benchmark configuration c3 as configured: the Q4_K layer over a 4096-token prompt
    (chunked SSD scan) from a zero state, then 512 single-token state updates
    carried from the state that scan left. Against the oracle's run of the same
    workload (tests/golden/mamba_c3_decode_oracle.npz: orc_mamba2_forward_q then
    orc_mamba2_step_q, inference/generator.cpp:510-616): sampled prompt rows and
    a state sample after the scan (2e-2, bf16 scan operands); step outputs at
    indices 0..511 and the state after the last step (2e-2: the GPU carries its
    own scan state, whose difference decays away over the steps); the final conv
    window (1e-3: raw in_proj rows of the last 3 step tokens)."""
    import cases
    g = golden("mamba_c3_decode_oracle")
    s = cases.C3
    d, di, nh, dh, ds, k, T = s["d"], s["d_inner"], s["heads"], s["d_head"], s["d_state"], s["conv_k"], s["T"]
    w, conv_dim = cases.c3_layer_weights()
    x = cases.c3_prompt()
    bufs = [gh.Buf.from_array(a) for a in w]
    dx = gh.Buf.from_array(x)
    st = gh.Buf.zeros(nh * dh * ds, np.float32)
    out = gh.Buf.zeros(T * d, np.float32)
    gh.call("gh_mamba2_forward_half", dx.p, *[b.p for b in bufs], st.p, out.p, 1, T, d, di, conv_dim, nh, dh, ds, k,
            gh.fl(1e-5), 3)
    rows, sidx = cases.c3_sample_rows(), cases.c3_state_sample()
    assert close(out.numpy().reshape(T, d)[rows], g["prompt_out_rows"], 2e-2)
    assert close(st.numpy()[sidx], g["prompt_state_sample"], 2e-2)
    del dx, out
    conv = gh.Buf.from_array(cases.c3_window(w, x, conv_dim))
    xs = gh.Buf.from_array(cases.c3_step_inputs())
    o = gh.Buf.zeros(d, np.float32)
    got = []
    for i in range(s["steps"]):
        xi = C.c_void_p(xs.ptr + i * d * 4)
        gh.call("gh_mamba2_step_half", xi, *[b.p for b in bufs], conv.p, st.p, o.p, d, di, conv_dim, nh, dh, ds, k,
                gh.fl(1e-5), 3)
        if i in cases.C3_STEP_CHECKS:
            got.append(o.numpy())
    for j, i in enumerate(cases.C3_STEP_CHECKS):
        assert close(got[j], g["step_out"][j], 2e-2), f"step {i}"
    assert close(st.numpy()[sidx], g["final_state_sample"], 2e-2)
    assert close(conv.numpy(), g["final_conv"], 1e-3)
