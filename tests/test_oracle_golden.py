"""CPU tests: the oracle against the reference's golden fixtures (written by
the compiled reference CPU path, tests/golden/make_golden.py) and against
closed forms / invariants where the reference has nothing (Q4_K)."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden, relerr

P = O.P


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_formats():
    g = golden("formats")
    assert np.array_equal(O.f32_to_f16(g["x"]), g["f16"])
    assert np.array_equal(O.f32_to_bf16(g["x"]), g["bf16"])
    allh = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(bits(O.f16_to_f32(allh)), bits(g["f16_all_to_f32"]))


def test_fp16_closed_forms():
    # RNE at the half-way points and the subnormal boundary (core/dtype.h:61-87)
    x = np.array([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2 ** -24, 2 ** -25, 2 ** -25 * 3, 65520.0, 65519.0],
                 np.float32)
    assert O.f32_to_f16(x).tolist() == [0x3C00, 0x3C02, 0x0001, 0x0000, 0x0002, 0x7C00, 0x7BFF]


def test_rng_streams():
    g = golden("rng")
    for seed in (0, 1, 2, 12345):
        assert np.array_equal(bits(O.rng_normal(seed, 257)), bits(g[f"normal_{seed}"]))
        assert np.array_equal(bits(O.rng_uniform(seed, 257, -2.0, 3.0)), bits(g[f"uniform_{seed}"]))
        assert np.array_equal(O.rng_below(seed, 257, 4096), g[f"below_{seed}"])


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_codec_golden(kind):
    g = golden("codec")
    x = g["x"]
    q = O.quantize(kind, x)
    assert np.array_equal(q, g[f"q{kind}"])
    assert np.array_equal(bits(O.dequantize(kind, q, x.size)), bits(g[f"deq{kind}"]))
    assert np.array_equal(O.materialize(kind, q, x.size), g[f"mat{kind}"])


def test_q8_tail_golden():
    g = golden("codec")
    assert np.array_equal(O.quantize(2, g["x_tail"]), g["q2_tail"])


def test_q8_roundtrip_bound():
    x = O.rng_normal(3, 32 * 500, 0, 1)
    q = O.quantize(2, x)
    d = O.dequantize(2, q, x.size)
    scale = O.f16_to_f32(q.reshape(-1, 34)[:, :2].copy().view(np.uint16).ravel())
    err = np.abs(d - x).reshape(-1, 32).max(1)
    # |q*s16 - x| <= s/2 (rounding of q) + 127 |s16 - s| (fp16 rounding of the scale)
    assert np.all(err <= scale * (0.5 + 127 * 2.0 ** -11) * (1 + 1e-6) + 1e-9)
    assert np.mean(np.abs(d - x)) < np.mean(scale) * 0.3  # ~ s/4 for uniform rounding


def _q4k_block(d, dmin, sc, m, q):
    """Hand-built GGML block_q4_K (f16 d, f16 dmin, 12 scale bytes, 128 nibble bytes)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(O.f32_to_f16(np.array([d], np.float32)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(O.f32_to_f16(np.array([dmin], np.float32)).tobytes(), np.uint8)
    S = b[4:16]
    for j in range(4):
        S[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        S[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
        S[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    for s in range(8):
        for l in range(32):
            b[16 + 32 * (s // 2) + l] |= (q[s][l] << 4) if s % 2 else q[s][l]
    return b


def test_q4k_closed_form():
    """Hand-built blocks decode to (d*sc)*q - (dmin*m) with the GGML nibble order
    (a dropped high scale bit or a swapped nibble half fails here)."""
    sc = [1, 63, 17, 32, 5, 48, 33, 62]
    m = [0, 7, 63, 16, 40, 1, 31, 50]
    q = [[(3 * s + l) % 16 for l in range(32)] for s in range(8)]
    d, dmin = 0.5, 0.25
    b = _q4k_block(d, dmin, sc, m, q)
    got = O.dequantize(3, b, 256).reshape(8, 32)
    exp = np.array([[np.float32(d * sc[s]) * q[s][l] - np.float32(dmin * m[s]) for l in range(32)]
                    for s in range(8)], np.float32)
    assert np.array_equal(got, exp)


def test_q4k_roundtrip_bound():
    x = O.rng_normal(4, 256 * 300, 0, 0.02)
    qb = O.quantize(3, x)
    y = O.dequantize(3, qb, x.size)
    blk = qb.reshape(-1, 144)
    d = O.f16_to_f32(blk[:, 0:2].copy().view(np.uint16).ravel())
    dmin = O.f16_to_f32(blk[:, 2:4].copy().view(np.uint16).ravel())
    err = np.abs(y - x).reshape(-1, 256).max(1)
    # one step of the sub-block scale (<= 63*d/63... bounded by 1.5 d*sc) plus the min rounding
    bound = 63 * d / 2 + dmin / 2 + 1.5 * (np.abs(x).reshape(-1, 256).max(1) / 15 / 63 * 2)
    assert np.all(err <= bound + 1e-6)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < 0.08


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_linear_golden(kind):
    g = golden("linear")
    M, K, N = int(g["M"]), int(g["K"]), int(g["N"])
    y = O.linear_q(g["x"], g[f"w{kind}"], M, K, N, kind)
    assert np.array_equal(bits(y.ravel()), bits(g[f"y{kind}"]))


def test_linear_f16_f32_golden():
    g = golden("linear")
    M, K, N = int(g["M"]), int(g["K"]), int(g["N"])
    y = np.zeros(M * N, np.float32)
    O.oracle().orc_linear_forward_fp16(P(g["x"]), P(g["w_f16"]), P(y), M, K, N)
    assert np.array_equal(bits(y), bits(g["y_f16"]))
    O.oracle().orc_linear_forward_f32(P(g["x"]), P(g["w_f32"]), P(y), M, K, N)
    assert np.array_equal(bits(y), bits(g["y_f32"]))


def test_linear_brute_force_fp64():
    """Tiny shape: the oracle equals an fp64 sum over fp16-rounded dequantised weights."""
    M, K, N = 2, 64, 5
    x = O.rng_normal(5, M * K)
    for kind in (0, 2):
        wq = O.quantize(kind, O.rng_normal(6, N * K, 0, 0.05))
        wd = O.f16_to_f32(O.materialize(kind, wq, N * K)).astype(np.float64).reshape(N, K)
        ref = x.astype(np.float64).reshape(M, K) @ wd.T
        assert np.max(np.abs(O.linear_q(x, wq, M, K, N, kind) - ref)) < 1e-5


def test_elementwise_golden():
    g = golden("elementwise")
    o = np.zeros_like(g["rms_x"])
    rr = np.zeros(5, np.float32)
    O.oracle().orc_rmsnorm_forward(P(g["rms_x"]), P(g["rms_w"]), P(o), P(rr), C.c_int64(5), 96, O.f(1e-5))
    assert np.array_equal(bits(o), bits(g["rms_out"])) and np.array_equal(bits(rr), bits(g["rms_rrms"]))
    s = np.zeros_like(g["sw_g"])
    O.oracle().orc_swiglu_forward(P(g["sw_g"]), P(g["sw_u"]), P(s), C.c_int64(1000))
    assert np.array_equal(bits(s), bits(g["sw_out"]))
    sm = g["sm_x"].copy()
    O.oracle().orc_softmax_row(P(sm), 64)
    assert np.array_equal(bits(sm), bits(g["sm_out"]))
    assert O.oracle().orc_argmax_token(P(g["am_x"]), 4096) == int(g["am_out"])
    assert O.oracle().orc_argmax_token(P(g["am_ties"]), 50) == int(g["am_ties_out"]) == 7
    e = np.zeros(240, np.float32)
    O.oracle().orc_embedding_forward_half(P(g["emb_ids"]), P(g["emb_table"]), P(e), C.c_int64(6), 40, 100)
    assert np.array_equal(bits(e), bits(g["emb_out"]))


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_attention_prefill_golden(tag):
    g = golden("attention")
    T, H, KV, hd, win = [int(v) for v in g[f"pf{tag}_shape"]]
    o = np.zeros_like(g[f"pf{tag}_q"])
    O.oracle().orc_attention_forward_ex(P(g[f"pf{tag}_q"]), P(g[f"pf{tag}_k"]), P(g[f"pf{tag}_v"]), P(o), 1, T, H, KV,
                                        hd, O.f(float(g[f"pf{tag}_scale"])), win)
    assert np.array_equal(bits(o), bits(g[f"pf{tag}_out"]))


@pytest.mark.parametrize("tag", ["r0", "r1", "r2", "r3", "r4"])
def test_attention_decode_golden(tag):
    g = golden("attention")
    H, KV, hd, rs, pin, cl, cm, win = [int(v) for v in g[f"{tag}_shape"]]
    o = np.zeros(H * hd, np.float32)
    assert O.oracle().orc_attention_decode_ring_fp16(P(g[f"{tag}_q"]), P(g[f"{tag}_k"]), P(g[f"{tag}_v"]), P(o), H, KV,
                                                     hd, rs, pin, cl, cm, O.f(float(g[f"{tag}_scale"])), win) == 0
    assert np.array_equal(bits(o), bits(g[f"{tag}_out"]))


def test_prefill_row_equals_decode():
    """Row t of the prefill equals ring decode with cur_len = t+1 (fp16-exact K/V)."""
    T, H, KV, hd = 12, 4, 2, 32
    q = O.rng_normal(1, T * H * hd)
    kh = O.f32_to_f16(O.rng_normal(2, T * KV * hd))
    vh = O.f32_to_f16(O.rng_normal(3, T * KV * hd))
    k, v = O.f16_to_f32(kh), O.f16_to_f32(vh)
    out = np.zeros_like(q)
    O.oracle().orc_attention_forward_ex(P(q), P(k), P(v), P(out), 1, T, H, KV, hd, O.f(0.2), 0)
    for t in range(T):
        o = np.zeros(H * hd, np.float32)
        O.oracle().orc_attention_decode_ring_fp16(P(np.ascontiguousarray(q[t * H * hd:(t + 1) * H * hd])), P(kh),
                                                  P(vh), P(o), H, KV, hd, 0, 0, t + 1, T, O.f(0.2), 0)
        assert relerr(out[t * H * hd:(t + 1) * H * hd], o) < 1e-5


@pytest.mark.parametrize("kind", [2, 0])
def test_mamba_forward_golden(kind):
    g = golden("mamba")
    B, T, d, di, conv_dim, nh, dh, ds, k = [int(v) for v in g["shape"]]
    names = ["x", "w_in", "conv_w", "conv_b", "dt_bias", "a_log", "D", "norm_w", "w_out"]
    st = g[f"k{kind}_state_in"].copy()
    out = np.zeros(B * T * d, np.float32)
    assert O.oracle().orc_mamba2_forward_q(*[P(g[f"k{kind}_{n}"]) for n in names], P(st), P(out), B, T, d, di,
                                           conv_dim, nh, dh, ds, k, O.f(1e-5), kind) == 0
    assert np.array_equal(bits(out), bits(g[f"k{kind}_out"]))
    assert np.array_equal(bits(st), bits(g[f"k{kind}_state_out"]))


def test_mamba_steps_equal_forward():
    """T single-token steps from a zero conv window == one forward over T tokens
    (the oracle's step restates the generator's host path)."""
    g = golden("mamba")
    B, T, d, di, conv_dim, nh, dh, ds, k = [int(v) for v in g["shape"]]
    kind = 2
    names = ["w_in", "conv_w", "conv_b", "dt_bias", "a_log", "D", "norm_w", "w_out"]
    x = g[f"k{kind}_x"]
    st = g[f"k{kind}_state_in"].copy()
    conv = np.zeros(conv_dim * (k - 1), np.float32)
    outs = []
    for t in range(T):
        o = np.zeros(d, np.float32)
        O.oracle().orc_mamba2_step_q(P(np.ascontiguousarray(x[t * d:(t + 1) * d])), *[P(g[f"k{kind}_{n}"]) for n in names],
                                     P(conv), P(st), P(o), d, di, conv_dim, nh, dh, ds, k, O.f(1e-5), kind)
        outs.append(o)
    assert relerr(np.concatenate(outs), g[f"k{kind}_out"]) < 1e-5
    assert relerr(st, g[f"k{kind}_state_out"]) < 1e-5


def test_ssd_sequential_special_cases():
    T, H, Pd, N = 9, 2, 4, 3
    xs = O.rng_normal(1, T * H * Pd)
    Bm = O.rng_normal(2, T * N)
    Cm = O.rng_normal(3, T * N)
    D = np.array([0.5, 2.0], np.float32)
    # dt = 0: y = D x, state untouched
    st = O.rng_normal(4, H * Pd * N)
    st0 = st.copy()
    y = np.zeros(T * H * Pd, np.float32)
    O.oracle().orc_ssd_scan_sequential(P(xs), P(Bm), P(Cm), P(np.zeros(T * H, np.float32)), P(np.array([-1.0, -3.0], np.float32)),
                                       P(D), P(st), P(y), T, H, Pd, N)
    exp = xs.reshape(T, H, Pd) * D[None, :, None] + np.einsum("tn,hpn->thp", Cm.reshape(T, N), st0.reshape(H, Pd, N))
    assert np.allclose(y, exp.ravel(), atol=1e-5) and np.array_equal(st, st0)
    # A = 0: state = sum dt B x (pure accumulation)
    dt = O.rng_uniform(5, T * H, 0.1, 1.0)
    st = np.zeros(H * Pd * N, np.float32)
    O.oracle().orc_ssd_scan_sequential(P(xs), P(Bm), P(Cm), P(dt), P(np.zeros(H, np.float32)), P(D), P(st), P(y), T, H,
                                       Pd, N)
    ref = np.einsum("th,thp,tn->hpn", dt.reshape(T, H), xs.reshape(T, H, Pd), Bm.reshape(T, N))
    assert np.allclose(st, ref.ravel(), atol=1e-5)


@pytest.mark.parametrize("tag", ["q8", "q8b", "q4"])
def test_moe_golden(tag):
    g = golden("moe")
    N, d, E, ne, K, SH = [int(v) for v in g["shape"]]
    biased = bool(g[f"{tag}_biased"])
    out = np.zeros(N * d, np.float32)
    idx = np.zeros(N * K, np.int32)
    w = np.zeros(N * K, np.float32)
    args = [g[f"{tag}_{n}"] for n in ("gates", "ups", "downs", "sh_g", "sh_u", "sh_d")]
    assert O.oracle().orc_moe_forward_q(P(g[f"{tag}_x"]), P(g[f"{tag}_router"]), P(g[f"{tag}_bias"]) if biased else None,
                                        *[P(a) for a in args], P(out), P(idx), P(w), C.c_int64(N), d, E, ne, K, SH,
                                        int(g[f"{tag}_kind"])) == 0
    assert np.array_equal(idx, g[f"{tag}_idx"])
    assert np.array_equal(bits(w), bits(g[f"{tag}_w"]))
    assert np.array_equal(bits(out), bits(g[f"{tag}_out"]))
    probs = np.zeros(N * ne, np.float32)
    O.oracle().orc_moe_route(P(g[f"{tag}_x"]), P(g[f"{tag}_router"]), P(g[f"{tag}_bias"]) if biased else None,
                             P(probs), P(idx), P(w), C.c_int64(N), d, ne, K)
    assert np.array_equal(bits(probs), bits(g[f"{tag}_probs"]))
    assert np.allclose(w.reshape(N, K).sum(1), 1.0, atol=1e-6)
    if biased:  # +2 forces membership
        assert all({1, 6} <= set(r) for r in idx.reshape(N, K).tolist())


def test_router_tie_breaks_lowest_index():
    d, ne, K = 8, 6, 3
    x = np.ones(d, np.float32)
    rw = np.zeros(ne * d, np.float32)  # all logits equal
    probs = np.zeros(ne, np.float32)
    idx = np.zeros(K, np.int32)
    w = np.zeros(K, np.float32)
    O.oracle().orc_moe_route(P(x), P(rw), None, P(probs), P(idx), P(w), C.c_int64(1), d, ne, K)
    assert idx.tolist() == [0, 1, 2] and np.allclose(w, 1 / 3)


def test_permute_stable():
    idx = O.rng_below(9, 3000, 7)
    g = np.zeros(3000, np.int32)
    off = np.zeros(8, np.int32)
    O.oracle().orc_moe_permute(P(idx), C.c_int64(1000), 3, 7, P(g), P(off))
    assert np.array_equal(g, np.argsort(idx, kind="stable"))
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(idx, minlength=7))]))


def test_synthetic_weights_hash():
    """The shared synthetic recipe reproduces the bytes the reference ran on."""
    import hashlib
    g = golden("granite_c1_q8")
    w = O.granite_weights(O.C1, 2)
    h = hashlib.sha256()
    for name in sorted(w):
        h.update(name.encode())
        h.update(np.ascontiguousarray(w[name]).tobytes())
    assert h.hexdigest() == str(g["weights_sha256"])


@pytest.mark.slow
def test_granite_greedy_golden():
    """The oracle generator reproduces the reference's greedy ids and margins
    (first 8 tokens; the full 64 are checked on the GPU box against the HIP path)."""
    g = golden("granite_c1_q8")
    w = O.granite_weights(O.C1, 2)
    ids, margins = O.granite_generate(O.oracle().orc_granite_generate, O.C1, 2, w, g["prompt"], 8)
    assert np.array_equal(ids, g["ids"][:8])
    assert np.array_equal(bits(margins), bits(g["margins"][:8]))


def test_granite_options_golden():
    """The oracle generator with the Granite-4.0 fields (untied lm_head, aux-free router
    biases, embedding / residual multipliers, logits scaling) reproduces the compiled
    reference Generator bit for bit: ids, margins and every step's logits (first 10
    steps here; the GPU tests take all 24)."""
    import cases
    g = golden("granite_c1_q8_opts")
    w = cases.granite_opts_weights()
    ids, margins, lg = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, cases.C1_OPTS, 2, w, g["prompt"],
                                             10, max_ctx=int(g["max_ctx"]), logits=True)
    assert np.array_equal(ids, g["ids"][:10])
    assert np.array_equal(bits(margins), bits(g["margins"][:10]))
    assert np.array_equal(bits(lg), bits(g["logits"][:10]))
    assert np.array_equal(np.stack([w[f"layers.{i}.moe_bias"] for i in range(6)]), g["moe_bias"])


def test_granite_options_change_the_result():
    """Each option moves the logits (so the fixture above pins each of them): the same
    weights with one option reset to its default give different first logits."""
    import cases
    g = golden("granite_c1_q8_opts")
    w = cases.granite_opts_weights()
    prompt = g["prompt"][:16]
    base = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, cases.C1_OPTS, 2, w, prompt, 1, max_ctx=64,
                                 logits=True)[2]
    for key, default in (("emb_mult", 1.0), ("res_mult", 1.0), ("logits_scaling", 1.0)):
        c = dict(cases.C1_OPTS, **{key: default})
        other = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, c, 2, w, prompt, 1, max_ctx=64,
                                      logits=True)[2]
        assert not np.array_equal(other, base), key
    wz = dict(w)
    for i in range(6):
        wz[f"layers.{i}.moe_bias"] = np.zeros(8, np.float32)
    other = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, cases.C1_OPTS, 2, wz, prompt, 1, max_ctx=64,
                                  logits=True)[2]
    assert not np.array_equal(other, base), "moe_bias"
    wt = dict(w)
    wt["lm_head"] = w["tok_embeddings"]
    other = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, cases.C1_OPTS, 2, wt, prompt, 1, max_ctx=64,
                                  logits=True)[2]
    tied = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, dict(cases.C1_OPTS, tied=1), 2, w, prompt, 1,
                                 max_ctx=64, logits=True)[2]
    assert not np.array_equal(other, base) and np.array_equal(other, tied), "lm_head"


def _orc_topk(lg, K):
    vals = np.zeros(K, np.float32)
    ids = np.zeros(K, np.int32)
    assert O.oracle().orc_topk_select(P(lg), len(lg), K, P(vals), P(ids)) == 0
    return vals, ids


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_topk_select_golden(tag):
    g = golden("sampling")
    lg, K = g[f"tk{tag}_x"], int(g[f"tk{tag}_k"])
    vals, ids = _orc_topk(lg, K)
    assert np.array_equal(ids, g[f"tk{tag}_ids"])
    assert np.array_equal(bits(vals), bits(g[f"tk{tag}_vals"]))
    # an independent order: numpy lexsort by (value descending, index ascending)
    order = np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:K]
    assert np.array_equal(ids, order)


@pytest.mark.parametrize("tag", ["a", "b", "c", "d", "e"])
def test_rep_penalties_golden(tag):
    g = golden("sampling")
    rep, freq, pres = [float(v) for v in g[f"rp{tag}_p"]]
    hist = g["rp_hist"]
    o = g[f"rp{tag}_x"].copy()
    O.oracle().orc_apply_rep_penalties(P(o), len(o), P(hist), len(hist), O.f(rep), O.f(freq), O.f(pres))
    assert np.array_equal(bits(o), bits(g[f"rp{tag}_out"]))


def test_rep_penalties_closed_forms():
    V = 64
    x = O.rng_normal(75, V, 0, 2)
    x[3] = 1.5
    x[4] = -1.5
    hist = np.array([3, 3, 3, 4, 70, -2], np.int32)  # 3 seen 3 times, 4 once, the rest out of range
    o = x.copy()
    O.oracle().orc_apply_rep_penalties(P(o), V, P(hist), len(hist), O.f(2.0), O.f(0.5), O.f(0.25))
    assert o[3] == np.float32(np.float32(1.5 / 2.0) - np.float32(1.5)) - np.float32(0.25)
    assert o[4] == np.float32(np.float32(-1.5 * 2.0) - np.float32(0.5)) - np.float32(0.25)
    rest = np.ones(V, bool)
    rest[[3, 4]] = False
    assert np.array_equal(bits(o[rest]), bits(x[rest]))
    o = x.copy()  # neutral settings leave the logits alone
    O.oracle().orc_apply_rep_penalties(P(o), V, P(hist), len(hist), O.f(1.0), O.f(0.0), O.f(0.0))
    assert np.array_equal(bits(o), bits(x))


@pytest.mark.parametrize("kind", [2, 3])
def test_exact_decoder_agrees_with_oracle(kind):
    """The float64 block decoder of tests/exact.py (written from the block layouts) and
    the oracle's fp32 decode agree to the fp32 rounding of the oracle's arithmetic
    (Q8_0: q * d is exact in fp32, so bit-exact), hand-built blocks included."""
    import exact
    n = 256 * 64
    x = O.rng_normal(61, n, 0, 0.5)
    q = O.quantize(kind, x)
    ex = exact.dequant(kind, q, n)
    orc = O.dequantize(kind, q, n).astype(np.float64)
    if kind == 2:
        assert np.array_equal(ex, orc)
    else:
        assert np.max(np.abs(ex - orc) / np.maximum(np.abs(ex), 1e-30)) < 2.0 ** -22
        # a hand-built block: d = 1, dmin = 0.5, scale j = j + 1, min j = 2 j, code = (i % 16)
        blk = np.zeros(144, np.uint8)
        blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
        blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
        sc, mn = np.arange(1, 9), 2 * np.arange(8)
        s12 = np.zeros(12, np.int64)
        for j in range(4):
            s12[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            s12[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
            s12[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
        blk[4:16] = s12.astype(np.uint8)
        codes = np.arange(256) % 16
        for i in range(4):
            blk[16 + 32 * i: 48 + 32 * i] = codes[64 * i: 64 * i + 32] | (codes[64 * i + 32: 64 * i + 64] << 4)
        want = np.array([(j + 1) * codes[32 * j + t] - 0.5 * 2 * j for j in range(8) for t in range(32)], np.float64)
        assert np.array_equal(exact.dequant_q4_k(blk, 256), want)
        assert np.array_equal(O.dequantize(3, blk, 256).astype(np.float64), want)
