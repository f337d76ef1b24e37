"""GPU parity of the MoE FFN: router indices bit-exact, routing weights and
probabilities to 1e-6, permutation bit-exact against a stable sort, FFN
output within 1e-3 on the decode GEMV path (fp32 accumulate) and 2e-2 on
the prefill grouped MFMA path (bf16 operands)."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import close, golden

pytestmark = pytest.mark.gpu


class MoE:
    def __init__(self, gh, x, rw, bias, g, u, dn, sg, su, sd, N, d, E, ne, K, SH, kind):
        self.gh = gh
        self.b = {k: gh.Buf.from_array(v) for k, v in dict(x=x, rw=rw, g=g, u=u, dn=dn).items()}
        for k, v in dict(sg=sg, su=su, sd=sd, bias=bias).items():
            self.b[k] = gh.Buf.from_array(v) if v is not None else None
        self.shape = (N, d, E, ne, K, SH, kind)

    def run(self):
        gh = self.gh
        N, d, E, ne, K, SH, kind = self.shape
        out = gh.Buf.zeros(N * d, np.float32)
        probs = gh.Buf.zeros(N * ne, np.float32)
        idx = gh.Buf.zeros(N * K, np.int32)
        w = gh.Buf.zeros(N * K, np.float32)
        P = lambda k: self.b[k].p if self.b[k] is not None else None  # noqa
        gh.call("gh_moe_forward_bias_half", P("x"), P("rw"), P("bias"), P("g"), P("u"), P("dn"), P("sg"), P("su"),
                P("sd"), out.p, probs.p, idx.p, w.p, None, None, None, gh.i64(N), d, E, ne, K, SH, kind)
        return out.numpy(), probs.numpy(), idx.numpy(), w.numpy()


@pytest.mark.parametrize("tag", ["q8", "q8b", "q4"])
def test_moe_golden(gh, tag):
    g = golden("moe")
    N, d, E, ne, K, SH = [int(v) for v in g["shape"]]
    biased = bool(g[f"{tag}_biased"])
    m = MoE(gh, g[f"{tag}_x"], g[f"{tag}_router"], g[f"{tag}_bias"] if biased else None, g[f"{tag}_gates"],
            g[f"{tag}_ups"], g[f"{tag}_downs"], g[f"{tag}_sh_g"], g[f"{tag}_sh_u"], g[f"{tag}_sh_d"], N, d, E, ne, K,
            SH, int(g[f"{tag}_kind"]))
    out, probs, idx, w = m.run()
    assert np.array_equal(idx, g[f"{tag}_idx"])
    assert np.allclose(w, g[f"{tag}_w"], rtol=1e-6, atol=1e-7)
    assert np.allclose(probs, g[f"{tag}_probs"], rtol=1e-6, atol=1e-7)
    assert close(out, g[f"{tag}_out"], 1e-3)


def make_case(N, d, E, ne, K, SH, kind, seed, skew=False):
    x = O.rng_normal(seed, N * d)
    rw = O.rng_normal(seed + 1, ne * d, 0, 0.02)
    bias = None
    if skew:
        bias = np.zeros(ne, np.float32)
        bias[[3, 17, 40, 63 % ne]] = 2.0
    q = lambda s, n: O.quantize(kind, O.rng_normal(s, n, 0, 0.02))  # noqa
    return (x, rw, bias, q(seed + 2, ne * E * d), q(seed + 3, ne * E * d), q(seed + 4, ne * d * E),
            q(seed + 5, SH * d), q(seed + 6, SH * d), q(seed + 7, d * SH))


def oracle_moe(case, N, d, E, ne, K, SH, kind):
    x, rw, bias, g, u, dn, sg, su, sd = case
    out = np.zeros(N * d, np.float32)
    idx = np.zeros(N * K, np.int32)
    w = np.zeros(N * K, np.float32)
    assert O.oracle().orc_moe_forward_q(O.P(x), O.P(rw), O.P(bias), O.P(g), O.P(u), O.P(dn), O.P(sg), O.P(su),
                                        O.P(sd), O.P(out), O.P(idx), O.P(w), O.C.c_int64(N), d, E, ne, K, SH,
                                        kind) == 0
    return out, idx, w


@pytest.mark.parametrize("kind", [2, 3])
@pytest.mark.parametrize("N,skew", [(1, False), (1, True), (5, False)])
def test_moe_c5_decode(gh, kind, N, skew):
    """benchmark configuration c5 shapes (d 1536, 64 experts top-6, E 512, SH 1024), decode path."""
    d, E, ne, K, SH = 1536, 512, 64, 6, 1024
    case = make_case(N, d, E, ne, K, SH, kind, 500 + N, skew)
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, kind).run()
    r_out, r_idx, r_w = oracle_moe(case, N, d, E, ne, K, SH, kind)
    assert np.array_equal(idx, r_idx)
    assert np.allclose(w, r_w, rtol=1e-6, atol=1e-7)
    assert close(out, r_out, 1e-3)
    if skew:  # +2 on four experts: they are always selected
        assert set([3, 17, 40, 63]).issubset(set(idx.reshape(N, K)[0].tolist()))


@pytest.mark.parametrize("kind", [2, 3])
@pytest.mark.parametrize("skew", [False, True])
def test_moe_c5_prefill(gh, kind, skew):
    """benchmark configuration c5 prefill path at 64 tokens (oracle cost), grouped MFMA GEMM."""
    N, d, E, ne, K, SH = 64, 1536, 512, 64, 6, 1024
    case = make_case(N, d, E, ne, K, SH, kind, 600, skew)
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, kind).run()
    r_out, r_idx, r_w = oracle_moe(case, N, d, E, ne, K, SH, kind)
    assert np.array_equal(idx, r_idx)
    assert close(out, r_out, 2e-2)


@pytest.mark.parametrize("kind", [2, 3])
@pytest.mark.parametrize("N,d,E,ne,K,SH", [(128, 512, 256, 8, 2, 512), (45, 512, 512, 8, 2, 256),
                                           (7, 256, 256, 4, 1, 512)])
def test_moe_prefill_small_groups(gh, N, d, E, ne, K, SH, kind):
    """The skinny grouped path (Q4_K / Q8_0, a few dozen rows per expert, K of 256 or 512;
    c1's MoE shape first): ids bit-exact, output against the oracle."""
    case = make_case(N, d, E, ne, K, SH, kind, 610, False)
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, kind).run()
    r_out, r_idx, r_w = oracle_moe(case, N, d, E, ne, K, SH, kind)
    assert np.array_equal(idx, r_idx)
    assert close(out, r_out, 2e-2)


def test_moe_c5_prefill_2048_matches_decode_path(gh):
    """2048-token prefill (full c5 size): rows equal the per-token decode path."""
    N, d, E, ne, K, SH, kind = 2048, 1536, 512, 64, 6, 1024, 3
    case = make_case(N, d, E, ne, K, SH, kind, 700)
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, kind).run()
    x = case[0].reshape(N, d)
    for t in (0, 1, 777, 2047):
        c1 = (np.ascontiguousarray(x[t]),) + case[1:]
        o1, _, i1, _ = MoE(gh, *c1, 1, d, E, ne, K, SH, kind).run()
        assert np.array_equal(i1, idx.reshape(N, K)[t])
        assert close(out.reshape(N, d)[t], o1, 2e-2)


@pytest.mark.parametrize("skew", [False, True])
def test_moe_c5_prefill_2048_vs_oracle_rows(gh, skew):
    """benchmark configuration c5 prefill at its full 2048 tokens (grouped MFMA path),
    plain and skewed (+2.0 on 4 experts), against the oracle on 48 sampled
    token rows: the MoE FFN is per token, so the oracle on those rows alone is
    the oracle of the full batch there. Ids bit-exact on every row."""
    N, d, E, ne, K, SH, kind = 2048, 1536, 512, 64, 6, 1024, 3
    case = make_case(N, d, E, ne, K, SH, kind, 710, skew)
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, kind).run()
    rows = np.unique(np.concatenate([[0, 1, 1023, 2047], O.rng_below(711, 44, N)]))
    x = case[0].reshape(N, d)
    sub = (np.ascontiguousarray(x[rows]).ravel(),) + case[1:]
    r_out, r_idx, r_w = oracle_moe(sub, len(rows), d, E, ne, K, SH, kind)
    assert np.array_equal(idx.reshape(N, K)[rows].ravel(), r_idx)
    assert np.allclose(w.reshape(N, K)[rows].ravel(), r_w, rtol=1e-6, atol=1e-7)
    assert close(out.reshape(N, d)[rows], r_out.reshape(len(rows), d), 2e-2)
    if skew:
        forced = np.isin(idx.reshape(N, K), [3, 17, 40, 63]).sum(1)
        assert np.all(forced == 4)


@pytest.mark.parametrize("N,K,ne", [(1, 2, 8), (7, 2, 8), (2048, 6, 64), (333, 3, 5)])
def test_permute_matches_stable_sort(gh, N, K, ne):
    idx = O.rng_below(N + K, N * K, ne)
    di = gh.Buf.from_array(idx)
    grouped = gh.Buf.zeros(N * K, np.int32)
    offsets = gh.Buf.zeros(ne + 1, np.int32)
    gh.call("gh_moe_permute", di.p, gh.i64(N), K, ne, grouped.p, offsets.p)
    r_g = np.zeros(N * K, np.int32)
    r_o = np.zeros(ne + 1, np.int32)
    O.oracle().orc_moe_permute(O.P(idx), O.C.c_int64(N), K, ne, O.P(r_g), O.P(r_o))
    assert np.array_equal(grouped.numpy(), r_g)
    assert np.array_equal(offsets.numpy(), r_o)
    assert np.array_equal(r_g, np.argsort(idx, kind="stable"))


def test_moe_fp16_experts(gh):
    """qkind -1: fp16 expert matrices (the fp16 weight storage mode)."""
    N, d, E, ne, K, SH = 3, 256, 128, 8, 2, 256
    x = O.rng_normal(800, N * d)
    rw = O.rng_normal(801, ne * d, 0, 0.05)
    h = lambda s, n: O.f32_to_f16(O.rng_normal(s, n, 0, 0.05))  # noqa
    case = (x, rw, None, h(802, ne * E * d), h(803, ne * E * d), h(804, ne * d * E), h(805, SH * d), h(806, SH * d),
            h(807, d * SH))
    out, probs, idx, w = MoE(gh, *case, N, d, E, ne, K, SH, -1).run()
    r_out, r_idx, r_w = oracle_moe(case, N, d, E, ne, K, SH, -1)
    assert np.array_equal(idx, r_idx)
    assert close(out, r_out, 1e-3)
