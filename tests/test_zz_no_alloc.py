"""The allocation-free decode attention entry point
(gh_attention_decode_ring_fp16_noalloc) against the allocating one
(gh_attention_decode_ring_fp16) through the C ABI: the same kernels and the
same split-K plan, so the outputs must be bit-identical. Two calls in a row,
the second smaller (the static scratch keeps the first call's contents), and
a request beyond the scratch limit is refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu


def _case(L, H, KV, hd, seed):
    q = O.rng_normal(seed, H * hd)
    kc = O.f32_to_f16(O.rng_normal(seed + 1, L * KV * hd))
    vc = O.f32_to_f16(O.rng_normal(seed + 2, L * KV * hd))
    return q, kc, vc


def _run(gh, fn, bufs, out, H, KV, hd, rs, pin, cl, cm, sc, win):
    q, k, v = bufs
    if fn == "gh_attention_decode_ring_fp16":
        gh.call(fn, q.p, k.p, v.p, out.p, H, KV, hd, rs, pin, cl, cm, gh.fl(sc), None, win)
    else:
        gh.call(fn, q.p, k.p, v.p, out.p, H, KV, hd, rs, pin, cl, cm, gh.fl(sc), win)
    return out.numpy()


@pytest.mark.parametrize("first,second", [((32768, 32, 8, 128, 0, 0), (1024, 32, 8, 128, 0, 0)),
                                          ((2000, 8, 2, 64, 37, 300), (17, 8, 2, 64, 0, 0))])
def test_noalloc_matches_allocating_entry(gh, first, second):
    for L, H, KV, hd, rs, win in (first, second):
        bufs = [gh.Buf.from_array(a) for a in _case(L, H, KV, hd, 4000 + L)]
        pin = 8 if L > 8 else 0
        rs_ = rs % max(1, L - pin)
        sc = 1.0 / np.sqrt(hd)
        o1 = gh.Buf.zeros(H * hd, np.float32)
        o2 = gh.Buf.zeros(H * hd, np.float32)
        ref = _run(gh, "gh_attention_decode_ring_fp16", bufs, o1, H, KV, hd, rs_, pin, L, L, sc, win)
        got = _run(gh, "gh_attention_decode_ring_fp16_noalloc", bufs, o2, H, KV, hd, rs_, pin, L, L, sc, win)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (L, H, KV, hd)
        assert np.all(np.isfinite(got))


def test_noalloc_rejects_oversize(gh):
    """More partials than the 4 MiB scratch holds (64 q heads x 256 dims over
    a long context) is an error, not a launch."""
    lib = gh.load()
    H, KV, hd, L = 64, 8, 256, 1 << 20
    p = C.c_void_p(1 << 40)  # never dereferenced: the size check comes first
    rc = lib.gh_attention_decode_ring_fp16_noalloc(p, p, p, p, H, KV, hd, 0, 0, L, L, C.c_float(0.0625), 0)
    assert rc == 1
    assert b"static scratch" in lib.gh_last_error()
