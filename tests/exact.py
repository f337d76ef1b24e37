"""Exact (float64) decoding of the packed weight blocks, written from the GGML
block layouts independently of the oracle, and float64 reference products.

Q8_0 (quantization/quantize.cpp:58-133): 34 bytes per 32 values, an fp16 scale d
then 32 int8 codes q; value = q * d.
Q4_K (the GGML format): 144 bytes per 256 values: fp16 d, fp16 dmin, 12 bytes of
eight 6-bit scales and eight 6-bit mins, 128 bytes of 4-bit codes. Sub-block j
(32 values) is d * sc_j * q - dmin * m_j; bytes 32 i .. 32 i + 31 hold sub-block
2 i in their low nibbles and sub-block 2 i + 1 in their high nibbles.

Every product of an fp16 number, a 6-bit integer and a 4-bit integer is exact in
float64, so these values are the weights exactly as the blocks define them (the
oracle, like the reference CPU path, rounds each to fp16 before multiplying)."""
import numpy as np


def dequant_q8_0(packed, n):
    b = np.frombuffer(np.ascontiguousarray(packed).tobytes(), np.uint8).reshape(-1, 34)[: n // 32]
    d = b[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.float64)
    return (q * d[:, None]).reshape(-1)


def q4k_scales(sc12):
    """The eight (scale, min) pairs of a Q4_K header, [blocks, 8] each."""
    s = sc12.astype(np.int64)
    sc = np.empty((s.shape[0], 8), np.int64)
    mn = np.empty((s.shape[0], 8), np.int64)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        mn[:, j] = s[:, j + 4] & 63
    for j in range(4, 8):
        sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
        mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def dequant_q4_k(packed, n):
    b = np.frombuffer(np.ascontiguousarray(packed).tobytes(), np.uint8).reshape(-1, 144)[: n // 256]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    sc, mn = q4k_scales(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 8, 32), np.float64)
    q[:, 0::2, :] = qs & 0xF
    q[:, 1::2, :] = qs >> 4
    v = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * mn[:, :, None]
    return v.reshape(-1)


def dequant(kind, packed, n):
    if kind == 2:
        return dequant_q8_0(packed, n)
    if kind == 3:
        return dequant_q4_k(packed, n)
    raise ValueError(kind)


def linear64(x, packed, M, K, N, kind):
    """y = x W^T in float64 over the exactly decoded weights."""
    W = dequant(kind, packed, N * K).reshape(N, K)
    return np.asarray(x, np.float64).reshape(M, K) @ W.T


def errs(got, ref, floor=0.1):
    """(normwise max|d|/max|ref|, elementwise max |d|/|ref| over |ref| >= floor max|ref|)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    m = np.max(np.abs(ref))
    sel = np.abs(ref) >= floor * m
    return float(np.max(np.abs(got - ref)) / m), float(np.max(np.abs(got[sel] - ref[sel]) / np.abs(ref[sel])))
