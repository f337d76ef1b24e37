#!/usr/bin/env python3
"""Benchmark of the MI355X backend on the headline metric:
"batch-1 decode tok/s + prefill tok/s (Q4_K hybrid); % HBM/MFMA roofline".

Workload (one "step"): the tiny Granite-4.0 hybrid of benchmark configuration c1
(vocab 4096, d 512, layers [M, M, A, M, M, A], MoE 8 experts top-2 + shared)
with its matrices in Q4_K (the metric's weight format; config 1 names Q8_0,
which is reported beside it), random-init by the shared synthetic recipe:
prefill of a 128-token prompt, then 64 greedy tokens with the decode step
replayed from a captured hipGraph. `value` is decode tok/s: the 63 decode
steps of a 64-token generate() call over its wall time (the first id comes
from the prefill's logits; the CPU baseline counts the same 63 steps); prefill
tok/s is reported beside it.

`roofline` is the path's dominant HBM kernel at production shape, the
single-token Q4_K GEMV of benchmark configuration c2 (14336x4096), timed alone over
repeated launches with HIP events on the backend stream, cold (10 copies of
the weights in rotation, 331 MB, more than the 256 MB MALL: every launch reads
HBM; the headline) and warm (the same copy every launch); `traffic` comes from
the committed rocprofv3 PMC summary of `--probe` (FETCH_SIZE + WRITE_SIZE per
launch, scaled by what the counters read for a plain copy of known size);
`stream_ceiling` is a read-only streaming kernel over the same cold rotation
(what the memory system delivers to a kernel that does nothing but read);
`kernels` gives the per-kernel figures for benchmark configurations c2-c5 at
full size. `cpu_baseline` times the CPU oracle (a restatement of the
reference's CPU path) on the same workload on the host's cores.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-kernels] [--no-cpu] [--eager-decode]
python bench.py --probe     # 20 cold launches of the roofline GEMV + 20 plain 64 MiB copies, for PMC runs
python bench.py --probe-mfma  # 5 launches of each MFMA-bound kernel (c3 scan, c2 GEMM, c4 prefill), for PMC runs
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jdm-ghassan_v1_flach_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_TFLOPS = 2500.0  # dense fp16/bf16 MFMA, MI355X

C1 = dict(V=4096, d=512, L=6, H=8, KV=2, hd=64, E=256, ne=8, K=2, SH=512, d_inner=1024, m_heads=16, m_dhead=64,
          m_dstate=64, conv_k=4, layer_types=[0, 0, 1, 0, 0, 1], eps=1e-5, scale=0.125)
PROMPT, N_NEW, MAX_CTX = 128, 64, 256


def cfg_arrays(c, qkind):
    ints = [c["V"], c["d"], c["L"], c["H"], c["KV"], c["hd"], c["E"], c["ne"], c["K"], c["SH"], c["d_inner"],
            c["m_heads"], c["m_dhead"], c["m_dstate"], c["conv_k"], qkind] + list(c["layer_types"])
    return np.array(ints, np.int32), np.array([c["eps"], c["scale"]], np.float32)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Model:
    def __init__(self, gh, qkind):
        self.gh = gh
        cfg, fcfg = cfg_arrays(C1, qkind)
        self.h = C.c_void_p()
        gh.call("gh_granite_create", cfg.ctypes.data_as(C.c_void_p), fcfg.ctypes.data_as(C.c_void_p), MAX_CTX,
                C.byref(self.h))
        gh.call("gh_granite_init_synthetic", self.h, C.c_uint64(0))
        self.ids = np.zeros(N_NEW, np.int32)

    use_graph = 1

    def step(self, prompt, t_pf, t_dec):
        gh = self.gh
        gh.call("gh_granite_reset", self.h)
        t_pf.start()
        gh.call("gh_granite_prefill", self.h, prompt.ctypes.data_as(C.c_void_p), len(prompt), None, 1)
        a = t_pf.stop_ms()
        t_dec.start()
        gh.call("gh_granite_generate_greedy", self.h, N_NEW, self.ids.ctypes.data_as(C.c_void_p), self.use_graph)
        b = t_dec.stop_ms()
        return a, b


def time_launches(gh, fn, reps, warm=3):
    for _ in range(warm):
        fn()
    t = gh.Timer()
    t.start()
    for _ in range(reps):
        fn()
    return t.stop_ms() / reps


def entry(name, ms, bytes_=None, flops=None, bound="hbm"):
    e = {"kernel": name, "us": round(ms * 1e3, 2)}
    if bytes_ is not None:
        gbs = bytes_ / (ms * 1e-3) / 1e9
        e["GB_s"] = round(gbs, 1)
        e["algorithmic_bytes"] = int(bytes_)
    if flops is not None:
        tf = flops / (ms * 1e-3) / 1e12
        e["TFLOP_s"] = round(tf, 2)
    if bound == "hbm":
        e["frac"] = round(e["GB_s"] / HBM_PEAK_GBS, 4)
    else:
        e["frac"] = round(e["TFLOP_s"] / MFMA_F16_TFLOPS, 4)
    e["bound"] = bound
    return e


def moe_decode_case(gh, d, E, ne, K, SH, kind, N=1, seed=5, skew=False):
    x = gh.rng_normal(seed, N * d)
    rw = gh.rng_normal(seed + 1, ne * d, 0, 0.02)
    bias = None
    if skew:
        bias = np.zeros(ne, np.float32)
        bias[[3, 17, 40, 63 % ne]] = 2.0
    q = lambda s, n: gh.quantize(kind, gh.rng_normal(s, n, 0, 0.02))  # noqa
    arrs = [x, rw, bias, q(seed + 2, ne * E * d), q(seed + 3, ne * E * d), q(seed + 4, ne * d * E),
            q(seed + 5, SH * d), q(seed + 6, SH * d), q(seed + 7, d * SH)]
    bufs = [gh.Buf.from_array(a) if a is not None else None for a in arrs]
    out = gh.Buf.zeros(N * d, np.float32)

    def run():
        gh.call("gh_moe_forward_bias_half", *[b.p if b is not None else None for b in bufs], out.p, None, None, None,
                None, None, None, gh.i64(N), d, E, ne, K, SH, kind)
    return run, bufs, out


def to_f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def to_bf16(x):
    """fp32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def kernel_suite(gh):
    res = {}
    # ---------------- c2: quantized GEMV / GEMM, W 14336x4096
    for kind, kname in ((3, "q4_k"), (2, "q8_0")):
        for (M, K, N) in ((1, 4096, 14336), (8, 4096, 14336), (1, 14336, 4096), (8, 14336, 4096),
                          (2048, 4096, 14336), (2048, 14336, 4096)):
            w = gh.quantize(kind, gh.rng_normal(2, N * K, 0, 0.02))
            x = gh.rng_normal(3, M * K)
            dw, dx = gh.Buf.from_array(w), gh.Buf.from_array(x)
            y = gh.Buf.zeros(M * N, np.float32)
            ms = time_launches(gh, lambda: gh.call("gh_linear_forward_q4", dx.p, dw.p, y.p, M, K, N, kind),
                               10 if M > 8 else 200)
            tag = f"c2_{kname}_M{M}_{N}x{K}"
            if M <= 8:
                g8 = "k_gemv8<Q4_K>" if kind == 3 else "k_gemv8<Q8_0>"
                kern = ("k_gemv_q4k_i8" if (kind == 3 and M == 1 and K <= 4096) else
                        "k_gemv_q4k_i8 (4 K slices) + k_g8_sum" if (kind == 3 and M == 1) else
                        "k_gemv_q4k_i8<Q8> (2 / 7 K slices) + k_g8_sum" if M == 1 else
                        g8 + " (2 K slices) + k_g8_sum" if (2 <= M <= 8 and K == 4096 and kind == 3) else
                        g8 if (2 <= M <= 8 and K <= 4096) else
                        g8 + " (4 K slices) + k_g8_sum" if 2 <= M <= 8 else "k_gemv_mfma")
                res[tag] = entry(kern, ms, bytes_=w.nbytes + x.nbytes + M * N * 4, flops=2.0 * M * N * K)
            else:
                res[tag] = entry("k_dequant_fused (weights + x to bf16)+hipBLASLt bf16 GEMM (fp32 out)", ms,
                                 bytes_=w.nbytes + x.nbytes + M * N * 4, flops=2.0 * M * N * K, bound="mfma")
            del dw, dx, y
    # ---------------- c3: SSD scan T=4096 + decode state update
    T, H, P, N = 4096, 48, 64, 128
    arrs = [gh.rng_normal(31, T * H * P), gh.rng_normal(32, T * N) / np.float32(np.sqrt(N)),
            gh.rng_normal(33, T * N) / np.float32(np.sqrt(N)),
            np.log1p(np.exp(gh.rng_normal(34, T * H, -2.0, 0.5).astype(np.float64))).astype(np.float32),
            -np.exp(gh.rng_uniform(35, H, 0.0, np.log(16.0))).astype(np.float32), np.ones(H, np.float32)]
    bufs = [gh.Buf.from_array(a) for a in arrs]
    st = gh.Buf.zeros(H * P * N, np.float32)
    yb = gh.Buf.zeros(T * H * P, np.float32)
    ms = time_launches(gh, lambda: gh.call("gh_ssd_scan", *[b.p for b in bufs], st.p, yb.p, T, H, P, N, 256), 10)
    scan_bytes = 2 * (T * H * P + 2 * T * N + T * H + T * H * P) + 2 * H * P * N * 4  # fp16-equivalent I/O + state
    flops = 2.0 * (16 * 256 * 256 * N) + H * 16 * (2.0 * 256 * 256 * P + 4.0 * 256 * N * P)
    res["c3_ssd_scan_T4096"] = entry("k_ssd_state_cb+k_ssd_state_pass+k_ssd_out (3 launches)", ms, bytes_=scan_bytes,
                                     flops=flops, bound="hbm")
    del bufs, st, yb
    d, di, nh, ds, kk = 1536, 3072, 48, 128, 4
    conv_dim = di + 2 * ds
    proj = di + conv_dim + nh
    w_in = gh.quantize(3, gh.rng_normal(36, proj * d, 0, 0.02))
    w_out = gh.quantize(3, gh.rng_normal(37, d * di, 0, 0.02))
    vecs = [gh.rng_normal(38, conv_dim * kk, 0, 0.3), gh.rng_normal(39, conv_dim, 0, 0.1), np.zeros(nh, np.float32),
            gh.rng_uniform(40, nh, 0.0, np.log(16.0)), np.ones(nh, np.float32), np.ones(di, np.float32)]
    b_in, b_out = gh.Buf.from_array(w_in), gh.Buf.from_array(w_out)
    bv = [gh.Buf.from_array(v) for v in vecs]
    conv = gh.Buf.zeros(conv_dim * (kk - 1), np.float32)
    ssm = gh.Buf.zeros(nh * 64 * ds, np.float32)
    xin = gh.Buf.from_array(gh.rng_normal(41, d))
    out = gh.Buf.zeros(d, np.float32)
    ms = time_launches(gh, lambda: gh.call("gh_mamba2_step_half", xin.p, b_in.p, *[b.p for b in bv], b_out.p, conv.p,
                                           ssm.p, out.p, d, di, conv_dim, nh, 64, ds, kk, gh.fl(1e-5), 3), 100)
    step_bytes = w_in.nbytes + w_out.nbytes + 2 * nh * 64 * ds * 4 + 4 * (proj + 2 * conv_dim * (kk - 1) + d + 2 * di)
    res["c3_mamba_step_layer"] = entry("gemv+k_step_conv+k_step_scan+k_gated_norm+gemv", ms, bytes_=step_bytes)
    del b_in, b_out, bv, conv, ssm
    # ---------------- c4: decode attention, L = 1k / 8k / 32k, ragged batch 16, prefill 4096
    Hq, KVh, hd = 32, 8, 128
    kv_all = gh.rng_normal(4, 2 * 32768 * KVh * hd)  # K then V, N(0,1) (benchmark configuration c4, seed 4)
    k16, v16 = to_f16(kv_all[:32768 * KVh * hd]), to_f16(kv_all[32768 * KVh * hd:])
    kb16, vb16 = to_bf16(kv_all[:32768 * KVh * hd]), to_bf16(kv_all[32768 * KVh * hd:])
    q = gh.Buf.from_array(gh.rng_normal(40, Hq * hd))
    o = gh.Buf.zeros(Hq * hd, np.float32)
    sc = 1.0 / np.sqrt(hd)
    for L in (1024, 8192, 32768):
        n = L * KVh * hd
        # bf16 cache as configured: the paged entry point with one sequence
        kp, vp = gh.Buf.from_array(kb16[:n]), gh.Buf.from_array(vb16[:n])
        npg = L // 64
        pt = gh.Buf.from_array(np.arange(npg, dtype=np.int32))
        ln = gh.Buf.from_array(np.array([L], np.int32))
        ms = time_launches(gh, lambda: gh.call("gh_attention_decode_paged_bf16", q.p, kp.p, vp.p, pt.p, ln.p, 1, npg, 64,
                                               L, o.p, Hq, KVh, hd, gh.fl(sc)), 100)
        res[f"c4_decode_bf16_L{L}"] = entry("k_attn_decode2<paged bf16>+k_attn_combine", ms,
                                            bytes_=n * 2 * 2 + 2 * Hq * hd * 4, flops=4.0 * Hq * hd * L)
        del kp, vp
        # the reference's fp16 ring cache (attention_decode_ring_fp16)
        kc, vc = gh.Buf.from_array(k16[:n]), gh.Buf.from_array(v16[:n])
        ms = time_launches(gh, lambda: gh.call("gh_attention_decode_ring_fp16", q.p, kc.p, vc.p, o.p, Hq, KVh, hd, 0,
                                               8, L, L, gh.fl(sc), None, 0), 100)
        res[f"c4_decode_L{L}"] = entry("k_attn_decode2+k_attn_combine (fp16 ring)", ms,
                                       bytes_=n * 2 * 2 + 2 * Hq * hd * 4, flops=4.0 * Hq * hd * L)
        del kc, vc
    del k16, v16, kb16, vb16, kv_all
    ps = 64
    lens = (512 + gh.rng_below(4, 16, 8192 - 512 + 1)).astype(np.int32)
    max_pages = (int(lens.max()) + ps - 1) // ps
    pt = np.zeros((16, max_pages), np.int32)
    nxt = 0
    for s in range(16):
        for i in range((int(lens[s]) + ps - 1) // ps):
            pt[s, i] = nxt
            nxt += 1
    kvr = gh.rng_normal(41, 2 * nxt * ps * KVh * hd)  # N(0,1) bf16 pages
    kp = gh.Buf.from_array(to_bf16(kvr[:nxt * ps * KVh * hd]))
    vp = gh.Buf.from_array(to_bf16(kvr[nxt * ps * KVh * hd:]))
    del kvr
    qb = gh.Buf.from_array(gh.rng_normal(5, 16 * Hq * hd))
    dpt, dl = gh.Buf.from_array(pt), gh.Buf.from_array(lens)
    ob = gh.Buf.zeros(16 * Hq * hd, np.float32)
    ms = time_launches(gh, lambda: gh.call("gh_attention_decode_paged_bf16", qb.p, kp.p, vp.p, dpt.p, dl.p, 16,
                                           max_pages, ps, int(lens.max()), ob.p, Hq, KVh, hd, gh.fl(0.0884)), 50)
    res["c4_ragged_decode_b16"] = entry("k_attn_decode2<paged>+k_attn_combine", ms,
                                        bytes_=int(lens.sum()) * KVh * hd * 2 * 2, flops=4.0 * Hq * hd * int(lens.sum()))
    del kp, vp
    Tp = 4096
    qf = gh.Buf.from_array(gh.rng_normal(6, Tp * Hq * hd))
    kf = gh.Buf.from_array(gh.rng_normal(7, Tp * KVh * hd))
    vf = gh.Buf.from_array(gh.rng_normal(8, Tp * KVh * hd))
    of = gh.Buf.zeros(Tp * Hq * hd, np.float32)
    ms = time_launches(gh, lambda: gh.call("gh_attention_forward_ex", qf.p, kf.p, vf.p, of.p, None, 1, Tp, Hq, KVh, hd,
                                           gh.fl(0.0884), 0, None), 10)
    res["c4_prefill_T4096"] = entry("k_kv_f16+k_attn_prefill_f16", ms, flops=4.0 * Hq * hd * Tp * (Tp + 1) / 2, bound="mfma")
    del qf, kf, vf, of
    # ---------------- c5: MoE FFN decode / prefill, skewed routing
    d5, E5, ne5, K5, SH5 = 1536, 512, 64, 6, 1024
    expert_bytes = 3 * E5 * d5 * 144 // 256
    for N, skew, tag in ((1, False, "c5_moe_decode"), (1, True, "c5_moe_decode_skewed"),
                         (2048, False, "c5_moe_prefill_2048"), (2048, True, "c5_moe_prefill_2048_skewed")):
        run, bufs, out = moe_decode_case(gh, d5, E5, ne5, K5, SH5, 3, N=N, skew=skew)
        ms = time_launches(gh, run, 100 if N == 1 else 10)
        fl = 2.0 * N * (K5 * 3 * E5 * d5 + 3 * SH5 * d5)
        if N == 1:
            res[tag] = entry("k_route_chain+k_moe_gemv (selection inside)+k_moe_down_par", ms, bytes_=K5 * expert_bytes + 3 * SH5 * d5 * 144 // 256,
                             flops=fl)
        else:
            res[tag] = entry("moe route+permute+group gemm x2+shared+combine", ms,
                             bytes_=ne5 * expert_bytes + 3 * SH5 * d5 * 144 // 256, flops=fl, bound="mfma")
        del bufs, out
    # ---------------- sampling ops of the decode loop (next-row scope: top-K, penalties)
    for V, K in ((4096, 40), (100352, 40), (262144, 128)):
        lg = gh.Buf.from_array(gh.rng_normal(9, V))
        tv, ti = gh.Buf.zeros(K, np.float32), gh.Buf.zeros(K, np.int32)
        ms = time_launches(gh, lambda: gh.call("gh_topk_select", lg.p, V, K, tv.p, ti.p), 50)
        res[f"topk_V{V}_K{K}"] = entry("k_topk_pass (1-3 passes)", ms, bytes_=V * 4)
        del lg, tv, ti
    V, n = 100352, 2048
    lg = gh.Buf.from_array(gh.rng_normal(10, V))
    hist = (np.arange(n, dtype=np.int32) * 7919) % V
    hp = hist.ctypes.data_as(C.c_void_p)
    ms = time_launches(gh, lambda: gh.call("gh_apply_rep_penalties", lg.p, V, hp, n, gh.fl(1.1), gh.fl(0.1),
                                           gh.fl(0.1)), 50)
    res[f"rep_penalties_V{V}_hist{n}"] = entry("H2D history + k_rep_penalties", ms, bytes_=n * 4 * 3 + n * 8)
    # ---------------- GGUF: packed Q4_K blocks of the c2 matrix from a mapped file into HBM
    res["gguf_read_packed_c2_q4k"] = gguf_load_case(gh)
    return res


def gguf_load_case(gh):
    """Writes the c2 14336x4096 Q4_K matrix to a GGUF file under the system temp
    folder and times gh_gguf_read_packed into device memory (host page cache -> HBM)."""
    import tempfile
    lib = gh.load()
    N, K = 14336, 4096
    w = gh.quantize(3, gh.rng_normal(2, N * K, 0, 0.02))
    fd, path = tempfile.mkstemp(suffix=".gguf")
    os.close(fd)
    try:
        names = (C.c_char_p * 1)(b"layers.0.moe_sh_up")
        types = (C.c_uint32 * 1)(12)
        nd = (C.c_int * 1)(2)
        dims = (C.c_uint64 * 8)(K, N)
        data = (C.c_void_p * 1)(w.ctypes.data)
        gh.check(lib.gh_gguf_write(path.encode(), 1, names, types, nd, dims, data, 0, None, None, None))
        h = C.c_void_p()
        gh.check(lib.gh_gguf_open(path.encode(), C.byref(h)))
        dev = gh.Buf.zeros(w.nbytes, np.uint8)
        read = lambda: gh.check(lib.gh_gguf_read_packed(h, b"layers.0.moe_sh_up", 3, dev.p, 1, C.c_size_t(w.nbytes)))
        read()
        t0 = time.perf_counter()
        for _ in range(5):
            read()
        ms = (time.perf_counter() - t0) / 5 * 1e3
        lib.gh_gguf_close(h)
        e = entry("gguf_read_packed (mapped file -> hipMemcpy, PCIe)", ms, bytes_=w.nbytes)
        e["bound"] = "pcie"
        e.pop("frac", None)
        return e
    finally:
        os.unlink(path)


def cpu_baseline(prompt, n_prefill=PROMPT, n_new=N_NEW):
    """The CPU oracle (restated reference CPU path) on the same workload: c1
    Q4_K, the 128-token prompt and 64 greedy tokens (about a minute of CPU
    time on 16 host threads)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    w = O.granite_weights(O.C1, 3)
    names, ptrs, npar = O._param_arrays(w)
    cfg, fcfg = O.granite_cfg(O.C1, 3)
    pr = np.ascontiguousarray(prompt[:n_prefill], np.int32)
    ids = np.zeros(n_new, np.int32)
    mg = np.zeros(n_new, np.float32)
    secs = np.zeros(2, np.float64)
    rc = O.oracle().orc_granite_generate_timed(O.P(cfg), O.P(fcfg), names, ptrs, npar, O.P(pr), n_prefill, n_new,
                                               MAX_CTX, O.P(ids), O.P(mg), secs.ctypes.data_as(C.c_void_p))
    assert rc == 0
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round((n_new - 1) / secs[1], 3), "unit": "decode tok/s", "cores": threads, "kind": "port",
            "prefill_tok_s": round(n_prefill / secs[0], 3),
            "sample": f"CPU oracle (restated reference CPU path, OpenMP {threads} threads where the reference "
                      f"parallelises): c1 Q4_K, {n_prefill}-token prompt prefill + {n_new - 1} greedy decode steps; "
                      f"prefill {secs[0]:.2f} s, decode {secs[1]:.2f} s"}


def calibrate(n_prefill=PROMPT, n_new=N_NEW):
    """Calibration row: the genuine reference CPU Generator (oracle/_ref, compiled from the
    reference sources in the build container; test infrastructure) and the CPU oracle timed on
    the same c1 Q8_0 workload (the reference has no K-quants), with equal greedy ids checked.
    The ratio says how closely the restated port's speed tracks the original's."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    if not O.ref_available():
        return {"skipped": "oracle/_ref/libgai_ref.so is not built here"}
    w = O.granite_weights(O.C1, 2)
    names, ptrs, npar = O._param_arrays(w)
    cfg, fcfg = O.granite_cfg(O.C1, 2)
    pr = O.rng_below(1, n_prefill, O.C1["V"])
    out = {}
    for kind, fn in (("reference", O.ref().ref_granite_generate_timed),
                     ("port", O.oracle().orc_granite_generate_timed)):
        ids = np.zeros(n_new, np.int32)
        mg = np.zeros(n_new, np.float32)
        secs = np.zeros(2, np.float64)
        rc = fn(O.P(cfg), O.P(fcfg), names, ptrs, npar, O.P(pr), n_prefill, n_new, MAX_CTX, O.P(ids), O.P(mg),
                secs.ctypes.data_as(C.c_void_p))
        assert rc == 0, (kind, rc)
        out[kind] = {"decode_tok_s": round((n_new - 1) / secs[1], 3), "prefill_tok_s": round(n_prefill / secs[0], 3),
                     "ids": ids}
    same = int(np.argmin(out["reference"]["ids"] == out["port"]["ids"])) if not np.array_equal(
        out["reference"]["ids"], out["port"]["ids"]) else n_new
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    for v in out.values():
        v.pop("ids")
    return {"workload": f"c1 Q8_0, {n_prefill}-token prompt prefill + {n_new - 1} greedy decode steps",
            "threads": threads, "reference": out["reference"], "port": out["port"],
            "port_over_reference_decode": round(out["port"]["decode_tok_s"] / out["reference"]["decode_tok_s"], 4),
            "port_over_reference_prefill": round(out["port"]["prefill_tok_s"] / out["reference"]["prefill_tok_s"], 4),
            "equal_ids": same}


COLD_COPIES = 10  # 10 x 33 MB of weights > the 256 MB Infinity Cache (MALL)


def roofline_gemv(gh, copies=1):
    """The c2 headline GEMV (Q4_K, 14336x4096, M=1): buffers and a launcher.
    copies > 1: that many distinct copies of the weights (and of x, y), used in
    rotation, so that every launch reads its weights from HBM rather than from
    the MALL a previous launch left them in (cold-cache measurement)."""
    K2, N2 = 4096, 14336
    w2 = gh.quantize(3, gh.rng_normal(2, N2 * K2, 0, 0.02))
    x2 = gh.rng_normal(3, K2)
    sets = [(gh.Buf.from_array(w2), gh.Buf.from_array(x2), gh.Buf.zeros(N2, np.float32)) for _ in range(copies)]
    nbytes = w2.nbytes + x2.nbytes + N2 * 4
    it = [0]

    def run():
        w, x, y = sets[it[0]]
        it[0] = (it[0] + 1) % copies
        gh.call("gh_linear_forward_q4", x.p, w.p, y.p, 1, K2, N2, 3)
    return run, sets, nbytes


def stream_ceiling(gh, nbytes, copies=COLD_COPIES, reps=500):
    """Read-only streaming of `nbytes` per launch over `copies` buffers in
    rotation (the same cold-cache rotation as the roofline GEMV): the fastest
    of a few grid sizes. Returns (us per launch, GB/s, blocks)."""
    nbytes = nbytes // 16 * 16
    bufs = [gh.Buf.zeros(nbytes // 4, np.float32) for _ in range(copies)]
    best = None
    for blocks in (1024, 2048, 4096, 8192):
        sink = gh.Buf.zeros(blocks, np.float32)
        it = [0]

        def run():
            b = bufs[it[0]]
            it[0] = (it[0] + 1) % copies
            gh.call("gh_stream_read", b.p, gh.i64(nbytes), sink.p, blocks)
        ms = time_launches(gh, run, reps)
        if best is None or ms < best[0]:
            best = (ms, blocks)
    del bufs
    return best[0] * 1e3, nbytes / (best[0] * 1e-3) / 1e9, best[1]


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_q4k_c2_traffic.txt")
COPY_FLOATS = 16 << 20  # 64 MiB per side


def probe(gh):
    run, bufs, nbytes = roofline_gemv(gh, COLD_COPIES)
    for _ in range(20):
        run()
    src = gh.Buf.from_array(np.ones(COPY_FLOATS, np.float32))
    dst = gh.Buf.zeros(COPY_FLOATS, np.float32)
    for _ in range(20):
        gh.call("gh_copy", dst.p, src.p, gh.i64(COPY_FLOATS))
    sbufs = [gh.Buf.zeros(33030144 // 4, np.float32) for _ in range(COLD_COPIES)]
    sink = gh.Buf.zeros(4096, np.float32)
    for i in range(20):
        gh.call("gh_stream_read", sbufs[i % COLD_COPIES].p, gh.i64(33030144 // 16 * 16), sink.p, 4096)
    gh.sync()
    log(f"probe: 20 x roofline GEMV, cold ({COLD_COPIES} weight copies in rotation; {nbytes} algorithmic bytes), "
        f"20 x k_copy ({COPY_FLOATS * 4} B read + written)")


def probe_mfma(gh):
    """5 launches each of the c3 SSD scan (T=4096), the c2 Q4_K prefill GEMM
    (M=2048) and the c4 causal prefill attention (T=4096), full size."""
    T, H, P, N = 4096, 48, 64, 128
    arrs = [gh.rng_normal(31, T * H * P), gh.rng_normal(32, T * N) / np.float32(np.sqrt(N)),
            gh.rng_normal(33, T * N) / np.float32(np.sqrt(N)),
            np.log1p(np.exp(gh.rng_normal(34, T * H, -2.0, 0.5).astype(np.float64))).astype(np.float32),
            -np.exp(gh.rng_uniform(35, H, 0.0, np.log(16.0))).astype(np.float32), np.ones(H, np.float32)]
    bufs = [gh.Buf.from_array(a) for a in arrs]
    st, yb = gh.Buf.zeros(H * P * N, np.float32), gh.Buf.zeros(T * H * P, np.float32)
    for _ in range(5):
        gh.call("gh_ssd_scan", *[b.p for b in bufs], st.p, yb.p, T, H, P, N, 256)
    gh.sync()
    del bufs, st, yb
    M, K, Nn = 2048, 4096, 14336
    dw = gh.Buf.from_array(gh.quantize(3, gh.rng_normal(2, Nn * K, 0, 0.02)))
    dx, dy = gh.Buf.from_array(gh.rng_normal(3, M * K)), gh.Buf.zeros(M * Nn, np.float32)
    for _ in range(5):
        gh.call("gh_linear_forward_q4", dx.p, dw.p, dy.p, M, K, Nn, 3)
    gh.sync()
    del dw, dx, dy
    Tp, Hq, KVh, hd = 4096, 32, 8, 128
    qf = gh.Buf.from_array(gh.rng_normal(6, Tp * Hq * hd))
    kf = gh.Buf.from_array(gh.rng_normal(7, Tp * KVh * hd))
    vf = gh.Buf.from_array(gh.rng_normal(8, Tp * KVh * hd))
    of = gh.Buf.zeros(Tp * Hq * hd, np.float32)
    for _ in range(5):
        gh.call("gh_attention_forward_ex", qf.p, kf.p, vf.p, of.p, None, 1, Tp, Hq, KVh, hd, gh.fl(0.0884), 0, None)
    gh.sync()
    del qf, kf, vf, of
    # c2 down-projection (K=14336 -> N=4096), c5 MoE prefill at 2048 tokens, and the
    # skinny GEMM of the c1 prefill (Mamba in_proj, 128 tokens x 2192 x 512)
    dw = gh.Buf.from_array(gh.quantize(3, gh.rng_normal(2, 4096 * 14336, 0, 0.02)))
    dx, dy = gh.Buf.from_array(gh.rng_normal(3, M * 14336)), gh.Buf.zeros(M * 4096, np.float32)
    for _ in range(5):
        gh.call("gh_linear_forward_q4", dx.p, dw.p, dy.p, M, 14336, 4096, 3)
    gh.sync()
    del dw, dx, dy
    run, bufs, out = moe_decode_case(gh, 1536, 512, 64, 6, 1024, 3, N=2048)
    for _ in range(5):
        run()
    gh.sync()
    del bufs, out
    dw = gh.Buf.from_array(gh.quantize(3, gh.rng_normal(2, 2192 * 512, 0, 0.02)))
    dx, dy = gh.Buf.from_array(gh.rng_normal(3, 128 * 512)), gh.Buf.zeros(128 * 2192, np.float32)
    for _ in range(5):
        gh.call("gh_linear_forward_q4", dx.p, dw.p, dy.p, 128, 512, 2192, 3)
    gh.sync()
    log("probe-mfma: 5 x SSD scan c3, 5 x GEMM c2 Q4_K M=2048, 5 x prefill attention c4 T=4096, "
        "5 x c2 down-projection M=2048, 5 x MoE prefill c5 2048 tokens, 5 x skinny GEMM c1 in_proj M=128")


def read_traffic():
    """HBM bytes per launch of the roofline GEMV from the committed PMC
    summary (a line `traffic_bytes_per_launch: N`), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(float(ln.split(":", 1)[1]))
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager-decode", action="store_true",
                    help="launch the decode step's kernels one by one instead of replaying the captured graph")
    ap.add_argument("--probe-mfma", action="store_true",
                    help="only run the MFMA-bound kernels (c3 SSD scan, c2 prefill GEMM, c4 prefill attention), "
                         "5 launches each, for rocprofv3 --pmc runs")
    ap.add_argument("--probe", action="store_true",
                    help="only run the roofline GEMV and a plain copy of known size (for rocprofv3 --pmc)")
    ap.add_argument("--calibrate", action="store_true",
                    help="CPU only: time the compiled reference (oracle/_ref) and the CPU oracle on c1 Q8_0")
    args = ap.parse_args()
    if args.calibrate:
        print(json.dumps({"calibration": calibrate()}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); multi-GPU sharding is a "
              "design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    import ghassan_hip as gh
    gh.load()
    if args.probe:
        probe(gh)
        return
    if args.probe_mfma:
        probe_mfma(gh)
        return
    Model.use_graph = 0 if args.eager_decode else 1
    prompt = gh.rng_below(1, PROMPT, C1["V"])

    model = Model(gh, 3)
    t_pf, t_dec = gh.Timer(), gh.Timer()
    for _ in range(args.warmup):
        model.step(prompt, t_pf, t_dec)
    gh.sync()
    t0 = time.perf_counter()
    pf_ms, dec_ms = [], []
    for _ in range(args.steps):
        a, b = model.step(prompt, t_pf, t_dec)
        pf_ms.append(a)
        dec_ms.append(b)
    gh.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    # a generate call of N_NEW tokens runs N_NEW - 1 decode steps (the first id
    # comes from the prefill's logits); the CPU baseline counts the same steps
    decode_tps = (N_NEW - 1) * args.steps / (sum(dec_ms) * 1e-3)
    prefill_tps = PROMPT * args.steps / (sum(pf_ms) * 1e-3)
    ids_q4k = model.ids.copy()

    # Q8_0 (config 1 as written) beside it
    m8 = Model(gh, 2)
    for _ in range(max(1, args.warmup)):
        m8.step(prompt, t_pf, t_dec)
    d8, p8 = [], []
    for _ in range(args.steps):
        a, b = m8.step(prompt, t_pf, t_dec)
        p8.append(a)
        d8.append(b)

    # dominant decode kernel: the grouped expert GEMV (gate+up+SwiGLU) of the
    # c1 MoE layer at its real shape, launched alone
    run, bufs, out = moe_decode_case(gh, C1["d"], C1["E"], C1["ne"], C1["K"], C1["SH"], 3, N=1, seed=9)
    moe_ms = time_launches(gh, run, 200)
    del bufs, out
    # per-launch time of the c1 decode step's biggest GEMV (the Mamba in_proj 2192x512, Q4_K)
    proj = C1["d_inner"] * 2 + 2 * C1["m_dstate"] + C1["m_heads"]
    w = gh.quantize(3, gh.rng_normal(2, proj * C1["d"], 0, 0.02))
    dw, dx, dy = gh.Buf.from_array(w), gh.Buf.from_array(gh.rng_normal(3, C1["d"])), gh.Buf.zeros(proj, np.float32)
    inproj_ms = time_launches(gh, lambda: gh.call("gh_linear_forward_q4", dx.p, dw.p, dy.p, 1, C1["d"], proj, 3), 500)

    # c2 headline GEMV (Q4_K, 14336x4096, M=1) is the roofline object: cold (weights from HBM,
    # the headline) and warm (the same weights every launch, partly served by the MALL)
    run2, bufs2, gemv_bytes = roofline_gemv(gh, COLD_COPIES)
    gemv_ms = time_launches(gh, run2, 500)
    achieved = gemv_bytes / (gemv_ms * 1e-3) / 1e9
    del bufs2
    st_us, st_gbs, st_blocks = stream_ceiling(gh, 33030144)
    run_w, bufs_w, _ = roofline_gemv(gh, 1)
    warm_ms = time_launches(gh, run_w, 500)
    achieved_warm = gemv_bytes / (warm_ms * 1e-3) / 1e9
    del bufs_w

    kernels = {}
    if not args.no_kernels:
        kernels = kernel_suite(gh)
    kernels["c1_decode_moe_layer"] = entry("moe route+gemv x2+combine (c1)", moe_ms,
                                           bytes_=(2 * 3 * 256 * 512 + 3 * 512 * 512) * 144 // 256)
    kernels["c1_decode_inproj_gemv"] = entry("k_gemv_q4k_i8 (c1 mamba in_proj 2192x512)", inproj_ms,
                                             bytes_=w.nbytes + 512 * 4 + proj * 4)

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(prompt)
        except Exception as e:  # noqa
            cpu = {"value": None, "error": repr(e)}

    line = {
        "metric": "batch-1 decode tok/s + prefill tok/s (Q4_K hybrid); % HBM/MFMA roofline",
        "value": round(decode_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 activations, Q4_K weights (fp32 accumulate; fp16 MFMA operands in prefill)",
        "data": "synthetic (random-init weights by the seeded recipe, uniform prompt ids seed 1)",
        "config": {"workload": "benchmark configuration c1 tiny Granite-hybrid (V4096 d512 [M,M,A,M,M,A], MoE 8x top-2 + "
                               "shared) in Q4_K: 128-token prefill + 64 greedy tokens, decode "
                               + ("eager" if args.eager_decode else "graph-replayed"),
                   "global_batch": 1, "seq_len": PROMPT + N_NEW, "parallelism": "single GPU"},
        "prefill_tok_s": round(prefill_tps, 1),
        "decode_tok_s_q8_0": round((N_NEW - 1) * args.steps / (sum(d8) * 1e-3), 2),
        "prefill_tok_s_q8_0": round(PROMPT * args.steps / (sum(p8) * 1e-3), 1),
        "decode_ms_per_token": round(sum(dec_ms) / args.steps / (N_NEW - 1), 4),
        "roofline": {"bound": "hbm", "kernel": "k_gemv_q4k_i8 (BASELINE c2: 14336x4096, M=1)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "avg_launch_us": round(gemv_ms * 1e3, 3), "algorithmic_bytes": int(gemv_bytes),
                     "cache": f"cold: {COLD_COPIES} weight copies ({COLD_COPIES * gemv_bytes / 1e6:.0f} MB) in rotation",
                     "frac_cold": round(achieved / HBM_PEAK_GBS, 4),
                     "achieved_warm": round(achieved_warm, 1), "frac_warm": round(achieved_warm / HBM_PEAK_GBS, 4),
                     "avg_launch_us_warm": round(warm_ms * 1e3, 3),
                     "stream_ceiling": {"kernel": f"k_stream_read ({st_blocks} blocks x 256 lanes, 16-byte loads)",
                                        "bytes": 33030144 // 16 * 16, "us": round(st_us, 3),
                                        "GB_s": round(st_gbs, 1), "frac_of_peak": round(st_gbs / HBM_PEAK_GBS, 4),
                                        "cache": "cold: same 10-copy rotation"},
                     "frac_vs_stream_ceiling": round(achieved / st_gbs, 4)},
        "cpu_baseline": cpu,
        "kernels": kernels,
        "greedy_ids_head": ids_q4k[:8].tolist(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
