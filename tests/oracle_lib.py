"""ctypes loader for the CPU oracle (oracle/liboracle.so) and, in the build
container only, the compiled reference (oracle/_ref/libgai_ref.so).

Test infrastructure: the oracle is the checker, never the thing measured.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libgai_ref.so")

# Tiny Granite-hybrid (benchmark configuration c1) in the oracle's int layout.
C1 = dict(V=4096, d=512, L=6, H=8, KV=2, hd=64, E=256, ne=8, K=2, SH=512, d_inner=1024,
          m_heads=16, m_dhead=64, m_dstate=64, conv_k=4, layer_types=[0, 0, 1, 0, 0, 1],
          eps=1e-5, scale=0.125)


OPTION_KEYS = ("tied", "aux_free", "emb_mult", "res_mult", "logits_scaling")


def has_options(c):
    return any(k in c for k in OPTION_KEYS)


def granite_cfg(c, qkind):
    """(ints, floats) of a config. With any of the optional Granite fields in c
    (tied, aux_free, emb_mult, res_mult, logits_scaling) both arrays carry the
    extended layout: ints + [tied, aux_free], floats + [emb, res, logits]."""
    ints = [c["V"], c["d"], c["L"], c["H"], c["KV"], c["hd"], c["E"], c["ne"], c["K"], c["SH"],
            c["d_inner"], c["m_heads"], c["m_dhead"], c["m_dstate"], c["conv_k"], qkind] + list(c["layer_types"])
    fl = [c["eps"], c["scale"]]
    if has_options(c):
        ints += [int(c.get("tied", 1)), int(c.get("aux_free", 0))]
        fl += [c.get("emb_mult", 1.0), c.get("res_mult", 1.0), c.get("logits_scaling", 1.0)]
    return np.array(ints, dtype=np.int32), np.array(fl, dtype=np.float32)


def P(a):
    """numpy array -> void pointer (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
    lib = C.CDLL(path)
    return lib


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        lib = _load(ORACLE_SO)
        lib.orc_fnv1a64.restype = C.c_uint64
        lib.orc_quant_row_bytes.restype = C.c_int64
        lib.orc_dot_f32.restype = C.c_float
        lib.orc_argmax_token.restype = C.c_int32
        for fn in ("orc_rng_normal", "orc_rng_uniform"):
            getattr(lib, fn).argtypes = [C.c_uint64, C.c_float, C.c_float, C.c_void_p, C.c_int64]
        lib.orc_rng_below.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_int64]
        lib.orc_synth_param_f32.argtypes = [C.c_char_p, C.c_uint64, C.c_void_p, C.c_int64]
        _oracle = lib
    return _oracle


_ref = None


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        lib = _load(REF_SO)
        for fn in ("ref_rng_normal", "ref_rng_uniform"):
            getattr(lib, fn).argtypes = [C.c_uint64, C.c_float, C.c_float, C.c_void_p, C.c_int64]
        lib.ref_rng_below.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_int64]
        lib.ref_argmax_token.restype = C.c_int32
        _ref = lib
    return _ref


# ------------------------------------------------------------------ helpers
def f(x):
    return C.c_float(x)


def rng_normal(seed, n, mean=0.0, sd=1.0):
    out = np.empty(n, np.float32)
    oracle().orc_rng_normal(seed, mean, sd, P(out), n)
    return out


def rng_uniform(seed, n, lo=0.0, hi=1.0):
    out = np.empty(n, np.float32)
    oracle().orc_rng_uniform(seed, lo, hi, P(out), n)
    return out


def rng_below(seed, n, bound):
    out = np.empty(n, np.int32)
    oracle().orc_rng_below(seed, bound, P(out), n)
    return out


BLOCK = {0: (32, 18), 1: (32, 20), 2: (32, 34), 3: (256, 144)}


def qbytes(kind, n):
    bv, bb = BLOCK[kind]
    return (n + bv - 1) // bv * bb


def quantize(kind, x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(qbytes(kind, x.size), np.uint8)
    assert oracle().orc_quantize(kind, P(x), P(out), C.c_int64(x.size)) == 0
    return out


def dequantize(kind, q, n):
    out = np.empty(n, np.float32)
    assert oracle().orc_dequantize(kind, P(q), P(out), C.c_int64(n)) == 0
    return out


def materialize(kind, q, n):
    out = np.empty(n, np.uint16)
    assert oracle().orc_quant_materialize(kind, P(q), P(out), C.c_int64(n)) == 0
    return out


def linear_q(x, w, M, K, N, kind):
    y = np.empty(M * N, np.float32)
    assert oracle().orc_linear_forward_q4(P(x), P(w), P(y), M, K, N, kind) == 0
    return y.reshape(M, N)


def f16_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.size, np.float32)
    oracle().orc_f16_to_f32(P(h), P(out), C.c_int64(h.size))
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint16)
    oracle().orc_f32_to_f16(P(x), P(out), C.c_int64(x.size))
    return out


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint16)
    oracle().orc_f32_to_bf16(P(x), P(out), C.c_int64(x.size))
    return out


def synth_param(name, numel, seed=0):
    out = np.empty(numel, np.float32)
    oracle().orc_synth_param_f32(name.encode(), seed, P(out), numel)
    return out


def granite_param_specs(c):
    """(name, numel, storage) of the reference Model's parameters for config c
    (model/model.cpp:1087-1160). storage: 'q' packed, 'f16', 'f32'."""
    d, E, ne, SH = c["d"], c["E"], c["ne"], c["SH"]
    qd, kvd = c["H"] * c["hd"], c["KV"] * c["hd"]
    di, mh, ds, ck = c["d_inner"], c["m_heads"], c["m_dstate"], c["conv_k"]
    conv_dim = di + 2 * ds
    proj = di + conv_dim + mh
    specs = [("tok_embeddings", c["V"] * d, "f16")]
    for i, lt in enumerate(c["layer_types"]):
        pre = f"layers.{i}."
        specs += [(pre + "attn_norm", d, "f32"), (pre + "ffn_norm", d, "f32")]
        if lt == 0:
            mp = pre + "mamba."
            specs += [(mp + "in_proj", proj * d, "q"), (mp + "conv1d.weight", conv_dim * ck, "f32"),
                      (mp + "conv1d.bias", conv_dim, "f32"), (mp + "dt_bias", mh, "f32"),
                      (mp + "A_log", mh, "f32"), (mp + "D", mh, "f32"), (mp + "norm.weight", di, "f32"),
                      (mp + "out_proj", d * di, "q")]
        else:
            specs += [(pre + "wq", qd * d, "q"), (pre + "wk", kvd * d, "q"), (pre + "wv", kvd * d, "q"),
                      (pre + "wo", d * qd, "q")]
        specs += [(pre + "moe_router", ne * d, "f32"), (pre + "moe_gate", ne * E * d, "q"),
                  (pre + "moe_up", ne * E * d, "q"), (pre + "moe_down", ne * d * E, "q"),
                  (pre + "moe_sh_gate", SH * d, "q"), (pre + "moe_sh_up", SH * d, "q"),
                  (pre + "moe_sh_down", d * SH, "q")]
        if c.get("aux_free", 0):
            specs.append((pre + "moe_bias", ne, "f32"))
    specs.append(("final_norm", d, "f32"))
    if not c.get("tied", 1):
        specs.append(("lm_head", c["V"] * d, "f16"))
    return specs


def granite_weights(c, qkind, seed=0):
    """Synthetic storage bytes for every parameter, by the shared recipe."""
    out = {}
    for name, n, st in granite_param_specs(c):
        w = synth_param(name, n, seed)
        if st == "q":
            out[name] = quantize(qkind, w)
        elif st == "f16":
            out[name] = f32_to_f16(w)
        else:
            out[name] = w
    return out


def _param_arrays(weights):
    names = list(weights.keys())
    arr_names = (C.c_char_p * len(names))(*[n.encode() for n in names])
    arr_ptrs = (C.c_void_p * len(names))(*[weights[n].ctypes.data for n in names])
    return arr_names, arr_ptrs, len(names)


def granite_generate_ex(lib_fn, c, qkind, weights, prompt, n_new, max_ctx=256, forced=None, logits=False):
    """orc_granite_generate_ex / ref_granite_generate_ex: (ids, margins, logits or None).
    forced: ids fed at each step instead of the greedy ones (teacher forcing)."""
    cfg, fcfg = granite_cfg(c, qkind)
    names, ptrs, n = _param_arrays(weights)
    prompt = np.ascontiguousarray(prompt, np.int32)
    ids = np.zeros(n_new, np.int32)
    margins = np.zeros(n_new, np.float32)
    lg = np.zeros((n_new, c["V"]), np.float32) if logits else None
    fo = None if forced is None else np.ascontiguousarray(forced, np.int32)
    rc = lib_fn(P(cfg), len(cfg), P(fcfg), len(fcfg), names, ptrs, n, P(prompt), len(prompt), n_new, max_ctx, P(fo),
                P(ids), P(margins), P(lg), None)
    assert rc == 0, rc
    return ids, margins, lg


def granite_generate(lib_fn, c, qkind, weights, prompt, n_new, max_ctx=256):
    cfg, fcfg = granite_cfg(c, qkind)
    names, ptrs, n = _param_arrays(weights)
    prompt = np.ascontiguousarray(prompt, np.int32)
    ids = np.zeros(n_new, np.int32)
    margins = np.zeros(n_new, np.float32)
    rc = lib_fn(P(cfg), P(fcfg), names, ptrs, n, P(prompt), len(prompt), n_new, max_ctx, P(ids), P(margins))
    assert rc == 0, rc
    return ids, margins
