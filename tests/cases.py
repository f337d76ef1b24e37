"""Seeded input recipes shared by the GPU tests and the oracle fixture writer
(tests/golden/make_oracle_fixtures.py), so both see the same bytes."""
import numpy as np

import oracle_lib as O

# c1 with the Granite-4.0 fields a real checkpoint sets: an untied fp16 lm_head, per-layer
# aux-free router biases, embedding / residual multipliers and logits scaling
# (tests/golden/granite_c1_q8_opts.npz is the compiled reference Generator on it, Q8_0).
C1_OPTS = dict(O.C1, tied=0, aux_free=1, emb_mult=12.0, res_mult=0.22, logits_scaling=8.0)

# A small Granite hybrid with every optional field set, written to GGUF by the reference's own
# exporter (tests/golden/granite_small.gguf): the loader builds the model from its metadata.
G_SMALL = dict(V=256, d=256, L=2, H=4, KV=2, hd=64, E=128, ne=4, K=2, SH=128, d_inner=512, m_heads=8, m_dhead=64,
               m_dstate=64, conv_k=4, layer_types=[0, 1], eps=1e-5, scale=0.125, tied=0, aux_free=1, emb_mult=4.0,
               res_mult=0.5, logits_scaling=2.0)


def g_small_weights(qkind=2):
    """Synthetic weights of G_SMALL (the shared recipe, seed 3) with router biases N(0, 0.05)."""
    w = O.granite_weights(G_SMALL, qkind, seed=3)
    for layer in range(G_SMALL["L"]):
        w[f"layers.{layer}.moe_bias"] = O.rng_normal(95 + layer, G_SMALL["ne"], 0, 0.05)
    return w


def granite_opts_weights(qkind=2):
    """Synthetic weights of C1_OPTS (the shared recipe) with router biases N(0, 0.05)
    (seeds 90 + layer) in place of the recipe's zeros."""
    w = O.granite_weights(C1_OPTS, qkind, seed=0)
    for layer in range(C1_OPTS["L"]):
        w[f"layers.{layer}.moe_bias"] = O.rng_normal(90 + layer, C1_OPTS["ne"], 0, 0.05)
    return w


# benchmark configuration c1 benched workload (bench.py): 128-token prompt + 64 greedy tokens.
C1_PROMPT, C1_NEW, C1_MAX_CTX = 128, 64, 256

# benchmark configuration c3: Mamba-2 layer, Q4_K, 4096-token prompt then 512 decode steps.
C3 = dict(d=1536, d_inner=3072, heads=48, d_head=64, d_state=128, conv_k=4, T=4096, steps=512)
C3_STEP_CHECKS = (0, 1, 2, 7, 63, 255, 511)


def c3_layer_weights(seed=30):
    """Weights of the c3 layer (matrices N(0,0.02) in Q4_K, conv N(0,0.3)/N(0,0.1),
    dt_bias 0, A_log U[0, ln 16], D 1, norm 1), as in the other Mamba tests."""
    s = C3
    d, di, nh, ds, k = s["d"], s["d_inner"], s["heads"], s["d_state"], s["conv_k"]
    conv_dim = di + 2 * ds
    proj = di + conv_dim + nh
    w_in = O.quantize(3, O.rng_normal(seed, proj * d, 0, 0.02))
    w_out = O.quantize(3, O.rng_normal(seed + 1, d * di, 0, 0.02))
    conv_w = O.rng_normal(seed + 2, conv_dim * k, 0, 0.3)
    conv_b = O.rng_normal(seed + 3, conv_dim, 0, 0.1)
    dt_bias = np.zeros(nh, np.float32)
    a_log = O.rng_uniform(seed + 4, nh, 0.0, np.log(16.0))
    D = np.ones(nh, np.float32)
    norm_w = np.ones(di, np.float32)
    return [w_in, conv_w, conv_b, dt_bias, a_log, D, norm_w, w_out], conv_dim


def c3_prompt():
    """Hidden states of the 4096-token prompt, N(0,1) (seed 3)."""
    return O.rng_normal(3, C3["T"] * C3["d"])


def c3_step_inputs():
    """The 512 decode tokens' hidden states, N(0,1) (seed 33), [steps, d]."""
    return O.rng_normal(33, C3["steps"] * C3["d"]).reshape(C3["steps"], C3["d"])


def c3_window(w, x, conv_dim):
    """The decode conv window after the prompt: raw (pre-conv) xBC projections
    of its last k-1 tokens, [conv_dim, k-1] oldest first, by the oracle's
    quantized linear (inference/generator.cpp:510-616 keeps raw in_proj rows)."""
    s = C3
    d, di, k = s["d"], s["d_inner"], s["conv_k"]
    proj = di + conv_dim + s["heads"]
    last = np.ascontiguousarray(x.reshape(s["T"], d)[-(k - 1):])
    pr = O.linear_q(last, w[0], k - 1, d, proj, 3)
    return np.ascontiguousarray(pr[:, di:di + conv_dim].T, np.float32).ravel()


def c3_sample_rows():
    return np.array([0, 1, 255, 256, 257, 1000, 2047, 2048, 3071, 4094, 4095])


def c3_state_sample():
    n = C3["heads"] * C3["d_head"] * C3["d_state"]
    return np.unique(O.rng_below(77, 16384, n)).astype(np.int64)
