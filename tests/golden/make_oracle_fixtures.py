"""Writes oracle fixtures for workloads whose CPU oracle run is too long for a
GPU test (the oracle restates the reference's CPU path, which dequantises
whole tensors on every call, core/ops.cpp:304-347):

  granite_c1_q4k_oracle.npz  benchmark configuration c1 in Q4_K at the benched workload:
                             128-token prompt (seed 1) + 64 greedy tokens; ids
                             and top-2 margins of orc_granite_generate.
  mamba_c3_decode_oracle.npz benchmark configuration c3: the Q4_K layer over a 4096-token
                             prompt from a zero state (orc_mamba2_forward_q),
                             then 512 single-token steps (orc_mamba2_step_q,
                             the restatement of inference/generator.cpp:510-616)
                             from the state the prompt left and the raw xBC
                             window of its last 3 tokens. Stored: sampled rows of
                             the prompt output, a sample of the state, the step
                             outputs at a few indices, the final conv window and
                             a state sample after the last step.

The inputs are regenerated from their seeds by the tests (the shared seeded
generators), so only outputs are stored. The oracle itself is pinned against
the compiled reference by tests/golden/*.npz (tests/test_oracle_golden.py).

    python tests/golden/make_oracle_fixtures.py [c1] [c3]
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402
import cases  # noqa: E402


def save(name, **arrs):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items()}, flush=True)


def c1_q4k():
    c = O.C1
    prompt = O.rng_below(1, cases.C1_PROMPT, c["V"])
    w = O.granite_weights(c, 3)
    t0 = time.time()
    ids, margins = O.granite_generate(O.oracle().orc_granite_generate, c, 3, w, prompt, cases.C1_NEW,
                                      max_ctx=cases.C1_MAX_CTX)
    print(f"c1 q4k oracle generate: {time.time() - t0:.1f} s", flush=True)
    save("granite_c1_q4k_oracle", prompt=prompt, ids=ids, margins=margins)


def c3_decode():
    s = cases.C3
    d, di, nh, dh, ds, k, T = s["d"], s["d_inner"], s["heads"], s["d_head"], s["d_state"], s["conv_k"], s["T"]
    w, conv_dim = cases.c3_layer_weights()
    x = cases.c3_prompt()
    st = np.zeros(nh * dh * ds, np.float32)
    out = np.zeros(T * d, np.float32)
    t0 = time.time()
    assert O.oracle().orc_mamba2_forward_q(O.P(x), *[O.P(a) for a in w[:-1]], O.P(w[-1]), O.P(st), O.P(out), 1, T,
                                           d, di, conv_dim, nh, dh, ds, k, O.f(1e-5), 3) == 0
    print(f"c3 forward T={T}: {time.time() - t0:.1f} s", flush=True)
    conv = cases.c3_window(w, x, conv_dim)
    prompt_state = st.copy()
    outs = {}
    t0 = time.time()
    xs = cases.c3_step_inputs()
    o = np.zeros(d, np.float32)
    for i in range(s["steps"]):
        assert O.oracle().orc_mamba2_step_q(O.P(np.ascontiguousarray(xs[i])), *[O.P(a) for a in w], O.P(conv),
                                            O.P(st), O.P(o), d, di, conv_dim, nh, dh, ds, k, O.f(1e-5), 3) == 0
        if i in cases.C3_STEP_CHECKS:
            outs[i] = o.copy()
    print(f"c3 {s['steps']} steps: {time.time() - t0:.1f} s", flush=True)
    rows, sidx = cases.c3_sample_rows(), cases.c3_state_sample()
    save("mamba_c3_decode_oracle", prompt_out_rows=out.reshape(T, d)[rows], prompt_state_sample=prompt_state[sidx],
         step_out=np.stack([outs[i] for i in cases.C3_STEP_CHECKS]), final_conv=conv, final_state_sample=st[sidx])


if __name__ == "__main__":
    which = sys.argv[1:] or ["c1", "c3"]
    if "c1" in which:
        c1_q4k()
    if "c3" in which:
        c3_decode()
