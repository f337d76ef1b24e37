"""End-to-end tiny Granite-hybrid (benchmark configuration c1): 128-token prompt, 64
greedy tokens, against the greedy ids and top-2 margins of the COMPILED
REFERENCE Generator (tests/golden/granite_c1_q8.npz). Ids must be identical
at every step up to the first step whose reference margin is <= 1e-3 (after
such a near-tie a different but equally valid choice changes the rest)."""
import ctypes as C
import hashlib

import numpy as np
import pytest

import oracle_lib as O
from conftest import close, golden

pytestmark = pytest.mark.gpu
MARGIN = 1e-3


class Granite:
    def __init__(self, gh, c, qkind, max_ctx=256, seed=0, weights=None):
        self.gh = gh
        cfg, fcfg = O.granite_cfg(c, qkind)
        self.c = c
        self.h = C.c_void_p()
        if O.has_options(c):
            gh.call("gh_granite_create_ex", cfg.ctypes.data_as(C.c_void_p), len(cfg), fcfg.ctypes.data_as(C.c_void_p),
                    len(fcfg), max_ctx, C.byref(self.h))
        else:
            gh.call("gh_granite_create", cfg.ctypes.data_as(C.c_void_p), fcfg.ctypes.data_as(C.c_void_p), max_ctx,
                    C.byref(self.h))
        gh.call("gh_granite_init_synthetic", self.h, C.c_uint64(seed))
        for name, arr in (weights or {}).items():
            arr = np.ascontiguousarray(arr)
            gh.call("gh_granite_set_param", self.h, name.encode(), arr.ctypes.data_as(C.c_void_p),
                    C.c_size_t(arr.nbytes))

    def teacher_forced(self, prompt, feed, mamba_mode=1):
        """Prefill, then one decode step per id of `feed`: the logits before each step
        (len(feed) + 1 rows)."""
        gh = self.gh
        gh.call("gh_granite_reset", self.h)
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros((len(feed) + 1, self.c["V"]), np.float32)
        gh.call("gh_granite_prefill", self.h, prompt.ctypes.data_as(C.c_void_p), len(prompt),
                out[0].ctypes.data_as(C.c_void_p), mamba_mode)
        for s, tok in enumerate(feed):
            gh.call("gh_granite_decode", self.h, int(tok), out[s + 1].ctypes.data_as(C.c_void_p))
        return out

    def weights_sha(self):
        lib = self.gh.load()
        n = lib.gh_granite_param_count(self.h)
        items = {}
        for i in range(n):
            name, nb = C.c_char_p(), C.c_size_t()
            self.gh.call("gh_granite_param_name", self.h, i, C.byref(name), C.byref(nb))
            buf = np.empty(nb.value, np.uint8)
            self.gh.call("gh_granite_get_param", self.h, name, buf.ctypes.data_as(C.c_void_p), nb)
            items[name.value.decode()] = buf
        h = hashlib.sha256()
        for k in sorted(items):
            h.update(k.encode())
            h.update(items[k].tobytes())
        return h.hexdigest()

    def generate(self, prompt, n_new, mamba_mode, use_graph):
        gh = self.gh
        gh.call("gh_granite_reset", self.h)
        prompt = np.ascontiguousarray(prompt, np.int32)
        logits = np.zeros(self.c["V"], np.float32)
        gh.call("gh_granite_prefill", self.h, prompt.ctypes.data_as(C.c_void_p), len(prompt),
                logits.ctypes.data_as(C.c_void_p), mamba_mode)
        ids = np.zeros(n_new, np.int32)
        gh.call("gh_granite_generate_greedy", self.h, n_new, ids.ctypes.data_as(C.c_void_p), int(use_graph))
        return ids, logits

    def close(self):
        self.gh.call("gh_granite_destroy", self.h)


def compare(ids, ref_ids, ref_margins):
    n = 0
    for i in range(len(ref_ids)):
        assert ids[i] == ref_ids[i], f"step {i}: {ids[i]} != {ref_ids[i]} (margin {ref_margins[i]:.4g})"
        n += 1
        if ref_margins[i] <= MARGIN:
            break
    return n


@pytest.fixture(scope="module")
def model(gh):
    m = Granite(gh, O.C1, 2)
    yield m
    m.close()


def test_weights_match_fixture(model):
    g = golden("granite_c1_q8")
    assert model.weights_sha() == str(g["weights_sha256"])


@pytest.mark.parametrize("mamba_mode,use_graph", [(0, 0), (1, 0), (1, 1), (1, 2)])
def test_greedy_ids_match_reference(model, mamba_mode, use_graph):
    g = golden("granite_c1_q8")
    ids, _ = model.generate(g["prompt"], int(g["n_new"]), mamba_mode, use_graph)
    n = compare(ids, g["ids"], g["margins"])
    assert n >= 8


def test_graph_replay_equals_eager(model):
    g = golden("granite_c1_q8")
    a, la = model.generate(g["prompt"], 24, 1, False)
    b, lb = model.generate(g["prompt"], 24, 1, True)
    c, lc = model.generate(g["prompt"], 24, 1, True)  # replays the already captured graph
    assert np.array_equal(a, b) and np.array_equal(a, c)
    assert np.array_equal(la, lb)


def test_graph_recaptured_after_workspace_growth(gh):
    """A longer prefill after the decode graph was captured grows backend workspaces the
    graph reads (the MoE routing slots among them); the next generate must capture again
    rather than replay stale addresses: ids equal eager decode on the same prompt."""
    gh.call("gh_free_workspace")  # every workspace starts small (other models' graphs recapture too)
    m = Granite(gh, O.C1, 3, max_ctx=256)
    try:
        short = O.rng_below(5, 8, 4096)
        long_ = O.rng_below(6, 160, 4096)
        m.generate(short, 6, 1, 1)  # captures the graph with small workspaces
        a, _ = m.generate(long_, 24, 1, 1)
        b, _ = m.generate(long_, 24, 1, 0)
        assert np.array_equal(a, b)
    finally:
        m.close()


def test_persistent_decode_equals_graph(model):
    """use_graph=2: the whole decode loop in one cooperative launch gives the ids
    of graph replay, twice in a row (the hand-over buffers are re-zeroed per call)."""
    g = golden("granite_c1_q8")
    a, _ = model.generate(g["prompt"], 40, 1, 1)
    b, _ = model.generate(g["prompt"], 40, 1, 2)
    c, _ = model.generate(g["prompt"], 40, 1, 2)
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_q4k_model_runs_and_matches_oracle(gh):
    """The Q4_K variant of the c1 model (the metric's weight format): greedy ids
    against the oracle generator (the reference has no Q4_K)."""
    c = dict(O.C1)
    m = Granite(gh, c, 3)
    try:
        prompt = O.rng_below(1, 64, 4096)
        ids, _ = m.generate(prompt, 12, 1, True)
        w = O.granite_weights(c, 3)
        r_ids, r_m = O.granite_generate(O.oracle().orc_granite_generate, c, 3, w, prompt, 12)
        assert compare(ids, r_ids, r_m) >= min(4, expected_matches(r_m))
    finally:
        m.close()


def expected_matches(margins):
    """Number of ids the comparison must cover: up to and including the first
    step whose oracle top-2 margin is <= MARGIN."""
    small = np.nonzero(np.asarray(margins) <= MARGIN)[0]
    return int(small[0]) + 1 if small.size else len(margins)


@pytest.mark.parametrize("use_graph", [0, 1, 2])
def test_q4k_benched_workload_vs_oracle(gh, use_graph):
    """The bench's headline workload: c1 in Q4_K, 128-token prompt (seed 1) and
    64 greedy tokens, SSD prefill, decode eager, graph-replayed and persistent. Ids against
    the oracle generator's run of the same workload
    (tests/golden/granite_c1_q4k_oracle.npz) up to its first near-tie."""
    import cases
    g = golden("granite_c1_q4k_oracle")
    assert np.array_equal(g["prompt"], O.rng_below(1, cases.C1_PROMPT, 4096))
    m = Granite(gh, O.C1, 3, max_ctx=cases.C1_MAX_CTX)
    try:
        ids, _ = m.generate(g["prompt"], cases.C1_NEW, 1, use_graph)
        assert compare(ids, g["ids"], g["margins"]) == expected_matches(g["margins"])
    finally:
        m.close()


def test_bench_greedy_ids_match_oracle(gh):
    """bench.py's own Model/step (the timed object) produces the oracle's ids on
    the benched workload, so its greedy_ids_head is checked, not just printed."""
    import os
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    import cases
    g = golden("granite_c1_q4k_oracle")
    assert (bench.PROMPT, bench.N_NEW, bench.MAX_CTX) == (cases.C1_PROMPT, cases.C1_NEW, cases.C1_MAX_CTX)
    model = bench.Model(gh, 3)
    try:
        prompt = gh.rng_below(1, bench.PROMPT, bench.C1["V"])
        model.step(prompt, gh.Timer(), gh.Timer())
        model.step(prompt, gh.Timer(), gh.Timer())  # second step replays the captured graph
        assert compare(model.ids, g["ids"], g["margins"]) == expected_matches(g["margins"])
    finally:
        gh.call("gh_granite_destroy", model.h)


def test_q4k_model_long_context(gh):
    """Q4_K, two attention layers of the c1 shape over a 700-token prompt: the
    decode attention splits the context into more chunks than the merge
    prologue of the output projection keeps in registers."""
    c = dict(O.C1)
    c.update(L=2, layer_types=[1, 1])
    m = Granite(gh, c, 3, max_ctx=1024)
    try:
        prompt = O.rng_below(2, 700, 4096)
        ids, _ = m.generate(prompt, 10, 1, True)
        w = O.granite_weights(c, 3)
        r_ids, r_m = O.granite_generate(O.oracle().orc_granite_generate, c, 3, w, prompt, 10, max_ctx=1024)
        assert compare(ids, r_ids, r_m) >= min(4, expected_matches(r_m))
    finally:
        m.close()


@pytest.mark.parametrize("qkind,prompt_len,n_new", [(2, 440, 16), (3, 440, 16), (2, 860, 24), (3, 860, 24)])
def test_persistent_long_context(gh, qkind, prompt_len, n_new):
    """use_graph=2 near the persistent kernel's limits: 7-14 attention position splits, so
    the merge phase waits on up to H * 14 * (hd + 2) partial words (more than one staging
    window of the hand-over wait). Ids equal graph replay."""
    m = Granite(gh, O.C1, qkind, max_ctx=1024)
    try:
        prompt = O.rng_below(7, prompt_len, 4096)
        a, _ = m.generate(prompt, n_new, 1, 1)
        b, _ = m.generate(prompt, n_new, 1, 2)
        assert np.array_equal(a, b)
    finally:
        m.close()


def test_persistent_unsupported_falls_back(gh):
    """A context whose attention partials exceed the persistent kernel's LDS area
    (1000 + 8 positions: 16 splits) makes use_graph=2 fall back to graph replay: same ids."""
    m = Granite(gh, O.C1, 3, max_ctx=1024)
    try:
        prompt = O.rng_below(8, 1000, 4096)
        a, _ = m.generate(prompt, 8, 1, 1)
        b, _ = m.generate(prompt, 8, 1, 2)
        assert np.array_equal(a, b)
    finally:
        m.close()


def test_persistent_abort_leaves_model_refusing_until_reset(gh):
    """The abort contract, forced from the host (the launch starts with its abort flag
    raised; every wait that misses returns, so the kernel ends normally): generate fails,
    the model then refuses decode / generate / prefill, and after a reset it decodes the
    same ids as before."""
    lib = gh.load()
    m = Granite(gh, O.C1, 3, max_ctx=256)
    try:
        prompt = np.ascontiguousarray(O.rng_below(9, 64, 4096), np.int32)
        ref, _ = m.generate(prompt, 12, 1, 1)
        gh.call("gh_granite_reset", m.h)
        gh.call("gh_granite_prefill", m.h, prompt.ctypes.data_as(C.c_void_p), len(prompt), None, 1)
        gh.call("gh_granite_test_force_abort", m.h)
        ids = np.zeros(12, np.int32)
        rc = lib.gh_granite_generate_greedy(m.h, 12, ids.ctypes.data_as(C.c_void_p), 2)
        assert rc != 0 and b"aborted" in lib.gh_last_error()
        rc = lib.gh_granite_generate_greedy(m.h, 2, ids.ctypes.data_as(C.c_void_p), 1)
        assert rc != 0 and b"invalid" in lib.gh_last_error()
        assert lib.gh_granite_decode(m.h, 5, None) != 0
        gh.call("gh_granite_reset", m.h)
        again, _ = m.generate(prompt, 12, 1, 2)
        assert np.array_equal(again, ref)
    finally:
        m.close()


def check_forced(logits, ref_logits, ref_ids, ref_margins, tol=1e-3):
    """Per step: logits within tol normwise of the reference's, and the argmax equal to
    the reference's greedy id wherever its top-2 margin exceeds MARGIN."""
    for s in range(len(ref_ids)):
        assert close(logits[s], ref_logits[s], tol), f"step {s}"
        if ref_margins[s] > MARGIN:
            assert int(np.argmax(logits[s])) == int(ref_ids[s]), f"step {s}: margin {ref_margins[s]:.3g}"


@pytest.mark.parametrize("mamba_mode", [0, 1])
def test_granite_options_teacher_forced_vs_reference(gh, mamba_mode):
    """Untied lm_head, aux-free router biases, embedding x12, residual x0.22, logits / 8
    (c1 shape, Q8_0): every step's logits against the compiled reference Generator's
    (tests/golden/granite_c1_q8_opts.npz), feeding the reference's ids, all 24 steps."""
    import cases
    g = golden("granite_c1_q8_opts")
    m = Granite(gh, cases.C1_OPTS, 2, max_ctx=int(g["max_ctx"]), weights=cases.granite_opts_weights())
    try:
        lg = m.teacher_forced(g["prompt"], g["ids"][:-1], mamba_mode)
        check_forced(lg, g["logits"], g["ids"], g["margins"])
    finally:
        m.close()


@pytest.mark.parametrize("use_graph", [0, 1, 2])
def test_granite_options_greedy_vs_reference(gh, use_graph):
    """The same model free-running: greedy ids equal the reference's up to its first
    near-tie, eager, graph-replayed and persistent (which falls back to the graph for
    these options)."""
    import cases
    g = golden("granite_c1_q8_opts")
    m = Granite(gh, cases.C1_OPTS, 2, max_ctx=int(g["max_ctx"]), weights=cases.granite_opts_weights())
    try:
        ids, _ = m.generate(g["prompt"], int(g["n_new"]), 1, use_graph)
        assert compare(ids, g["ids"], g["margins"]) == expected_matches(g["margins"])
    finally:
        m.close()


@pytest.mark.parametrize("qkind", [2, 3])
def test_granite_bias_untied_fused_vs_oracle(gh, qkind):
    """Untied lm_head and router biases with unit multipliers: the decode step stays on the
    fused launches (router bias inside the fused MoE, the untied head in the one-launch
    tail). Teacher-forced logits against the oracle (pinned to the reference above)."""
    import cases
    c = dict(O.C1, tied=0, aux_free=1)
    w = O.granite_weights(c, qkind)
    for layer in range(c["L"]):
        w[f"layers.{layer}.moe_bias"] = O.rng_normal(90 + layer, c["ne"], 0, 0.05)
    prompt = O.rng_below(12, 40, 4096)
    r_ids, r_m, r_lg = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, c, qkind, w, prompt, 16, max_ctx=96,
                                             logits=True)
    m = Granite(gh, c, qkind, max_ctx=96, weights=w)
    try:
        lg = m.teacher_forced(prompt, r_ids[:-1])
        check_forced(lg, r_lg, r_ids, r_m)
        ids, _ = m.generate(prompt, 16, 1, 1)
        assert compare(ids, r_ids, r_m) == expected_matches(r_m)
    finally:
        m.close()


def test_q4k_benched_workload_teacher_forced(gh):
    """The benched workload (c1 Q4_K, 128-token prompt, 64 tokens) teacher-forced with the
    oracle's ids: all 64 steps' logits within 1e-3 of the oracle's and the argmax equal
    wherever the oracle's margin exceeds 1e-3 (free-running comparisons stop at the first
    near-tie, step 11)."""
    import cases
    g = golden("granite_c1_q4k_oracle")
    w = O.granite_weights(O.C1, 3)
    r_ids, r_m, r_lg = O.granite_generate_ex(O.oracle().orc_granite_generate_ex, O.C1, 3, w, g["prompt"],
                                             cases.C1_NEW, max_ctx=cases.C1_MAX_CTX, logits=True)
    assert np.array_equal(r_ids, g["ids"])
    m = Granite(gh, O.C1, 3, max_ctx=cases.C1_MAX_CTX)
    try:
        lg = m.teacher_forced(g["prompt"], r_ids[:-1])
        check_forced(lg, r_lg, r_ids, r_m)
    finally:
        m.close()
