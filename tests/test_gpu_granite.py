"""End-to-end tiny Granite-hybrid: 128-token prompt, 64
greedy tokens, against the greedy ids and top-2 margins of the COMPILED
REFERENCE Generator (tests/golden/granite_c1_q8.npz). Ids must be identical
at every step up to the first step whose reference margin is <= 1e-3 (after
such a near-tie a different but equally valid choice changes the rest)."""
import ctypes as C
import hashlib

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden

pytestmark = pytest.mark.gpu
MARGIN = 1e-3


class Granite:
    def __init__(self, gh, c, qkind, max_ctx=256, seed=0):
        self.gh = gh
        cfg, fcfg = O.granite_cfg(c, qkind)
        self.c = c
        self.h = C.c_void_p()
        gh.call("gh_granite_create", cfg.ctypes.data_as(C.c_void_p), fcfg.ctypes.data_as(C.c_void_p), max_ctx,
                C.byref(self.h))
        gh.call("gh_granite_init_synthetic", self.h, C.c_uint64(seed))

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
