"""GGUF into the device: packed Q4_K / Q8_0 blocks go from the file straight
into device buffers, and a whole Granite model loaded from a GGUF file
(gh_granite_load_gguf) holds the same bytes and generates the same ids as the
one built from the same weights in memory."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden
from test_gguf import GT, check, open_file, write
from test_gpu_granite import Granite

pytestmark = pytest.mark.gpu


def row_len(c, name):
    """Values per row (GGUF innermost dimension) of a packed parameter."""
    d, qd = c["d"], c["H"] * c["hd"]
    last = name.split(".")[-1]
    return {"out_proj": c["d_inner"], "wo": qd, "moe_down": c["E"], "moe_sh_down": c["SH"]}.get(last, d)


def model_tensors(c, qkind):
    w = O.granite_weights(c, qkind)
    out = []
    for name, n, st in O.granite_param_specs(c):
        if st == "q":
            k = row_len(c, name)
            out.append((name, GT["Q4_K"] if qkind == 3 else GT["Q8_0"], [k, n // k], w[name]))
        elif st == "f16":
            out.append((name, GT["F16"], [c["d"], n // c["d"]], w[name]))
        else:
            out.append((name, GT["F32"], [n], w[name]))
    return out


@pytest.mark.parametrize("qkind", [3, 2])
def test_granite_from_gguf(gh, tmp_path, qkind):
    lib = gh.load()
    lib.gh_gguf_find_tensor.restype = C.c_int64
    lib.gh_gguf_find_tensor.argtypes = [C.c_void_p, C.c_char_p]
    c = dict(O.C1)
    path = str(tmp_path / "c1.gguf")
    tensors = model_tensors(c, qkind)
    write(lib, path, tensors, [("general.architecture", 8, "ghassan")])
    f = open_file(lib, path)
    a = Granite(gh, c, qkind)
    b = Granite(gh, c, qkind, seed=1)  # other weights until the file is loaded
    try:
        # packed blocks into device memory, verbatim
        name, _, _, wq = next(t for t in tensors if t[0].endswith("mamba.in_proj"))
        dev = gh.Buf.zeros(wq.nbytes, np.uint8)
        check(lib, lib.gh_gguf_read_packed(f, name.encode(), qkind, dev.p, 1, C.c_size_t(wq.nbytes)))
        assert np.array_equal(dev.numpy(np.uint8), wq.view(np.uint8))
        assert a.weights_sha() != b.weights_sha()
        gh.call("gh_granite_load_gguf", b.h, f)
        assert a.weights_sha() == b.weights_sha()
        prompt = O.rng_below(1, 32, c["V"])
        ia, _ = a.generate(prompt, 8, 1, True)
        ib, _ = b.generate(prompt, 8, 1, True)
        assert np.array_equal(ia, ib)
    finally:
        a.close()
        b.close()
        lib.gh_gguf_close(f)


def test_load_gguf_shape_mismatch(gh, tmp_path):
    lib = gh.load()
    c = dict(O.C1)
    tensors = model_tensors(c, 3)
    i = next(k for k, t in enumerate(tensors) if t[0] == "final_norm")
    tensors[i] = ("final_norm", GT["F32"], [c["d"] - 8], tensors[i][3][: c["d"] - 8].copy())
    path = str(tmp_path / "bad.gguf")
    write(lib, path, tensors, [])
    f = open_file(lib, path)
    m = Granite(gh, c, 3)
    try:
        with pytest.raises(gh.GHError, match="final_norm has 504 values"):
            gh.call("gh_granite_load_gguf", m.h, f)
    finally:
        m.close()
        lib.gh_gguf_close(f)


@pytest.mark.parametrize("use_graph", [0, 1])
def test_open_reference_gguf_generates_reference_ids(gh, use_graph):
    """A file the compiled reference exported (export_model_gguf, hybrid profile: Q8_0 matrices,
    F16 in_proj, F32 vectors, untied lm_head, router biases, Granite multipliers), opened with
    gh_granite_open_gguf alone (configuration from its metadata, then every weight): the greedy
    ids equal those the reference generated after its own load_model_from_gguf of the same
    file, up to the first near-tie of the reference's top-2 margin."""
    import os
    from conftest import GOLDEN
    from test_gpu_granite import compare
    g = golden("granite_small_gguf")
    from cases import G_SMALL
    h = C.c_void_p()
    gh.call("gh_granite_open_gguf", os.path.join(GOLDEN, "granite_small.gguf").encode(), 2, int(g["max_ctx"]),
            C.byref(h))
    m = Granite.__new__(Granite)
    m.gh, m.c, m.h = gh, dict(G_SMALL), h
    try:
        ids, _ = m.generate(g["prompt"], len(g["ids"]), 1, use_graph)
        assert compare(ids, g["ids"], g["margins"]) == len(g["ids"])
    finally:
        m.close()
