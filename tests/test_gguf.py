"""GGUF reader / writer of the backend (host side; runs without a GPU).

Pinned by a file written by the reference's own GGUFWriter and the bytes its
GGUFReader returned for it (golden ref_small.gguf + gguf.npz), by an
independent numpy parser of the format, and by the oracle quantiser for the
host re-quantisation path. Q4_K (type 12) has no reference reader: its
passthrough is pinned by the round trip of known packed bytes."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import oracle_lib as O
from conftest import GOLDEN, golden

REF_FILE = os.path.join(GOLDEN, "ref_small.gguf")
GT = dict(F32=0, F16=1, Q4_0=2, Q4_1=3, Q8_0=8, Q4_K=12)


@pytest.fixture(scope="module")
def lib():
    import ghassan_hip
    lib = ghassan_hip.load(init_device=False)
    lib.gh_gguf_tensor_count.restype = C.c_int64
    lib.gh_gguf_find_tensor.restype = C.c_int64
    lib.gh_gguf_find_tensor.argtypes = [C.c_void_p, C.c_char_p]
    lib.gh_gguf_tensor_count.argtypes = [C.c_void_p]
    return lib


def check(lib, rc):
    if rc != 0:
        raise RuntimeError(lib.gh_last_error().decode())


def parse(path):
    """Independent reader of the GGUF layout: header, metadata, tensor infos."""
    b = open(path, "rb").read()
    at = 0

    def take(fmt):
        nonlocal at
        v = struct.unpack_from("<" + fmt, b, at)
        at += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def s():
        nonlocal at
        n = take("Q")
        v = b[at:at + n].decode()
        at += n
        return v

    scal = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
    assert take("I") == 0x46554747
    ver, nt, nkv = take("I"), take("Q"), take("Q")
    kv = {}
    for _ in range(nkv):
        k, t = s(), take("I")
        if t == 8:
            kv[k] = s()
        elif t == 9:
            et, n = take("I"), take("Q")
            kv[k] = [s() if et == 8 else take(scal[et]) for _ in range(n)]
        else:
            kv[k] = take(scal[t])
    infos = []
    for _ in range(nt):
        name, nd = s(), take("I")
        dims = [take("Q") for _ in range(nd)]
        infos.append((name, dims, take("I"), take("Q")))
    align = kv.get("general.alignment", 32)
    start = (at + align - 1) // align * align
    return ver, kv, infos, start, b


def open_file(lib, path):
    h = C.c_void_p()
    check(lib, lib.gh_gguf_open(path.encode(), C.byref(h)))
    return h


def info(lib, h, i):
    name, t, nd, nb = C.c_char_p(), C.c_uint32(), C.c_int(), C.c_uint64()
    dims = (C.c_uint64 * 8)()
    check(lib, lib.gh_gguf_tensor_info(h, C.c_int64(i), C.byref(name), C.byref(t), C.byref(nd), dims, C.byref(nb)))
    return name.value.decode(), t.value, list(dims[:nd.value]), nb.value


def read_packed(lib, h, name, kind, nbytes):
    out = np.zeros(nbytes, np.uint8)
    check(lib, lib.gh_gguf_read_packed(h, name.encode(), kind, out.ctypes.data_as(C.c_void_p), 0, C.c_size_t(nbytes)))
    return out


def read_f32(lib, h, name, n):
    out = np.zeros(n, np.float32)
    check(lib, lib.gh_gguf_read_f32(h, name.encode(), out.ctypes.data_as(C.c_void_p), 0, C.c_size_t(n)))
    return out


def test_reference_written_file(lib):
    g = golden("gguf")
    ver, kv, infos, start, raw = parse(REF_FILE)
    h = open_file(lib, REF_FILE)
    try:
        assert lib.gh_gguf_tensor_count(h) == len(infos) == 3
        got = {info(lib, h, i)[0]: info(lib, h, i) for i in range(3)}
        for name, dims, t, off in infos:
            assert got[name][1] == t and got[name][2] == dims
        assert got["layers.0.wq"][1] == GT["Q8_0"] and got["layers.0.wq"][2] == [64, 16]
        assert got["layers.0.wq"][3] == 16 * 2 * 34
        # packed Q8_0 blocks: exactly the reference reader's bytes (and the file's)
        q = read_packed(lib, h, "layers.0.wq", 2, 16 * 2 * 34)
        assert np.array_equal(q, g["wq_packed"])
        off = [i for i in infos if i[0] == "layers.0.wq"][0][3]
        assert np.array_equal(q, np.frombuffer(raw, np.uint8, q.size, start + off))
        # F32 and F16 tensors as read_tensor_f32 returns them
        assert np.array_equal(read_f32(lib, h, "layers.0.attn_norm", 192).view(np.uint32),
                              g["attn_norm_f32"].view(np.uint32))
        assert np.array_equal(read_f32(lib, h, "tok_embeddings", 640).view(np.uint32),
                              g["tok_embeddings_f32"].view(np.uint32))
        h16 = np.zeros(640, np.uint16)
        check(lib, lib.gh_gguf_read_f16(h, b"tok_embeddings", h16.ctypes.data_as(C.c_void_p), 0, C.c_size_t(640)))
        assert np.array_equal(O.f16_to_f32(h16), g["tok_embeddings_f32"])
        # F32 file tensor -> Q8_0 on the host (the reference's slow path): the oracle quantiser's bytes
        assert np.array_equal(read_packed(lib, h, "layers.0.attn_norm", 2, 6 * 34), O.quantize(2, g["a"]))
        # metadata as the independent parser sees it
        buf = C.create_string_buffer(64)
        check(lib, lib.gh_gguf_get_str(h, b"general.architecture", buf, C.c_size_t(64)))
        assert buf.value.decode() == kv["general.architecture"]
        for k, v in kv.items():
            if isinstance(v, int) and not isinstance(v, bool):
                u = C.c_uint64()
                check(lib, lib.gh_gguf_get_u64(h, k.encode(), C.byref(u)))
                assert u.value == v, k
            elif isinstance(v, float):
                f = C.c_float()
                check(lib, lib.gh_gguf_get_f32(h, k.encode(), C.byref(f)))
                assert f.value == np.float32(v), k
        assert lib.gh_gguf_find_tensor(h, b"nope") == -1
    finally:
        lib.gh_gguf_close(h)


def write(lib, path, tensors, meta):
    """tensors: (name, ggml_type, dims, packed bytes); meta: (key, gguf type, value)."""
    n = len(tensors)
    names = (C.c_char_p * n)(*[t[0].encode() for t in tensors])
    types = (C.c_uint32 * n)(*[t[1] for t in tensors])
    nd = (C.c_int * n)(*[len(t[2]) for t in tensors])
    dims = (C.c_uint64 * (8 * n))()
    for i, t in enumerate(tensors):
        for j, d in enumerate(t[2]):
            dims[8 * i + j] = d
    data = (C.c_void_p * n)(*[t[3].ctypes.data for t in tensors])
    keep = []
    vals = []
    for k, t, v in meta:
        if t == 8:
            b = C.create_string_buffer(v.encode())
        else:
            b = np.array([v], {4: np.uint32, 6: np.float32, 10: np.uint64, 7: np.uint8}[t])
        keep.append(b)
        vals.append(C.cast(b, C.c_void_p) if t == 8 else b.ctypes.data)
    m = len(meta)
    keys = (C.c_char_p * m)(*[k.encode() for k, _, _ in meta])
    kt = (C.c_uint32 * m)(*[t for _, t, _ in meta])
    kvv = (C.c_void_p * m)(*vals)
    check(lib, lib.gh_gguf_write(path.encode(), n, names, types, nd, dims, data, m, keys, kt, kvv))


@pytest.mark.parametrize("align", [32, 64, 256])
def test_write_read_q4k_roundtrip(lib, tmp_path, align):
    w4 = O.quantize(3, O.rng_normal(83, 12 * 512, 0, 0.02))        # Q4_K [12][512]
    w8 = O.quantize(2, O.rng_normal(84, 5 * 96, 0, 0.02))          # Q8_0 [5][96]
    v32 = O.rng_normal(85, 7)
    v16 = O.f32_to_f16(O.rng_normal(86, 40))
    tensors = [("layers.3.mamba.in_proj", GT["Q4_K"], [512, 12], w4), ("blk.1.attn_q.weight", GT["Q8_0"], [96, 5], w8),
               ("layers.0.mamba.D", GT["F32"], [7], v32), ("token_embd.weight", GT["F16"], [8, 5], v16)]
    meta = [("general.alignment", 4, align), ("general.architecture", 8, "ghassan"), ("ghassan.block_count", 4, 6),
            ("ghassan.attention.layer_norm_rms_epsilon", 6, 1e-5), ("ghassan.context_length", 10, 4096)]
    path = str(tmp_path / "w.gguf")
    write(lib, path, tensors, meta)
    ver, kv, infos, start, raw = parse(path)
    assert ver == 3 and kv["general.alignment"] == align and start % align == 0
    assert [(i[0], i[1], i[2]) for i in infos] == [(t[0], t[2], t[1]) for t in tensors]
    for (name, dims, t, off), tt in zip(infos, tensors):
        assert off % align == 0
        assert np.array_equal(np.frombuffer(raw, np.uint8, tt[3].nbytes, start + off), tt[3].view(np.uint8))
    h = open_file(lib, path)
    try:
        assert np.array_equal(read_packed(lib, h, "layers.3.mamba.in_proj", 3, w4.nbytes), w4.view(np.uint8))
        # by the backend name through the llama.cpp alias (attn_q / token_embd)
        assert np.array_equal(read_packed(lib, h, "layers.1.wq", 2, w8.nbytes), w8.view(np.uint8))
        assert lib.gh_gguf_find_tensor(h, b"tok_embeddings") == 3
        assert np.array_equal(read_f32(lib, h, "layers.0.mamba.D", 7), v32)
        u = C.c_uint64()
        check(lib, lib.gh_gguf_get_u64(h, b"ghassan.context_length", C.byref(u)))
        assert u.value == 4096
        # a Q4_K tensor asked for as Q8_0 is not decoded here: an error, not a silent conversion
        with pytest.raises(RuntimeError, match="not F32/F16"):
            read_packed(lib, h, "layers.3.mamba.in_proj", 2, 12 * 16 * 34)
        with pytest.raises(RuntimeError, match="needs"):
            read_packed(lib, h, "layers.3.mamba.in_proj", 3, w4.nbytes - 1)
    finally:
        lib.gh_gguf_close(h)


def test_rejects_bad_files(lib, tmp_path):
    h = C.c_void_p()
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML" + b"\0" * 60)
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "not a GGUF file" in lib.gh_last_error().decode()
    good = open(REF_FILE, "rb").read()
    p.write_bytes(good[:40])  # truncated metadata
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    p.write_bytes(good[:4] + struct.pack("<I", 4) + good[8:])
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "unsupported version" in lib.gh_last_error().decode()
    # a Q6_K (type 14) tensor: refused by name, like the reference
    q6 = np.zeros(210, np.uint8)
    write(lib, str(p), [("x", GT["Q8_0"], [256], np.zeros(8 * 34, np.uint8))], [])
    b = bytearray(open(p, "rb").read())
    _, _, infos, _, _ = parse(str(p))
    i = b.find(b"x") + 1 + 4 + 8  # name, ndims, dims -> type
    b[i:i + 4] = struct.pack("<I", 14)
    p.write_bytes(bytes(b))
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "unsupported GGML type 14" in lib.gh_last_error().decode()
    del q6
    # a tensor whose data would run past the end of the file
    write(lib, str(p), [("x", GT["F32"], [64], np.zeros(64, np.float32))], [])
    p.write_bytes(open(p, "rb").read()[:-8])
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "overruns" in lib.gh_last_error().decode()
