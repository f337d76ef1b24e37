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
GT = dict(F32=0, F16=1, Q4_0=2, Q4_1=3, Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14)


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
        # a Q4_K tensor asked for as Q8_0: decoded and quantised again (read_tensor_quant's
        # slow path, format/gguf_codec.cpp:1495-1500)
        want = O.quantize(2, O.dequantize(3, w4, 12 * 512))
        assert np.array_equal(read_packed(lib, h, "layers.3.mamba.in_proj", 2, 12 * 16 * 34), want.view(np.uint8))
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
    # a tensor of a GGML type the backend does not decode (15, Q8_K): refused by name
    write(lib, str(p), [("x", GT["Q8_0"], [256], np.zeros(8 * 34, np.uint8))], [])
    b = bytearray(open(p, "rb").read())
    _, _, infos, _, _ = parse(str(p))
    i = b.find(b"x") + 1 + 4 + 8  # name, ndims, dims -> type
    b[i:i + 4] = struct.pack("<I", 15)
    p.write_bytes(bytes(b))
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "unsupported GGML type 15" in lib.gh_last_error().decode()
    # a tensor whose data would run past the end of the file
    write(lib, str(p), [("x", GT["F32"], [64], np.zeros(64, np.float32))], [])
    p.write_bytes(open(p, "rb").read()[:-8])
    assert lib.gh_gguf_open(str(p).encode(), C.byref(h)) != 0
    assert "overruns" in lib.gh_last_error().decode()


# ---- K-quant super-blocks of real Granite-4.0-H files (Q4_K_M carries Q6_K tensors). The
# reference has no K-quant decoder: these are pinned by hand-built blocks with closed-form
# values and by an independent numpy decoder written from the GGML block layouts.
def f16b(v):
    return np.array([v], np.float16).view(np.uint8)


def pack_k_scales(sc, mn):
    """The 12-byte (6-bit scale, 6-bit min) packing of Q4_K / Q5_K."""
    s12 = np.zeros(12, np.int64)
    for j in range(4):
        s12[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s12[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s12[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return s12.astype(np.uint8)


def np_q5_k(b):
    """float32 arithmetic in the decoder's order: (d s) q - dmin m."""
    b = b.reshape(-1, 176)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int64)
    qh, qs = b[:, 16:48].astype(np.int64), b[:, 48:176].astype(np.int64)
    out = np.empty((b.shape[0], 256), np.float32)
    for j in range(8):
        if j < 4:
            sc, mn = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
        q = qs[:, 32 * (j // 2): 32 * (j // 2) + 32]
        q = (q >> 4) if j % 2 else (q & 0xF)
        q = q | (((qh >> j) & 1) << 4)
        d1 = (d * sc.astype(np.float32)).astype(np.float32)
        m1 = (dmin * mn.astype(np.float32)).astype(np.float32)
        out[:, 32 * j: 32 * j + 32] = (d1[:, None] * q.astype(np.float32)).astype(np.float32) - m1[:, None]
    return out.ravel()


def np_q6_k(b):
    """float32 arithmetic in the decoder's order: (d sc) (q - 32)."""
    b = b.reshape(-1, 210)
    ql, qh = b[:, 0:128].astype(np.int64), b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.empty((b.shape[0], 256), np.float32)
    for h in range(2):
        for r in range(4):
            lb = ql[:, 64 * h + 32 * (r % 2): 64 * h + 32 * (r % 2) + 32]
            lo = (lb & 0xF) if r < 2 else (lb >> 4)
            q = lo | (((qh[:, 32 * h: 32 * h + 32] >> (2 * r)) & 3) << 4)
            s = np.repeat(sc[:, 8 * h + 2 * r: 8 * h + 2 * r + 2], 16, axis=1)
            out[:, 128 * h + 32 * r: 128 * h + 32 * r + 32] = ((d[:, None] * s).astype(np.float32) *
                                                               (q - 32).astype(np.float32))
    return out.ravel()


def decode_via_file(lib, tmp_path, gtype, blocks, nvals):
    p = str(tmp_path / "k.gguf")
    write(lib, p, [("t", gtype, [256, nvals // 256], blocks)], [])
    h = open_file(lib, p)
    try:
        return read_f32(lib, h, "t", nvals)
    finally:
        lib.gh_gguf_close(h)


def test_q6_k_closed_form(lib, tmp_path):
    """d = 0.5, scales[i] = i - 8, and value v of the super-block carrying code (v * 7) % 64:
    every value is 0.5 * sc * (code - 32) with its scale picked by the layout."""
    codes = (np.arange(256) * 7) % 64
    blk = np.zeros(210, np.uint8)
    for h in range(2):
        for r in range(4):
            for l in range(32):
                c = int(codes[128 * h + 32 * r + l])
                i = 64 * h + 32 * (r % 2) + l
                blk[i] |= (c & 0xF) << (0 if r < 2 else 4)
                blk[128 + 32 * h + l] |= (c >> 4) << (2 * r)
    blk[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    blk[208:210] = f16b(0.5)
    want = np.array([0.5 * ((v // 128) * 8 + 2 * ((v % 128) // 32) + (v % 32) // 16 - 8) * (codes[v] - 32)
                     for v in range(256)], np.float64)
    got = decode_via_file(lib, tmp_path, GT["Q6_K"], blk, 256)
    assert np.array_equal(got.astype(np.float64), want)


def test_q5_k_closed_form(lib, tmp_path):
    """d = 2, dmin = 0.25, scale j = 2 j + 1, min j = 3 j, code of value v = v % 32 (the
    fifth bit in qh): value = 2 (2 j + 1) code - 0.25 (3 j)."""
    codes = np.arange(256) % 32
    blk = np.zeros(176, np.uint8)
    blk[0:2], blk[2:4] = f16b(2.0), f16b(0.25)
    blk[4:16] = pack_k_scales(2 * np.arange(8) + 1, 3 * np.arange(8))
    for j in range(8):
        for l in range(32):
            c = int(codes[32 * j + l])
            blk[48 + 32 * (j // 2) + l] |= (c & 0xF) << (4 if j % 2 else 0)
            blk[16 + l] |= (c >> 4) << j
    want = np.array([2.0 * (2 * (v // 32) + 1) * codes[v] - 0.25 * 3 * (v // 32) for v in range(256)])
    got = decode_via_file(lib, tmp_path, GT["Q5_K"], blk, 256)
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("gtype,nb,dec", [("Q5_K", 176, np_q5_k), ("Q6_K", 210, np_q6_k)])
def test_k_quant_random_blocks(lib, tmp_path, gtype, nb, dec):
    """Random super-blocks (finite fp16 scales) decode bit-exactly as the independent numpy
    decoder computes them in fp32."""
    rs = np.random.RandomState(7)
    blocks = rs.randint(0, 256, size=(24, nb)).astype(np.uint8)
    dpos = [0, 2] if gtype == "Q5_K" else [208]
    for o in dpos:
        blocks[:, o:o + 2] = np.float16(rs.uniform(-0.05, 0.05, 24)).view(np.uint8).reshape(24, 2)
    got = decode_via_file(lib, tmp_path, GT[gtype], blocks.ravel(), 24 * 256)
    assert np.array_equal(got.view(np.uint32), dec(blocks.ravel()).view(np.uint32))


def test_k_quant_read_as_model_kind(lib, tmp_path):
    """A Q6_K tensor read as the model's Q4_K / Q8_0 storage: decoded, then quantised by the
    backend's own quantiser (read_tensor_quant's slow path), and as fp16 for the lm head."""
    rs = np.random.RandomState(8)
    blocks = rs.randint(0, 256, size=(8, 210)).astype(np.uint8)
    blocks[:, 208:210] = np.float16(rs.uniform(0.001, 0.01, 8)).view(np.uint8).reshape(8, 2)
    vals = np_q6_k(blocks.ravel())
    p = str(tmp_path / "q6.gguf")
    write(lib, p, [("output.weight", GT["Q6_K"], [512, 4], blocks.ravel())], [])
    h = open_file(lib, p)
    try:
        for kind in (3, 2):
            nbytes = O.quantize(kind, vals).nbytes
            assert np.array_equal(read_packed(lib, h, "lm_head", kind, nbytes), O.quantize(kind, vals).view(np.uint8))
        out = np.zeros(2048, np.uint16)
        check(lib, lib.gh_gguf_read_f16(h, b"lm_head", out.ctypes.data_as(C.c_void_p), 0, C.c_size_t(2048)))
        assert np.array_equal(out, O.f32_to_f16(vals))
    finally:
        lib.gh_gguf_close(h)


def granite_config(lib, path, qkind=2):
    f = open_file(lib, path)
    try:
        cfg = np.zeros(18 + 1024, np.int32)
        fcfg = np.zeros(5, np.float32)
        n = C.c_int()
        check(lib, lib.gh_gguf_granite_config(f, qkind, cfg.ctypes.data_as(C.c_void_p), len(cfg),
                                              fcfg.ctypes.data_as(C.c_void_p), len(fcfg), C.byref(n)))
        return cfg[: n.value], fcfg
    finally:
        lib.gh_gguf_close(f)


def test_granite_config_from_reference_file(lib):
    """The model configuration read from the exporter's ghassan.* keys of a file the compiled
    reference wrote (export_model_gguf, hybrid profile) equals the configuration the reference's
    GGUFReader::model_config returned for the same file (tests/golden/granite_small_gguf.npz)."""
    g = golden("granite_small_gguf")
    path = os.path.join(GOLDEN, "granite_small.gguf")
    import hashlib
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(g["file_sha256"])
    for qkind in (2, 3):
        cfg, fcfg = granite_config(lib, path, qkind)
        want = g["cfg"].copy()
        want[15] = qkind
        assert np.array_equal(cfg, want), (cfg, want)
        assert np.array_equal(fcfg.view(np.uint32), g["fcfg"].view(np.uint32))


HYBRID_META = [("ghassan.block_count", 4, 2), ("ghassan.hybrid", 7, 1), ("ghassan.use_moe", 7, 1),
               ("ghassan.layer_types", 8, "0,1"), ("ghassan.position_embedding", 4, 1)]


def test_granite_config_defaults(lib, tmp_path):
    """Keys the file lacks take the ModelConfig defaults (model/model.h): dims, experts, Mamba
    sizes, multipliers 1, attention scale 1/sqrt(head_dim), shared width = routed width, tied."""
    p = str(tmp_path / "m.gguf")
    write(lib, p, [], HYBRID_META + [("ghassan.moe.expert_feed_forward_length", 4, 512)])
    cfg, fcfg = granite_config(lib, p, 3)
    assert list(cfg) == [16000, 768, 2, 12, 4, 64, 512, 8, 2, 512, 1536, 48, 64, 128, 4, 3, 0, 1, 1, 0]
    assert list(fcfg) == [np.float32(1e-5), np.float32(1 / 8), 1, 1, 1]


@pytest.mark.parametrize("meta,err", [
    ([("ghassan.hybrid", 7, 0)], "not a Granite hybrid"),
    ([("ghassan.use_moe", 7, 0)], "dense FFN"),
    ([("ghassan.moe.shared_expert", 7, 0)], "shared expert"),
    ([("ghassan.mamba.n_groups", 4, 2)], "n_groups"),
    ([("ghassan.use_qk_norm", 7, 1)], "use_qk_norm"),
    ([("ghassan.mamba.proj_bias", 7, 1)], "proj_bias"),
    ([("ghassan.position_embedding", 4, 0)], "NoPE"),
    ([("ghassan.sliding_window", 4, 128)], "sliding window"),
    ([("ghassan.layer_types", 8, "0,1,1")], "length does not match"),
    ([("ghassan.layer_types", 8, "0,2")], "expected '0' or '1'"),
    ([("ghassan.block_count", 4, 3)], "length does not match"),
])
def test_granite_config_rejects(lib, tmp_path, meta, err):
    p = str(tmp_path / "m.gguf")
    keys = {k for k, _, _ in meta}
    write(lib, p, [], [m for m in HYBRID_META if m[0] not in keys] + meta)
    with pytest.raises(RuntimeError, match=err):
        granite_config(lib, p)


def test_granite_config_needs_architecture_keys(lib, tmp_path):
    p = str(tmp_path / "m.gguf")
    write(lib, p, [], [("general.architecture", 8, "ghassan")])
    with pytest.raises(RuntimeError, match="no architecture keys"):
        granite_config(lib, p)


def test_open_gguf_refuses_before_allocating(lib, tmp_path):
    """gh_granite_open_gguf checks the file and its configuration before any device work: a
    missing file, a file without architecture keys and a dense (non-hybrid) model fail with
    the reader's message and leave the output handle null."""
    cases = [(str(tmp_path / "missing.gguf"), "cannot open")]
    p1 = str(tmp_path / "noarch.gguf")
    write(lib, p1, [], [("general.architecture", 8, "llama")])
    cases.append((p1, "no architecture keys"))
    p2 = str(tmp_path / "dense.gguf")
    write(lib, p2, [], [m for m in HYBRID_META if m[0] != "ghassan.hybrid"] + [("ghassan.hybrid", 7, 0)])
    cases.append((p2, "not a Granite hybrid"))
    for path, msg in cases:
        h = C.c_void_p(1)
        rc = lib.gh_granite_open_gguf(path.encode(), 2, 64, C.byref(h))
        assert rc != 0 and not h.value, path
        assert msg in lib.gh_last_error().decode(), (path, lib.gh_last_error())
