"""CPU tests of the product library without a GPU: it loads, exports every
entry point include/ghassan_hip.h declares, and its host-side codecs and
synthetic-weight recipe match the oracle (no compute calls on the device)."""
import ctypes as C

import numpy as np
import pytest

import ghassan_hip as gh
import oracle_lib as O


@pytest.fixture(scope="module")
def lib():
    return gh.load(init_device=False)


def test_exports_every_declared_symbol(lib):
    syms = gh.header_symbols()
    assert len(syms) >= 50
    missing = [s for s in syms if not hasattr(lib, s)]
    assert missing == []


def test_no_oracle_or_reference_dependency():
    """The product library must not link the oracle or the reference build."""
    import subprocess
    out = subprocess.run(["ldd", gh.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out and "gai_ref" not in out


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_host_quantizer_matches_oracle(lib, kind):
    x = O.rng_normal(7, 256 * 64, 0, 0.5)
    x[1000] = np.inf
    assert np.array_equal(gh.quantize(kind, x), O.quantize(kind, x))


def test_host_q8_tail_matches_oracle(lib):
    x = O.rng_normal(8, 77)
    assert np.array_equal(gh.quantize(2, x), O.quantize(2, x))


def test_host_rng_matches_oracle(lib):
    for seed in (0, 5, 123456789):
        assert np.array_equal(gh.rng_normal(seed, 999).view(np.uint32), O.rng_normal(seed, 999).view(np.uint32))
        assert np.array_equal(gh.rng_uniform(seed, 99, -1, 2).view(np.uint32),
                              O.rng_uniform(seed, 99, -1, 2).view(np.uint32))
        assert np.array_equal(gh.rng_below(seed, 99, 4096), O.rng_below(seed, 99, 4096))


@pytest.mark.parametrize("name", ["tok_embeddings", "layers.0.mamba.A_log", "layers.2.wq", "layers.1.attn_norm",
                                  "layers.4.mamba.conv1d.bias", "layers.5.moe_router"])
def test_synthetic_recipe_matches_oracle(lib, name):
    n = 4096
    assert np.array_equal(gh.synth_param(name, n).view(np.uint32), O.synth_param(name, n).view(np.uint32))


def test_quantize_rejects_bad_sizes(lib):
    x = np.zeros(100, np.float32)
    out = np.zeros(1000, np.uint8)
    assert lib.gh_quantize_host(3, x.ctypes.data, out.ctypes.data, 100) != 0
    assert b"multiple" in lib.gh_last_error()


def test_product_has_no_cpu_fallback():
    """Every compute entry point is a device launch: with no GPU they fail
    loudly instead of computing on the host."""
    import torch  # noqa: F401  (only to ask whether a GPU is present)
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = gh.load(init_device=False)
    assert lib.gh_init(0) != 0


def test_m0_only_set_for_lds_transfers(tmp_path):
    """The direct global -> LDS transfers set M0 from inline assembly. M0 is a register the
    compiler reserves (a clobber on it is rejected), so the guard is the generated code: in
    every file that issues such transfers, each M0 write is ours, immediately followed by its
    global_load_lds_dwordx4, and no compiler-generated instruction reads or writes M0."""
    import os
    import re
    import subprocess
    src = os.path.join(os.path.dirname(gh.LIB_PATH), "csrc")
    for f in ("gemv_mfma", "gemv8", "attention", "gemm", "decode_persistent"):
        out = tmp_path / (f + ".s")
        subprocess.run(["/opt/rocm/bin/hipcc", "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang",
                        "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                        os.path.join(src, f + ".hip"), "-o", str(out)], check=True, capture_output=True)
        lines = [ln.strip() for ln in out.read_text().splitlines()]
        n = 0
        for i, ln in enumerate(lines):
            if ln.startswith(";") or not re.search(r"\bm0\b", ln):
                continue
            assert ln.startswith("s_mov_b32 m0,"), f"{f}: compiler use of m0: {ln}"
            assert lines[i + 1].startswith("global_load_lds_dwordx4"), f"{f}: {ln} / {lines[i + 1]}"
            n += 1
        assert n > 0, f
