"""The drop-in boundary without a GPU: libmythos_oil.so loads and exports
exactly the entry points include/mythos_oil.h declares, each rejects invalid
arguments with MTH_EINVAL and a message before touching the device, and
libmythos_host.so exports the reference's oil::kernel signatures
(include/oil/kernel.h:13-65 of the reference).  The GPU half of the façade is
in test_gpu_facade.py.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mythos.cpp_amd")
HDR = os.path.join(ROOT, "include", "mythos_oil.h")


DEC_HDR = os.path.join(ROOT, "include", "mythos_decoder.h")


def declared(hdr=HDR):
    src = open(hdr).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mth_[a-z0-9_]+)\s*\(", src)))


def dynsyms(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}


def test_header_matches_exports(mth):
    import decoder
    decl, dec = declared(), declared(DEC_HDR)
    assert decl == sorted(mth.EXPORTS)
    assert dec == sorted(decoder.EXPORTS)
    syms = dynsyms(mth.LIB_PATH)
    missing = [d for d in decl + dec if d not in syms]
    assert not missing, missing
    extra = sorted(s for s in syms if s.startswith("mth_") and s not in decl + dec)
    assert not extra, f"exported but undeclared: {extra}"
    for d in decl + dec:                 # resolvable through the loader too
        assert getattr(mth.lib, d) is not None


def test_file_reader_header_matches_exports():
    """include/mythos_oil_file.h (the .oil reader) is served by libmythos_host.so."""
    import oil_file
    hdr = os.path.join(ROOT, "include", "mythos_oil_file.h")
    src = re.sub(r"/\*.*?\*/", "", open(hdr).read(), flags=re.S)
    decl = sorted(set(re.findall(r"\b(mth_[a-z0-9_]+)\s*\(", src)))
    assert decl == sorted(oil_file.EXPORTS)
    syms = dynsyms(oil_file.HOST_LIB_PATH)
    assert not [d for d in decl if d not in syms]
    for d in decl:
        assert getattr(oil_file.lib, d) is not None


def test_version(mth):
    assert mth.version() >> 16 == 2   # 2.0: mth_decoder_config.struct_size


NULL = None
# (entry point, arguments with a null pointer, arguments with a bad size)
P = C.c_void_p(16)   # never dereferenced: validation fails first
CASES = [
    ("mth_oil8_gemm", (NULL, P, P, P, 4, 1, 4, NULL), (P, P, P, P, 0, 1, 4, NULL)),
    ("mth_oil8_gemv", (P, NULL, P, P, 4, 4, 1, NULL), (P, P, P, P, 4, -1, 1, NULL)),
    ("mth_oil4_gemm", (P, P, NULL, P, 4, 1, 4, NULL), (P, P, P, P, 4, 1, 0, NULL)),
    ("mth_oil4_gemv", (P, P, 128, NULL, P, 4, 128, 1, NULL), (P, P, 100, P, P, 4, 128, 1, NULL)),
    ("mth_oil4_gemm_prefill", (P, P, P, 128, NULL, 4, 4, 128, NULL), (P, P, P, 128, P, 4, 4, 100, NULL)),
    ("mth_quantize_per_token", (NULL, P, P, P, 1, 4, NULL), (P, P, P, P, 0, 4, NULL)),
    ("mth_dequantize_per_tensor", (NULL, P, 4, C.c_float(1.0), NULL), (P, P, -4, C.c_float(1.0), NULL)),
    ("mth_i2s_gemv", (P, C.c_float(1.0), P, NULL, P, 4, 8, 1, NULL), (P, C.c_float(1.0), P, P, P, 4, 6, 1, NULL)),
    ("mth_i2s_gemv_f32", (NULL, C.c_float(1.0), P, P, 4, 8, 1, NULL), (P, C.c_float(1.0), P, P, 4, 10, 1, NULL)),
    ("mth_i2s_gemm", (P, NULL, P, 4, 1, 8, NULL), (P, P, P, 4, 1, 0, NULL)),
    ("mth_i2s_gemm_vnni", (P, P, NULL, 4, 1, 8, NULL), (P, P, P, -4, 1, 8, NULL)),
    ("mth_tl1_gemm", (NULL, P, P, 4, 1, 8, NULL), (P, P, P, 4, 0, 8, NULL)),
    ("mth_tl2_gemm", (P, NULL, P, 4, 1, 6, NULL), (P, P, P, 4, 1, 8, NULL)),
    ("mth_tl_precompute_lut", (NULL, P, 6, 3, NULL), (P, P, 6, 4, NULL)),
    ("mth_rms_norm", (P, NULL, P, 1, 8, C.c_float(1e-5), NULL), (P, P, P, 0, 8, C.c_float(1e-5), NULL)),
    ("mth_add_rms_norm", (P, NULL, P, P, 1, 8, C.c_float(1e-5), NULL), (P, P, P, P, 1, -8, C.c_float(1e-5), NULL)),
    ("mth_silu", (NULL, P, 8, NULL), (P, P, 0, NULL)),
    ("mth_silu_mul", (P, NULL, P, 1, 8, 8, 8, NULL), (P, P, P, 1, 8, 4, 8, NULL)),
    ("mth_silu_mul_quant", (P, P, NULL, P, 1, 8, 8, 8, NULL), (P, P, P, P, 1, 12289, 12289, 12289, NULL)),
    ("mth_add", (P, P, NULL, 8, NULL), (P, P, P, -1, NULL)),
    ("mth_mul", (NULL, P, P, 8, NULL), (P, P, P, 0, NULL)),
    ("mth_softmax", (P, NULL, 1, 8, NULL), (P, P, 1, 0, NULL)),
    ("mth_rope_kv", (P, P, P, P, P, NULL, P, 0, 1, 2, 2, 64, 8, NULL), (P, P, P, P, P, P, P, 8, 1, 2, 2, 64, 8, NULL)),
    ("mth_attention_decode", (P, P, NULL, P, 1, 2, 2, 64, 1, 8, NULL), (P, P, P, P, 1, 2, 2, 64, 9, 8, NULL)),
    ("mth_argmax", (P, NULL, 1, 8, NULL), (P, P, 1, 0, NULL)),
]


@pytest.mark.parametrize("name,nullargs,badargs", CASES, ids=[c[0] for c in CASES])
def test_invalid_arguments_rejected(mth, name, nullargs, badargs):
    f = getattr(mth.lib, name)
    for args in (nullargs, badargs):
        rc = f(*args)
        assert rc == mth.MTH_EINVAL, (name, args, rc)
        msg = mth.last_error()
        assert msg.startswith(name), msg
    # the message stays readable until the calling thread's next call
    assert mth.last_error().startswith(name)


def test_errors_raise_in_wrapper(mth):
    with pytest.raises(TypeError):
        mth.oil8_gemv(None, None, None, None, 4, 4)


# Reference signatures (include/oil/kernel.h:13-65) the façade must export,
# demangled; Tensor-based ones take oil::Tensor exactly as the reference.
FACADE = [
    "oil::kernel::i2s_gemm(oil::Tensor const&, oil::Tensor const&, oil::Tensor&, int, int, int)",
    "oil::kernel::i2s_gemv(unsigned char const*, float, signed char const*, float, float*, int)",
    "oil::kernel::tl1_gemm(oil::Tensor const&, oil::Tensor const&, oil::Tensor&, int, int, int)",
    "oil::kernel::tl1_precompute_lut(signed char const*, signed char*, int, float)",
    "oil::kernel::tl2_gemm(oil::Tensor const&, oil::Tensor const&, oil::Tensor&, int, int, int)",
    "oil::kernel::tl2_precompute_lut(signed char const*, signed char*, int, float)",
    "oil::kernel::oil8_gemm(unsigned char const*, float const*, float const*, float*, int, int, int)",
    "oil::kernel::oil4_gemm(unsigned char const*, unsigned short const*, float const*, float*, int, int, int)",
    "oil::kernel::i2s_gemm_avx2(oil::Tensor const&, oil::Tensor const&, oil::Tensor&, int, int, int)",
    "oil::kernel::i2s_gemm_vnni(unsigned char const*, signed char const*, float*, int, int, int)",
    # src/int8_quant.cpp:8-41 / include/oil/int8_quant.h:7-28
    "oil::quantize_per_token(float const*, signed char*, long, long)",
    "oil::quantize_per_tensor(float const*, signed char*, long)",
    "oil::dequantize_per_tensor(signed char const*, float*, long, float)",
    # include/oil/backend.h:79,87,96 (the HIP ComputeBackend behind the factory)
    "oil::backend::ComputeBackend::create(oil::backend::BackendConfig const&)",
    "oil::backend::is_cuda_available()",
    "oil::backend::gpu_memory_free(long)",
    "oil::mi355x::make_hip_backend(long)",
]


def test_facade_exports_reference_signatures(mth):
    path = mth.HOST_LIB_PATH
    assert os.path.exists(path), "libmythos_host.so not built"
    out = subprocess.run(["nm", "-DC", "--defined-only", path], check=True, capture_output=True, text=True).stdout
    have = {ln.split(None, 2)[2] for ln in out.splitlines() if len(ln.split(None, 2)) == 3}
    missing = [s for s in FACADE if s not in have]
    assert not missing, missing


REF_INCLUDE = os.environ.get("MYTHOS_REFERENCE", "/root/reference") + "/include"


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference headers not present on this host")
def test_facade_compiles_against_reference_headers():
    """The façade sources build against the reference's own oil/*.h (its
    Tensor, Error, Int8QuantParams, and its ComputeBackend declaration, which
    the HIP backend overrides), so they link into the reference's tree in
    place of its CPU kernel library and its backend factory."""
    for name, defs in (("kernel.cpp", []), ("backend.cpp", []), ("backend.cpp", ["-DOIL_HAS_MI355X=1"])):
        src = os.path.join(PKG, "host", name)
        r = subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++20", "-fsyntax-only", *defs, f"-I{REF_INCLUDE}",
                            f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(PKG, 'host', 'include')}", src],
                           capture_output=True, text=True)
        assert r.returncode == 0, (name, defs, r.stderr)


def test_decoder_argument_errors(mth):
    import decoder
    lib = mth.lib
    h = C.c_void_p()
    size = C.sizeof(decoder.Config)
    cfg = decoder.Config(size, 1000, 256, 2, 2, 2, 128, 512, 16, 128, 1, 1e-5, 1e4)
    bad = [dict(max_batch=17), dict(head_dim=96), dict(heads=3), dict(cb_block=100), dict(hidden=254),
           dict(max_seq=0), dict(struct_size=size - 8), dict(struct_size=1000)]
    for b in bad:
        c = decoder.Config(b.get("struct_size", size), *[b.get(k, getattr(cfg, k)) for k in decoder.CONFIG_KEYS],
                           cfg.eps, cfg.theta)
        rc = lib.mth_decoder_create(C.byref(c), C.byref(h))
        assert rc in (mth.MTH_EINVAL, mth.MTH_EUNSUPPORTED), (b, rc)
        assert mth.last_error().startswith("mth_decoder_create"), mth.last_error()
        if "struct_size" in b:
            assert "struct_size" in mth.last_error(), mth.last_error()
    # a caller of the 1.x header (no struct_size: vocab first) is refused
    old = (C.c_int64 * 11)(1000, 256, 2, 2, 2, 128, 512, 16, 128, 1, 0)
    assert lib.mth_decoder_create(C.cast(old, C.POINTER(decoder.Config)), C.byref(h)) == mth.MTH_EINVAL
    assert mth.version() >> 16 == 2
    assert lib.mth_decoder_step(None, 1, 1, None) == mth.MTH_EINVAL
    assert lib.mth_decoder_start(None, P, 1, 1, None) == mth.MTH_EINVAL
    assert lib.mth_decoder_read(None, None, None, None) == mth.MTH_EINVAL

