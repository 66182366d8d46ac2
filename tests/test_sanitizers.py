"""The CPU side under AddressSanitizer + UndefinedBehaviorSanitizer.

`make -C oracle sanitize` and `make -C mythos.cpp_amd sanitize` build the
oracle, the C ABI library (host code: every entry point's argument
validation, the workspace, the decoder's host logic) and the host library
(the .oil reader, the C++ facade) with -fsanitize=address,undefined and no
recovery, all with ROCm's clang so that one process holds them under one
sanitizer runtime.  A child pytest then runs the CPU suites that exercise
them -- the oracle against its pins and golden vectors, the .oil reader on
valid, truncated and corrupt files, the C ABI's validation of bad
arguments, the decoder oracle -- with the runtime preloaded and the
libraries selected by MYTHOS_ORACLE_LIB / MYTHOS_OIL_LIB / MYTHOS_HOST_LIB.
Any report ends the child with a failure.  No GPU is used.
"""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang"
SUITES = ["tests/test_oracle.py", "tests/test_golden.py", "tests/test_oil_file.py", "tests/test_abi.py",
          "tests/test_decoder_oracle.py"]


def sanitized_libs():
    return {
        "MYTHOS_ORACLE_LIB": os.path.join(ROOT, "oracle", "_asan", "liboracle.so"),
        "MYTHOS_OIL_LIB": os.path.join(ROOT, "mythos.cpp_amd", "_build", "asan", "libmythos_oil.so"),
        "MYTHOS_HOST_LIB": os.path.join(ROOT, "mythos.cpp_amd", "_build", "asan", "libmythos_host.so"),
    }


def test_cpu_suites_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "mythos.cpp_amd"), "-j8", "sanitize"], check=True)
    rt = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True,
                        check=True).stdout.strip()
    assert os.path.exists(rt), rt
    libs = sanitized_libs()
    for path in libs.values():
        syms = subprocess.run(["nm", "-D", path], capture_output=True, text=True, check=True).stdout
        assert "__asan_report_load" in syms and "__ubsan_handle" in syms, f"{path} is not instrumented"
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", **libs)
    # the child loads exactly these builds
    probe = ("import sys; sys.path[:0] = ['tests', 'mythos.cpp_amd', '.']\n"
             "import mythos_oil, oil_file\n"
             "from oracle import Oracle\n"
             "Oracle()\n"
             "maps = open('/proc/self/maps').read()\n"
             "import os\n"
             "missing = [p for p in (os.environ['MYTHOS_ORACLE_LIB'], os.environ['MYTHOS_OIL_LIB'],"
             " os.environ['MYTHOS_HOST_LIB']) if p not in maps]\n"
             "assert not missing, missing\n"
             "assert 'libclang_rt.asan' in maps\n")
    r = subprocess.run([sys.executable, "-c", probe], env=env, cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
                        *SUITES], env=env, cwd=ROOT, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-4000:]
    assert " passed" in r.stdout
