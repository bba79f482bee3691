"""The library's host C++ -- the GGUF reader, the draft-tree builders, the
argument checks of the C ABI -- under AddressSanitizer.  The CPU tests of those
parts run again in a child process against libspeculate_hip_asan.so (every
host pass of the library compiled with -fsanitize=address, the gfx950 code
unchanged), with the sanitizer runtime preloaded into the uninstrumented
Python.  Any invalid read or write (the seeded header mutations of
test_gguf_host.py walk the reader through truncated and corrupted files) ends
the child with the sanitizer's report."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "abyo-speculate_amd")

HOST_TESTS = ["tests/test_gguf_host.py", "tests/test_host_tree.py", "tests/test_abi_exports.py",
              "tests/test_host_layout.py"]


def test_host_code_under_address_sanitizer():
    sys.path.insert(0, PKG)
    import build_lib
    srcs = [os.path.join(build_lib.CSRC, f) for f in os.listdir(build_lib.CSRC)]
    if not os.path.exists(build_lib.ASAN_LIB) or os.path.getmtime(build_lib.ASAN_LIB) < max(map(os.path.getmtime, srcs)):
        build_lib.build_asan(verbose=False)
    env = dict(os.environ)
    env.update(LD_PRELOAD=build_lib.asan_runtime(), SPECULATE_HIP_LIB=build_lib.ASAN_LIB,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1:exitcode=86")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu"]
                       + HOST_TESTS, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "AddressSanitizer" not in out, out
    assert " passed" in r.stdout, out
