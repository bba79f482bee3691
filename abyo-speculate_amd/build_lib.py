"""Build recipe of libspeculate_hip.so (gfx950) -- run by __graft_entry__.build().

Compiles every .hip / .cpp under csrc/ with hipcc for gfx950 into _build/,
in parallel, then links the shared library next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libspeculate_hip.so")
INCLUDE = os.environ.get("SD_INCLUDE_DIR", os.path.join(os.path.dirname(HERE), "include"))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
          # multiply-adds (and products rounded to fp16) fuse only where one
          # source expression forms them, so every kernel that inlines the
          # same device code rounds the same way (the default, fast, lets the
          # backend fuse across statements depending on the surrounding code)
          "-ffp-contract=on",
          # no packed-FP32 instructions anywhere (hipcc's host pass warns that it
          # does not know the feature; that warning is expected)
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-result", "-I" + INCLUDE]


# The host-checking variant (CPU tests only): every host pass instrumented by
# AddressSanitizer, the gfx950 code unchanged, the sanitizer runtime linked as
# a shared library so that a test can preload it into an uninstrumented Python.
ASAN_BUILD = os.path.join(HERE, "_build_asan")
ASAN_LIB = os.path.join(HERE, "libspeculate_hip_asan.so")
ASAN_FLAGS = "-Xarch_host -fsanitize=address -Xarch_host -fno-omit-frame-pointer".split()


def _compile(src: str, build_dir: str = BUILD, extra=()) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC] + COMMON + list(extra) + ["-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC] + COMMON + list(extra) + ["-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def _build(lib: str, build_dir: str, extra=(), link_extra=(), verbose: bool = True) -> str:
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, extra), srcs))
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + list(link_extra) + ["-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}", file=sys.stderr)
    return lib


def build(verbose: bool = True) -> str:
    return _build(LIB, BUILD, verbose=verbose)


def build_asan(verbose: bool = True) -> str:
    return _build(ASAN_LIB, ASAN_BUILD, ASAN_FLAGS, ASAN_FLAGS + ["-shared-libasan"], verbose)


def asan_runtime() -> str:
    """Path of the shared AddressSanitizer runtime the ASan variant links."""
    r = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        raise RuntimeError("AddressSanitizer runtime not found")
    return path


if __name__ == "__main__":
    build_asan() if sys.argv[1:] == ["asan"] else build()
