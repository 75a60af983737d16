"""Build the C ABI with AddressSanitizer on its host code and the host checks.

Every HIP source of the library is compiled as for libltx_hip.so (gfx950
device code unchanged) with ``-fsanitize=address`` on the host side only
(``-Xarch_host``: the GPU code is not instrumented), and linked with
``host_checks.cpp`` into one executable, ``_asan_build/host_checks``.
Objects are rebuilt only when their source or a header is newer.  Run
``python ltx-2-mlx_amd/asan/build.py`` to build and run it.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
SRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT = PKG / "_asan_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang++"
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def _headers_mtime() -> float:
    return max(p.stat().st_mtime for p in list(SRC.glob("*.h")) + list(INCLUDE.glob("*.h")))


def _compile(src: Path) -> Path:
    obj = OUT / (src.stem + ".o")
    if obj.exists() and obj.stat().st_mtime >= max(src.stat().st_mtime, _headers_mtime()):
        return obj
    cmd = [str(HIPCC), *FLAGS, *ASAN_HOST, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-4000:]}")
    return obj


def build() -> Path:
    OUT.mkdir(exist_ok=True)
    srcs = sorted(SRC.glob("*.hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    exe = OUT / "host_checks"
    main = HERE / "host_checks.cpp"
    cmd = [str(CLANG), "-std=c++17", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", str(main),
           *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-4000:]}")
    return exe


def run(exe: Path) -> subprocess.CompletedProcess:
    env = dict(os.environ)
    # leak checking needs ptrace-free stack unwinding of the HIP runtime's
    # threads; the checks are about the library's own accesses
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    return subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)


if __name__ == "__main__":
    proc = run(build())
    sys.stdout.write(proc.stdout)
    sys.stderr.write(proc.stderr)
    sys.exit(proc.returncode)
