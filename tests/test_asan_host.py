"""The C ABI's host code under AddressSanitizer (CPU only).

``ltx-2-mlx_amd/asan/build.py`` compiles every library source with
``-fsanitize=address`` on the host side and links ``host_checks.cpp``, which
drives every entry point through its argument-validation paths (null
pointers, unsupported shapes, misalignment, empty problems, workspace and
padding helpers) and then, where no GPU is present, makes valid calls at the
workloads' shapes (every GEMM tile choice and epilogue, split counts, the
few-row and MX forms, every attention call shape with its split-KV
workspace and the no-allocation scratch, the row kernels, guidance and
latent kernels): their host code runs up to the kernel launch, which the
HIP runtime refuses for want of a device.  The first build takes about a
minute and a half; later runs reuse the objects.
"""

from __future__ import annotations

import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _builder():
    sys.path.insert(0, str(ROOT / "ltx-2-mlx_amd" / "asan"))
    try:
        import build as asan_build  # noqa: PLC0415
    finally:
        sys.path.pop(0)
    return asan_build


@pytest.mark.timeout(900)
def test_host_checks_clean_under_address_sanitizer():
    if shutil.which("/opt/rocm/bin/hipcc") is None:
        pytest.skip("hipcc not available")
    b = _builder()
    exe = b.build()
    proc = b.run(exe)
    assert "AddressSanitizer" not in proc.stderr, proc.stderr[-3000:]
    assert proc.returncode == 0, proc.stdout + proc.stderr[-2000:]
    assert "ok: 0 failure(s)" in proc.stdout
    # and the instrumentation is live: a planted one-byte heap overrun is caught
    bad = subprocess.run([str(exe), "--overflow-selftest"], capture_output=True, text=True, timeout=120,
                         env={"ASAN_OPTIONS": "detect_leaks=0"})
    assert bad.returncode != 0 and "heap-buffer-overflow" in bad.stderr
