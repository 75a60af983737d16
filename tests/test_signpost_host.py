"""Phase ranges (ltx_amd.utils.signpost), the counterpart of the reference's
os_signpost wrapper (LTX_2_MLX/utils/signpost.py:68-121): free and silent
when LTX_PROFILE_SIGNPOSTS is unset; with it set, a sidecar log of nested
begin / end events in the reference's line format, and rocTX ranges when
libroctx64 loads.  CPU only: each case runs in a fresh interpreter so the
module's one-time set-up sees the environment under test."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "ltx-2-mlx_amd"

SCRIPT = """
import sys
sys.path.insert(0, {pkg!r})
from ltx_amd.utils import signpost as sp
with sp.signpost("video_ff"):
    with sp.signpost("v_ff_adaln"):
        pass
    sp.begin("v_ff_inner"); sp.end("v_ff_inner")
sp.begin("not_a_phase"); sp.end("not_a_phase")
sp.begin(None); sp.end(None)
sp.signpost_barrier()
print("enabled", sp.enabled())
"""


def _run(env_extra: dict, tmp: Path) -> str:
    env = {k: v for k, v in os.environ.items() if not k.startswith("LTX_PROFILE")}
    env.update(env_extra)
    proc = subprocess.run([sys.executable, "-c", SCRIPT.format(pkg=str(PKG))], env=env, capture_output=True,
                          text=True, timeout=120, cwd=tmp)
    assert proc.returncode == 0, proc.stderr
    return proc.stdout


def test_signposts_off_by_default(tmp_path):
    assert "enabled False" in _run({}, tmp_path)


def test_signpost_sidecar_log_nests_phases(tmp_path):
    log = tmp_path / "sp.log"
    out = _run({"LTX_PROFILE_SIGNPOSTS": "1", "LTX_PROFILE_SIGNPOST_LOG": str(log)}, tmp_path)
    assert "enabled True" in out
    lines = [ln.split() for ln in log.read_text().splitlines() if not ln.startswith("#")]
    assert [(k, p) for _, k, p in lines] == [("begin", "video_ff"), ("begin", "v_ff_adaln"), ("end", "v_ff_adaln"),
                                            ("begin", "v_ff_inner"), ("end", "v_ff_inner"), ("end", "video_ff")]
    stamps = [int(t) for t, _, _ in lines]
    assert stamps == sorted(stamps)
