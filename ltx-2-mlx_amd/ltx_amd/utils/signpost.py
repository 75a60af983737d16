"""Phase ranges of the transformer block for ROCm profilers (rocTX).

The MI355X counterpart of the reference's os_signpost wrapper
(LTX_2_MLX/utils/signpost.py:68-121, wired at
model/transformer/transformer.py:457-650): the same phase names, the same
switches, the same API -- ``with signpost("video_self_attn"): ...`` and
``signpost_barrier(*tensors)``.

* ``LTX_PROFILE_SIGNPOSTS=1`` turns it on; unset, ``signpost`` is a no-op
  that loads nothing and formats nothing.
* Ranges are rocTX ranges (``roctxRangePushA`` / ``roctxRangePop`` of
  rocprofiler-sdk's ``librocprofiler-sdk-roctx.so``), recorded by
  ``rocprofv3 --marker-trace`` beside the kernels of the same process.
* ``LTX_PROFILE_SIGNPOST_LOG=<path>``: a sidecar log, one line per event,
  ``<ns> <begin|end> <phase>`` on ``time.monotonic_ns()``.
* ``LTX_PROFILE_SIGNPOSTS_SYNC=1``: ``signpost_barrier`` synchronises the
  device, so a range ends when the GPU has finished the phase rather than
  when the host has enqueued it (kernels run asynchronously on HIP streams,
  as MLX's lazy graph does on Metal).
"""

from __future__ import annotations

import ctypes
import os
import threading
import time
from collections.abc import Iterator
from contextlib import contextmanager

# The eight sub-layers of BasicAVTransformerBlock and the sub-phases nested in
# them (the reference's phase list).
PHASES = (
    "video_self_attn",
    "video_text_ca",
    "audio_self_attn",
    "audio_text_ca",
    "a2v_cross",
    "v2a_cross",
    "video_ff",
    "audio_ff",
    "attn_qkv",
    "attn_sdpa",
    "attn_out",
    "v_ff_adaln",
    "v_ff_inner",
)

_lock = threading.Lock()
_init_done = False
_roctx: ctypes.CDLL | None = None
_log_fh = None
_sync = False


def _init() -> None:
    global _init_done, _roctx, _log_fh, _sync
    if _init_done:
        return
    with _lock:
        if _init_done:
            return
        _init_done = True
        if not os.environ.get("LTX_PROFILE_SIGNPOSTS"):
            return
        path = os.environ.get("LTX_PROFILE_SIGNPOST_LOG")
        if path:
            _log_fh = open(path, "w", buffering=1)
            _log_fh.write(f"# LTX signpost log  pid={os.getpid()}  phases={','.join(PHASES)}\n")
        # rocprofiler-sdk's rocTX (what rocprofv3 --marker-trace records) first,
        # the roctracer-era library after it
        lib_dir = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
        for name in ("librocprofiler-sdk-roctx.so", os.path.join(lib_dir, "librocprofiler-sdk-roctx.so"),
                     "libroctx64.so", os.path.join(lib_dir, "libroctx64.so")):
            try:
                lib = ctypes.CDLL(name)
            except OSError:
                continue
            lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            lib.roctxRangePushA.restype = ctypes.c_int
            lib.roctxRangePop.argtypes = []
            lib.roctxRangePop.restype = ctypes.c_int
            _roctx = lib
            break
        _sync = bool(os.environ.get("LTX_PROFILE_SIGNPOSTS_SYNC"))


def enabled() -> bool:
    """Whether phase ranges are recorded (rocTX loaded or a sidecar log open)."""
    _init()
    return _roctx is not None or _log_fh is not None


def begin(phase: str | None) -> None:
    """Open the range of ``phase`` (None or an unknown name: nothing)."""
    _init()
    if _roctx is None and _log_fh is None:
        return
    if phase not in PHASES:
        return
    if _roctx is not None:
        _roctx.roctxRangePushA(phase.encode())
    if _log_fh is not None:
        _log_fh.write(f"{time.monotonic_ns()} begin {phase}\n")


def end(phase: str | None) -> None:
    """Close the range that ``begin(phase)`` opened."""
    if _roctx is None and _log_fh is None:
        return
    if phase not in PHASES:
        return
    if _roctx is not None:
        _roctx.roctxRangePop()
    if _log_fh is not None:
        _log_fh.write(f"{time.monotonic_ns()} end {phase}\n")


@contextmanager
def signpost(phase: str) -> Iterator[None]:
    """A rocTX range (and sidecar-log interval) around a block of code; free
    when ``LTX_PROFILE_SIGNPOSTS`` is unset."""
    begin(phase)
    try:
        yield
    finally:
        end(phase)


def signpost_barrier(*tensors) -> None:
    """With ``LTX_PROFILE_SIGNPOSTS_SYNC=1``, wait until the device has finished
    the work enqueued so far (the tensors name the phase's outputs, as in the
    reference); otherwise nothing."""
    _init()
    if not _sync:
        return
    import torch

    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            torch.cuda.synchronize(t.device)
            return
    if torch.cuda.is_available():
        torch.cuda.synchronize()
