"""Oracle: CPU restatement of the LTX-2-MLX denoise-path algorithms.

THIS PACKAGE IS TEST INFRASTRUCTURE.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker (or, for ``cpu_baseline``, as the timed CPU
baseline).  The product path (``ltx-2-mlx_amd/ltx_amd``) never imports it.

The reference (Python on MLX 0.31.2, Python >= 3.14, Apple Metal) cannot run
in this environment, so every function here is restated from the reference
source text and cites the file:line it follows (paths relative to the
LTX-2-MLX tree).  Rounding points follow the reference's ``.astype`` casts:
``bf16r`` marks each place where the reference rounds to bfloat16.

Pinning: each function is checked in ``tests/test_oracle_*.py`` against the
reference's own known answers where they exist (distilled sigma constants,
E4M3 0x38 -> 1.0, fallback equalities), against library routines for the
special cases that reduce to them (torch bfloat16 / float8_e4m3fn casts,
float64 matmul and softmax), and against invariants that a dropped term or a
wrong index breaks (identity rotations, norm preservation, gate=0 identity,
brute-force minimisation).  Functions with no such check are marked
"parity unpinned" in their docstring.
"""
