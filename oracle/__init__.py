"""CPU oracle for the fxpr fixed-point reduction kernels.

TEST INFRASTRUCTURE ONLY. This package is a numpy restatement of the
reference algorithms (Gursukh/vLLM-Triton-Fixed-Point-Reductions, package
fxpr_vllm) and of the semantics this build defines where the reference has no
code. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker (or the timed CPU baseline). The product
package (fxpr_vllm) never imports it and has no CPU fallback.

Every function cites the reference file:line it follows. How each function's
parity is pinned (reference known-answer values, closed forms, brute force,
invariants) is listed in tests/test_oracle_*.py; functions whose absolute bits
no reference artefact can pin say "parity unpinned" in their docstring and
are pinned by tolerance and invariants only.

Modules:
    numerics   fp32/bf16/f16 rounding helpers, float_to_fixed,
               fixed_to_float, fixed_row_sum, exp_scaled, log_own
    rows       rms_norm (+residual), log_softmax
    gemm       gemm_fxp emulation
    attention  unified paged attention emulation
"""
