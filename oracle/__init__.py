"""CPU oracle for the fxpr fixed-point reduction kernels.

TEST INFRASTRUCTURE ONLY. This package is a numpy restatement of the
reference algorithms (Gursukh/vLLM-Triton-Fixed-Point-Reductions, package
fxpr_vllm) and of the semantics this build defines where the reference has no
code. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker (or the timed CPU baseline). The product
package (fxpr_vllm) never imports it and has no CPU fallback.

Every function cites the reference file:line it follows. How each function's
parity is pinned (reference known-answer values, closed forms, brute force,
invariants) is listed in tests/test_oracle_*.py.

Parity unpinned (bit level): gemm.gemm and attention.unified_attention on
general inputs. The order of the fp32 additions inside one K-tile (GEMM) or
one key tile (attention) belongs to the matrix hardware (NVIDIA mma in the
reference, MFMA on MI355X, BLAS here), and the reference's exp2 is NVIDIA
libdevice; no artefact of the reference fixes those bits. They are pinned by
tolerance, by exact results on inputs whose tile dot products are exact in
fp32, and by exact invariants (tile permutation, batch, split count).

Modules:
    numerics   fp32/bf16/f16 rounding helpers, float_to_fixed,
               fixed_to_float, fixed_row_sum, exp_scaled, log_own
    rows       rms_norm (+residual), log_softmax
    gemm       gemm_fxp emulation
    attention  unified paged attention emulation
"""
