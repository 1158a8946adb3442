"""CPU oracle for the block-FP8 GEMM -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline).  The
product (fp8_gemm_h20) never imports it and has no CPU fallback.

blockfp8.py restates, in numpy:
  * OCP e4m3 ("float8_e4m3fn") decode/encode and fp32 -> bf16 RNE rounding;
  * the reference math C = bf16(dequant(A, As) @ dequant(B, Bs)^T) with fp32
    accumulation (reference scripts/validate.py:32-34, bench.py:25-30);
  * the accuracy metric max|C - C_ref| / max|C_ref| (validate.py:36-37) and
    cosine similarity;
  * the quantisation recipe amax/448 per 1x128 / 128x128 block
    (validate.py:26-29).
How each function is pinned (tests/test_oracle.py): e4m3 decode exhaustively
against torch's float8_e4m3fn and the OCP special values; encode and bf16
rounding against torch on dense value sweeps including ties; the GEMM against
a float64 brute-force triple loop, closed forms (one-hot weights, zero
activations) and exact invariants (power-of-two scale linearity, row
independence, non-square shapes that fail a transposed operand).
"""
