"""The reference's CPU dequant-matmul in torch -- TEST INFRASTRUCTURE ONLY.

C = bf16( (A.float() * As) @ (B.float() * Bs).T ) on the CPU in fp32, the
expression of the reference's scripts/validate.py:32-34 followed by the bf16
cast of its bench.py:30.  bench.py times it as the CPU baseline; it is pinned
against the numpy oracle (blockfp8.dequant_matmul) in tests/test_oracle.py.
"""


def dequant_matmul_bf16(A, B, As, Bs):
    """A[M,K], B[N,K] float8_e4m3fn CPU tensors, As[M,K/128], Bs[N/128,K/128] fp32 -> bf16 [M,N]."""
    import torch
    m, k = A.shape
    n = B.shape[0]
    a = (A.float().view(m, k // 128, 128) * As[..., None]).reshape(m, k)
    b = (B.float().view(n // 128, 128, k // 128, 128) * Bs[:, None, :, None]).reshape(n, k)
    return (a @ b.T).to(torch.bfloat16)
