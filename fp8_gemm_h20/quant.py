"""Block quantisation helpers and the seeded synthetic-input recipe (torch, any device).

quantize_per_token_group: x[M,K] -> (e4m3 [M,K], fp32 As[M,K/128]), one scale
    per 1x128 K group (the layout SGLang's per-token-group quantiser hands to
    the reference adapter, sgl_patch/fp8mm_sglang_patch.py:51-53).
quantize_per_block: w[N,K] -> (e4m3 [N,K], fp32 Bs[N/128,K/128]), one scale
    per 128x128 block.
Both use scale = max(amax, eps) / 448 and q = e4m3(x / scale)
(reference scripts/validate.py:26-29, test_correct.py:26-30).

make_inputs(M, N, K, seed=..., mode=...) builds one GEMM's operands following
the benchmark recipe: activations bf16 N(0,1), weights N(0,0.02) rounded to
bf16, drawn on the CPU from torch.Generator(seed) and quantised on the CPU, so
identical on every machine; then moved to `device`.
"""
import math

E4M3_MAX = 448.0
GROUP = 128

MODES = ("normal", "outlier_rows", "outlier_cols", "skew", "zero")


def quantize_per_token_group(x, eps=1e-6):
    import torch
    m, k = x.shape
    xf = x.float().view(m, k // GROUP, GROUP)
    s = xf.abs().amax(-1).clamp_min(eps) / E4M3_MAX
    q = (xf / s[..., None]).reshape(m, k).to(torch.float8_e4m3fn)
    return q, s.contiguous()


def quantize_per_block(w, eps=1e-6):
    import torch
    n, k = w.shape
    wf = w.float().view(n // GROUP, GROUP, k // GROUP, GROUP)
    s = wf.abs().amax((1, 3)).clamp_min(eps) / E4M3_MAX
    q = (wf / s[:, None, :, None]).reshape(n, k).to(torch.float8_e4m3fn)
    return q, s.contiguous()


def outlier_rows(m, gen):
    """Rows scaled x50 in mode 'outlier_rows': max(1, round(0.01*M)) distinct rows."""
    import torch
    count = max(1, int(math.floor(0.01 * m + 0.5)))
    return torch.randperm(m, generator=gen)[:count]


def sample(m, n, k, seed, mode="normal"):
    """Unquantised fp32 activations [M,K] and weights [N,K] (values are bf16-exact)."""
    import torch
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}")
    gen = torch.Generator().manual_seed(int(seed))
    a = torch.randn(m, k, generator=gen).to(torch.bfloat16).float()
    b = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).float()
    if mode == "outlier_rows":      # 1% outlier tokens x50 (decode regime)
        a[outlier_rows(m, gen)] *= 50.0
    elif mode == "outlier_cols":    # hot channels (scripts/validate.py:23)
        a[:, ::127] *= 100.0
    elif mode == "skew":            # weight blocks spanning 4 decades (validate.py:24)
        b *= torch.logspace(-3, 1, n // GROUP).repeat_interleave(GROUP)[:, None]
    elif mode == "zero":            # all-zero activations (validate.py:25)
        a.zero_()
    return a, b


def make_inputs(m, n, k, *, seed=None, mode="normal", device="cuda"):
    """(A, B, As, Bs) for one GEMM; default seed M+N+K+113 (scripts/validate.py:59)."""
    if seed is None:
        seed = m + n + k + 113
    a, b = sample(m, n, k, seed, mode)
    A, As = quantize_per_token_group(a)
    B, Bs = quantize_per_block(b)
    return tuple(t.to(device) for t in (A, B, As, Bs))
