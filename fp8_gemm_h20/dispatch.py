"""Validated public entry point (reference fp8_gemm_h20/dispatch.py:5-30)."""
from .config import _has_fused_table, _select, _select_fused
from .engine import run

_SHUF_BLOCK = 2048      # bytes of one 16-row x 128-K block of a shuffled weight


def _shuffled(B):
    return B.ndim == 3 and B.shape[2] == _SHUF_BLOCK


def _weight_dims(B):
    """(N, K) of a row-major [N, K] weight or of a shuffled one."""
    return (B.shape[0] * 16, B.shape[1] * 128) if _shuffled(B) else tuple(B.shape)


def matmul(A, B, As, Bs, *, profile="35b_tp1", bias=None, out=None):
    """FP8 A[M,K], B[N,K] with fp32 block scales -> bf16 C[M,N] on A's device.

    Checks run in the reference's order and raise ValueError with its
    messages (dispatch.py:12-27); scale strides are not restricted.  Shapes
    outside the profile and M outside 1..16384 raise ValueError.  There is
    no fallback: the gfx950 HIP library must be built.

    Additions to the reference signature (defaults keep its behaviour):
    `bias` - bf16 [N] added in the kernel epilogue, bit-identical to a
    separate bf16 `C + bias` (the adapter's sgl_patch/fp8mm_sglang_patch.py:55-56);
    `out` - a contiguous bf16 [M, N] tensor on A's device to write into
    instead of allocating C (returned);
    B may also be the [N/16, K/128, 2048] tensor that shuffle_weight returns
    (same C, bit for bit; faster weight loads at small M).
    """
    import torch
    if A.ndim != 2 or (B.ndim != 2 and not _shuffled(B)):
        raise ValueError("A and B must be rank-2 tensors")
    m, k = A.shape
    n, bk = _weight_dims(B)
    if k != bk or k % 128 or n % 128:
        raise ValueError("A/B dimensions must match and N,K must be multiples of 128")
    if A.dtype != torch.float8_e4m3fn or B.dtype != torch.float8_e4m3fn:
        raise ValueError("A and B must be float8_e4m3fn")
    if not A.is_cuda or any(t.device != A.device for t in (B, As, Bs)):
        raise ValueError("All tensors must reside on the same CUDA device")
    if not A.is_contiguous() or not B.is_contiguous():
        raise ValueError("A and B must be contiguous row-major tensors")
    if As.dtype != torch.float32 or Bs.dtype != torch.float32:
        raise ValueError("Scales must be float32")
    if tuple(As.shape) != (m, k // 128) or tuple(Bs.shape) != (n // 128, k // 128):
        raise ValueError("Expected As[M,K/128] and Bs[N/128,K/128]")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (n,)
                             or bias.device != A.device or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous bfloat16 [N] tensor on A's device")
    if out is not None and (out.dtype != torch.bfloat16 or tuple(out.shape) != (m, n)
                            or out.device != A.device or not out.is_contiguous()):
        raise ValueError("out must be a contiguous bfloat16 [M, N] tensor on A's device")
    entry, _ = _select(profile, m, n, k)
    with torch.cuda.device(A.device):
        if bias is None and out is None:
            return run(entry, (A, B, As, Bs))
        return run(entry, (A, B, As, Bs), bias=bias, out=out)


def shuffle_weight(B):
    """e4m3 B[N, K] -> the same weight in the shuffled layout, a new
    [N/16, K/128, 2048] tensor that matmul and linear take in place of B.

    Each 2048-byte block holds 16 rows x 128 K of B in the order the MFMA
    operands are loaded (C ABI fp8bg_shuffle_b), so the kernels read the
    weights coalesced and use them without exchanging bytes between lanes.
    The result of every GEMM is bitwise the one with B.  A one-time
    transform for weights that stay resident (one HIP kernel, no host sync);
    no counterpart in the reference, whose adapter keeps B row-major.
    """
    import torch
    from . import kernels
    if B.ndim != 2 or B.dtype != torch.float8_e4m3fn or not B.is_cuda or not B.is_contiguous():
        raise ValueError("B must be a contiguous rank-2 float8_e4m3fn CUDA tensor")
    n, k = B.shape
    if n % 128 or k % 128:
        raise ValueError("A/B dimensions must match and N,K must be multiples of 128")
    with torch.cuda.device(B.device):
        return kernels.shuffle_b(B)


def quantize_act(x, *, eps=1e-10, column_major_scales=False):
    """bf16 x[..., K] -> (e4m3 q[M, K], fp32 s[M, K/128]) per 1x128 K group on x's GPU.

    s = max(amax(group), eps) / 448 and q = e4m3(x / s) with round to
    nearest even: the operands the reference's SGLang adapter feeds to
    matmul after sglang_per_token_group_quant_fp8 (eps=1e-10 default there;
    sgl_patch/fp8mm_sglang_patch.py:51-53).  Leading dims of x are flattened
    into M.  column_major_scales=True returns s as the transposed view of a
    [K/128, M] buffer (same values).  One HIP kernel, no host sync.
    """
    import torch
    from . import kernels
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("x must be a bfloat16 CUDA tensor")
    k = x.shape[-1]
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    x2 = x.reshape(-1, k)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.clone(memory_format=torch.contiguous_format)    # kernel reads 16-byte row chunks
    m = x2.shape[0]
    if m < 1:
        raise ValueError("x must have at least one row")
    with torch.cuda.device(x.device):
        return kernels.quant_act(x2, m, k, eps, column_major_scales)


def linear(x, B, Bs, *, profile="35b_tp1", bias=None, eps=1e-10, fused=None):
    """y = x @ dequant(B, Bs)^T (+ bias) for bf16 activations x[..., K].

    The dense block-FP8 linear of the reference's SGLang adapter
    (fp8mm_w8a8_block_fp8_linear, sgl_patch/fp8mm_sglang_patch.py:34-57):
    per-token-group quantisation of x, matmul with the bias added in the
    kernel epilogue (bit-identical to the adapter's `out + bias`), and the
    result viewed as x.shape[:-1] + (N,).  No host sync.  Shapes the profile
    does not cover raise ValueError (the adapter's own fallback decision
    stays with the caller, as `supports` answers it).

    At decode sizes the quantiser can run inside the GEMM kernel (one launch
    instead of two, fp8bg_gemm_bf16a); its codes are e4m3(x * (1/s)) rather
    than e4m3(x / s), equal except on rare rounding ties of the two
    quotients.  Where the profile has a fused table for (N, K), its entry for
    M decides: the fused launch runs when it measured faster than the two
    kernels ("use").  Without one, the fused launch runs where the matmul
    entry itself is a skinny configuration with a fused instance.
    fused=False forces the two-kernel path, fused=True the fused one
    (ValueError where no fused configuration applies).  B may be a shuffled
    weight (shuffle_weight).
    """
    import torch
    from . import kernels
    n, k = _weight_dims(B)
    if fused is not False and x.dtype == torch.bfloat16 and x.is_cuda and x.shape[-1] == k \
            and x.numel() > 0:
        m = x.numel() // k
        cfg, use = _fused_choice(profile, m, n, k)
        ok = cfg is not None and eps >= 1e-30
        if fused and not ok:
            raise ValueError("no fused-quantiser configuration for this shape in the profile; "
                             "the fused linear does not apply")
        if ok and (use or fused):
            _check_weights(B, Bs, x.device, bias)
            x2 = x.reshape(-1, k)
            if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
                x2 = x2.clone(memory_format=torch.contiguous_format)
            with torch.cuda.device(x.device):
                out = kernels.linear_fused(x2, B, Bs, cfg, eps, bias=bias)
            return out.view(*x.shape[:-1], n)
    elif fused:
        raise ValueError("fused linear needs bf16 CUDA activations with last dim K")
    q, s = quantize_act(x, eps=eps)
    out = matmul(q, B, s, Bs, profile=profile, bias=bias)
    return out.view(*x.shape[:-1], n)


def _fused_choice(profile, m, n, k):
    """(config, use) of the fused-quantiser launch for (M, N, K): from the
    profile's fused table where it has one for (N, K), else the matmul entry
    when that is a skinny configuration with a fused instance; (None, False)
    where neither applies."""
    from . import kernels
    if _has_fused_table(profile, n, k):
        entry = _select_fused(profile, m, n, k)
        return (None, False) if entry is None else (dict(entry["config"]), entry["use"])
    entry, _ = _select(profile, m, n, k)
    return (dict(entry["config"]), True) if kernels.fused_config_ok(entry) else (None, False)


def _check_weights(B, Bs, device, bias):
    """Weight-side checks of matmul (dispatch.py:12-27 order) for the fused linear."""
    import torch
    if B.ndim != 2 and not _shuffled(B):
        raise ValueError("A and B must be rank-2 tensors")
    n, k = _weight_dims(B)
    if k % 128 or n % 128:
        raise ValueError("A/B dimensions must match and N,K must be multiples of 128")
    if B.dtype != torch.float8_e4m3fn:
        raise ValueError("A and B must be float8_e4m3fn")
    if B.device != device or Bs.device != device:
        raise ValueError("All tensors must reside on the same CUDA device")
    if not B.is_contiguous():
        raise ValueError("A and B must be contiguous row-major tensors")
    if Bs.dtype != torch.float32:
        raise ValueError("Scales must be float32")
    if tuple(Bs.shape) != (n // 128, k // 128):
        raise ValueError("Expected As[M,K/128] and Bs[N/128,K/128]")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (n,)
                             or bias.device != device or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous bfloat16 [N] tensor on A's device")
