"""numpy restatement of the block-FP8 GEMM math (test infrastructure only; see __init__)."""
import numpy as np

GROUP = 128
E4M3_MAX = 448.0


def _e4m3_table():
    # OCP 8-bit FP (E4M3, "fn" variant): bias 7, no infinities, S.1111.111 = NaN.
    t = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            t[code] = np.nan
        elif e == 0:
            t[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t.astype(np.float32)


E4M3_TABLE = _e4m3_table()


def e4m3_decode(u8):
    """uint8 codes -> float32 values."""
    return E4M3_TABLE[np.asarray(u8, dtype=np.uint8)]


def e4m3_encode(x):
    """float32 -> e4m3fn codes, round to nearest even.

    Matches torch's float -> float8_e4m3fn cast: results above 448 after
    rounding (|x| > 464) and +-inf become NaN (0x7F with the sign), NaN stays
    NaN.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = (np.signbit(x).astype(np.uint8)) << 7
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -6.0)                       # subnormals share the 2^-6 binade quantum
    quantum = np.exp2(e - 3.0)
    with np.errstate(invalid="ignore"):
        q = np.rint(a / quantum) * quantum        # rint = round half to even
    out = np.zeros(x.shape, dtype=np.uint8)
    nan = np.isnan(x) | np.isinf(x) | ~(q <= E4M3_MAX)
    sub = (q > 0) & (q < 2.0 ** -6) & ~nan
    out[sub] = np.rint(q[sub] / 2.0 ** -9).astype(np.uint8)
    nrm = (q >= 2.0 ** -6) & ~nan
    en = np.floor(np.log2(q[nrm]))
    mant = np.rint((q[nrm] / np.exp2(en) - 1.0) * 8.0).astype(np.int64)
    out[nrm] = (((en + 7).astype(np.int64) << 3) | mant).astype(np.uint8)
    out[nan] = 0x7F
    return out | sign


def bf16_bits(x):
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even; NaN -> 0x7FC0."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = r.astype(np.uint16)
    r[np.isnan(np.asarray(x, dtype=np.float32))] = 0x7FC0
    return r


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant_a(A, As):
    m, k = A.shape
    a = e4m3_decode(A).reshape(m, k // GROUP, GROUP) * np.asarray(As, np.float32)[:, :, None]
    return a.reshape(m, k)


def dequant_b(B, Bs):
    n, k = B.shape
    b = e4m3_decode(B).reshape(n // GROUP, GROUP, k // GROUP, GROUP)
    b = b * np.asarray(Bs, np.float32)[:, None, :, None]
    return b.reshape(n, k)


def dequant_matmul(A, B, As, Bs, dtype=np.float32):
    """fp32 (or float64) dequant(A,As) @ dequant(B,Bs)^T (reference validate.py:32-34)."""
    a = dequant_a(A, As).astype(dtype)
    b = dequant_b(B, Bs).astype(dtype)
    return a @ b.T


def reference_bf16(A, B, As, Bs):
    """bf16 bits of the fp32 reference (reference bench.py:25-30)."""
    return bf16_bits(dequant_matmul(A, B, As, Bs))


def brute_force(A, B, As, Bs):
    """float64 scalar triple loop over dequantised elements; tiny inputs only."""
    m, k = A.shape
    n = B.shape[0]
    da = e4m3_decode(A).astype(np.float64)
    db = e4m3_decode(B).astype(np.float64)
    out = np.zeros((m, n), dtype=np.float64)
    for i in range(m):
        for j in range(n):
            s = 0.0
            for kk in range(k):
                g = kk // GROUP
                s += (da[i, kk] * float(As[i, g])) * (db[j, kk] * float(Bs[j // GROUP, g]))
            out[i, j] = s
    return out


def error(out, ref):
    """max|out - ref| / max(max|ref|, 1e-30) (reference validate.py:36-37)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-30))


def cosine(out, ref):
    out = np.asarray(out, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.linalg.norm(out) * np.linalg.norm(ref)
    return float(out @ ref / den) if den > 0 else float("nan")


def quantize_act(x, eps=1e-6):
    """x[M,K] fp32 -> (e4m3 codes [M,K], As[M,K/128]); scale = max(amax, eps)/448."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    xg = x.reshape(m, k // GROUP, GROUP)
    s = (np.maximum(np.abs(xg).max(-1), np.float32(eps)) / np.float32(E4M3_MAX)).astype(np.float32)
    q = e4m3_encode((xg / s[:, :, None]).astype(np.float32)).reshape(m, k)
    return q, s


def quantize_act_reciprocal(x, eps=1e-10):
    """The fused-quantiser GEMM's activation recipe (fp8bg_gemm_bf16a):
    scales as quantize_act, codes e4m3(x * (1/s)) with 1/s and the product
    rounded to fp32.  It differs from quantize_act's x / s only where the two
    fp32 values straddle an e4m3 rounding boundary."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    xg = x.reshape(m, k // GROUP, GROUP)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        s = (np.maximum(np.abs(xg).max(-1), np.float32(eps)) / np.float32(E4M3_MAX)).astype(np.float32)
        r = (np.float32(1) / s).astype(np.float32)
        q = e4m3_encode((xg * r[:, :, None]).astype(np.float32)).reshape(m, k)
    return q, s


def quantize_weight(w, eps=1e-6):
    """w[N,K] fp32 -> (e4m3 codes [N,K], Bs[N/128,K/128]) per 128x128 block."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    wb = w.reshape(n // GROUP, GROUP, k // GROUP, GROUP)
    s = (np.maximum(np.abs(wb).max((1, 3)), np.float32(eps)) / np.float32(E4M3_MAX)).astype(np.float32)
    q = e4m3_encode((wb / s[:, None, :, None]).astype(np.float32)).reshape(n, k)
    return q, s
