"""Host functions of the kernel registry: fn(A, B, As, Bs, config) -> C.

Each function keeps the reference's L0 wrapper contract
(fp8_gemm_h20/engine.py:18-19): A[M,K], B[N,K] contiguous e4m3fn CUDA tensors,
As[M,K/128] and Bs[N/128,K/128] fp32 with any strides, `config` a plain dict;
it allocates C = empty(M, N, bf16) on A's device, enqueues the HIP kernel(s)
on the current stream through the C ABI (include/fp8bg.h) and returns C
without synchronising.  Optional keywords (beyond the reference contract):
`bias` (bf16 [N], added in the epilogue like a separate bf16 `C + bias`) and
`out` (a bf16 [M, N] contiguous buffer to write instead of allocating).

Two families of config dicts are accepted:

* gfx950-native entries written by this package's tuner:
  - impl "tiled": BLOCK_W, BLOCK_T, WAVES_W, WAVES_T, SPLIT, SPLIT_MODE,
    GROUP_SIZE_M, SCALE_LDS, XCD_REMAP, LDS_SWIZZLE (LDS-tiled kernel);
  - impl "skinny": BLOCK_W, BLOCK_T, WAVES_K, UNROLL, SPLIT, SPLIT_MODE
    ("none", "full" or "last": the split reduced inside the kernel),
    XCD_REMAP (small-M kernel, waves split K);
  - impl "ring": BLOCK_W, BLOCK_T, WAVES_W, WAVES_T, STAGES, K_UNROLL, WAVES_K, SPLIT,
    SPLIT_MODE ("none", "tail", "full", "last" on token tiles up to 64, or
    "stream": stream-K), GROUP_SIZE_M, XCD_REMAP, LDS_SWIZZLE (direct-to-LDS
    ring kernel);
  - impl "shortk": BLOCK_W, BLOCK_T (K == 256, no K loop).
* the reference's H20 entries (impl "triton", "gluon", "v2", "scale_tma",
  "shortk" with BM/BN keys), translated onto the nearest compiled gfx950 tile
  so that an existing reference profile table still runs unchanged.
"""
import ctypes
from functools import lru_cache

from . import _lib

# Compiled kernel instances; must equal FP8BG_TILED / FP8BG_SKINNY in
# csrc/fp8bg.hip (checked by tests).
# tiled: (block_w, block_t, waves_w, waves_t, k_fixed)
TILED = (
    (64, 16, 4, 1, 0), (128, 16, 4, 1, 0), (256, 16, 4, 1, 0),
    (64, 32, 4, 1, 0), (128, 32, 4, 1, 0), (256, 32, 4, 1, 0),
    (64, 64, 4, 1, 0), (128, 64, 4, 1, 0), (256, 64, 4, 1, 0),
    (128, 64, 2, 2, 0), (128, 128, 2, 2, 0), (128, 128, 4, 1, 0),
    (256, 128, 4, 1, 0), (256, 128, 2, 2, 0), (128, 256, 2, 2, 0),
    (64, 16, 4, 1, 2), (128, 16, 4, 1, 2), (64, 32, 4, 1, 2),
    (128, 32, 4, 1, 2), (128, 64, 4, 1, 2), (128, 128, 2, 2, 2),
    (256, 128, 4, 1, 2),
)
# skinny: (16-row weight blocks, 16-token blocks, waves_k, unroll)
SKINNY = (
    (1, 1, 4, 1), (1, 1, 4, 2), (1, 1, 8, 1), (1, 1, 8, 2), (1, 1, 8, 4),
    (2, 1, 4, 1), (2, 1, 4, 2), (2, 1, 8, 1), (2, 1, 8, 2), (2, 1, 8, 4),
    (4, 1, 4, 1), (4, 1, 4, 2), (4, 1, 8, 1), (4, 1, 8, 2), (4, 1, 8, 4),
    (1, 2, 4, 2), (1, 2, 8, 1), (1, 2, 8, 2),
    (2, 2, 4, 2), (2, 2, 8, 1), (2, 2, 8, 2),
    (4, 2, 4, 2), (4, 2, 8, 1), (4, 2, 8, 2),
    (1, 4, 4, 2), (1, 4, 8, 1), (1, 4, 8, 2),
    (2, 4, 4, 2), (2, 4, 8, 1), (2, 4, 8, 2),
    (4, 4, 4, 1), (4, 4, 8, 1), (4, 4, 4, 2),
    # four waves with four 128-K groups in flight each: every group of a
    # K=2048 wave in one batch (decode)
    (1, 1, 4, 4), (2, 1, 4, 4), (4, 1, 4, 4),
    # sixteen waves splitting K: one or two groups per wave, for shapes with
    # few weight tiles (narrow N) whose waves would otherwise make several
    # dependent memory round trips
    (1, 1, 16, 1), (1, 1, 16, 2), (2, 1, 16, 1), (2, 1, 16, 2), (4, 1, 16, 1),
    (1, 2, 16, 1), (2, 2, 16, 1), (1, 4, 16, 1),
    # 48 weight rows: N = 12288 in 256 tiles, one per CU (a tile may reach
    # into a second 128-row Bs block)
    (3, 1, 4, 1), (3, 1, 4, 2), (3, 1, 8, 1), (3, 1, 8, 2),
    (3, 2, 4, 2), (3, 2, 8, 1), (3, 2, 8, 2),
    (3, 4, 4, 1), (3, 4, 8, 1), (3, 4, 4, 2),
    (3, 1, 16, 1), (3, 2, 16, 1),
    # two waves: K = 256 (two 128-K groups) gives each wave one
    (1, 1, 2, 1), (2, 1, 2, 1),
)
# skinny instances as (block_w, block_t, waves_k, unroll)
SKINNY_TILES = tuple((16 * w, 16 * t, s, u) for w, t, s, u in SKINNY)
# skinny with the activation quantiser fused (16-, 32- and 64-token tiles,
# except those whose bf16 staging would spill); must match FP8BG_SKINNY_QA in
# csrc/fp8bg.hip
SKINNY_QA = tuple(c for c in SKINNY
                  if c not in ((4, 1, 8, 4), (4, 1, 4, 4), (4, 1, 16, 1), (2, 4, 8, 2), (1, 4, 16, 1),
                               (3, 2, 16, 1))
                  and c[0] * c[1] <= 8)
# ring: (block_w, block_t, waves_w, waves_t, stages, k_fixed, groups per barrier,
#        K slices)
RING = (
    (256, 128, 4, 1, 3, 0, 1, 1), (256, 128, 2, 2, 3, 0, 1, 1), (128, 128, 2, 2, 4, 0, 1, 1),
    (128, 128, 4, 1, 4, 0, 1, 1), (128, 128, 2, 2, 3, 0, 1, 1), (128, 64, 2, 2, 4, 0, 1, 1),
    (128, 64, 4, 1, 4, 0, 1, 1), (128, 64, 2, 2, 3, 0, 1, 1), (64, 64, 4, 1, 4, 0, 1, 1),
    (256, 64, 4, 1, 3, 0, 1, 1), (128, 32, 4, 1, 4, 0, 1, 1), (256, 256, 4, 2, 2, 0, 1, 1),
    (256, 128, 4, 2, 3, 0, 1, 1), (256, 128, 4, 2, 2, 0, 1, 1), (128, 256, 2, 4, 2, 0, 1, 1),
    (256, 128, 4, 1, 2, 2, 1, 1), (128, 128, 2, 2, 2, 2, 1, 1),
    (64, 64, 4, 1, 8, 0, 1, 1), (128, 64, 4, 1, 6, 0, 1, 1), (128, 32, 4, 1, 7, 0, 1, 1),
    (128, 128, 2, 2, 2, 0, 1, 1),
    # 192-row weight tiles, 12 waves (3 per SIMD): whole waves of tiles on 256
    # CUs where N is a multiple of 192 (12288, 9216, 4608, 3072)
    (192, 256, 3, 4, 2, 0, 1, 1), (192, 128, 6, 2, 2, 0, 1, 1), (192, 128, 6, 2, 3, 0, 1, 1),
    (192, 128, 3, 4, 3, 0, 1, 1), (192, 64, 6, 2, 4, 0, 1, 1),
    # small tiles with two (or four) 128-K groups per barrier
    (64, 64, 4, 1, 4, 0, 2, 1), (64, 64, 4, 1, 8, 0, 2, 1), (64, 64, 4, 1, 8, 0, 4, 1),
    (128, 64, 4, 1, 4, 0, 2, 1), (128, 64, 4, 1, 6, 0, 2, 1),
    (128, 32, 4, 1, 4, 0, 2, 1), (128, 32, 4, 1, 7, 0, 2, 1),
    (128, 64, 2, 2, 4, 0, 2, 1), (192, 64, 6, 2, 4, 0, 2, 1),
    # K slices: two (or four) groups of waves split a tile's K groups and sum
    # their partial tiles through LDS (narrow N, long K, few workgroups)
    (64, 64, 4, 1, 4, 0, 2, 2), (64, 64, 4, 1, 8, 0, 2, 2),
    (64, 64, 4, 1, 8, 0, 4, 2), (64, 64, 4, 1, 8, 0, 4, 4),
    (128, 64, 4, 1, 6, 0, 2, 2), (128, 32, 4, 1, 4, 0, 2, 2),
    # 8 waves on a 128x128 tile (two per SIMD): mid M with ~256 tiles
    (128, 128, 4, 2, 2, 0, 1, 1), (128, 128, 4, 2, 3, 0, 1, 1), (128, 128, 4, 2, 4, 0, 2, 1),
    # token tiles that are not powers of two, for M that they cover with
    # little waste (M=777 in 5 tiles of 160: 97% of the rows used)
    (256, 160, 4, 2, 2, 0, 1, 1), (256, 192, 4, 2, 2, 0, 1, 1),
    (128, 160, 2, 2, 3, 0, 1, 1), (128, 96, 2, 2, 4, 0, 1, 1),
    # 64x64 with 2x2 waves (two weight blocks per wave)
    (64, 64, 2, 2, 8, 0, 4, 1),
    # 96 weight rows: N = 12288 in 128 tiles, 256 with two token tiles
    # (a tile may span two 128-row Bs blocks)
    (96, 64, 3, 1, 4, 0, 2, 1), (96, 128, 3, 2, 3, 0, 1, 1),
)
# ring instances with the in-kernel split-K reduction (fp8bg_ring_last,
# SPLIT_MODE "last"): token tiles up to 64, no fixed K; must match
# ring_has_last in csrc/fp8bg.hip
RING_LAST = tuple(c for c in RING if c[1] <= 64 and c[5] == 0)
# ring instances with a stream-K kernel (fp8bg_ring_sk, SPLIT_MODE "stream"):
# no fixed K, one K slice, and at most 64 accumulator VGPRs per wave (32 with
# more than 8 waves); must match ring_has_sk in csrc/fp8bg.hip
RING_SK = tuple(c for c in RING if c[5] == 0 and c[7] == 1
                and (c[0] // c[2]) * (c[1] // c[3]) // 64 <= (32 if c[2] * c[3] > 8 else 64))
SPLIT_MODES = {"none": _lib.SPLIT_NONE, "tail": _lib.SPLIT_TAIL, "full": _lib.SPLIT_FULL,
               "last": _lib.SPLIT_LAST, "stream": _lib.SPLIT_STREAM}


def default_waves(block_w, block_t, k_fixed=0):
    """Wave grid of the first compiled tiled instance with this tile."""
    for tw, tt, ww, wt, kf in TILED:
        if (tw, tt, kf) == (block_w, block_t, k_fixed):
            return ww, wt
    return None


def is_compiled(block_w, block_t, waves_w, waves_t, k_fixed=0):
    return (block_w, block_t, waves_w, waves_t, k_fixed) in TILED


def nearest_tile(block_w, block_t, k_fixed=0):
    """Closest compiled tiled (block_w, block_t) for a requested tile.

    Used to run reference (H20) table entries: their tiles (16..64 wide)
    are sized for 78 SMs and warp-level wgmma; gfx950 tiled kernels start at
    64 weight rows.  Preference: keep the token tile, then the nearest weight
    tile.
    """
    best = None
    for tw, tt, _, _, kf in TILED:
        if kf != k_fixed:
            continue
        cost = (abs((tt or 1).bit_length() - max(block_t, 1).bit_length()) * 4
                + abs(tw.bit_length() - max(block_w, 1).bit_length()))
        if best is None or cost < best[0]:
            best = (cost, tw, tt)
    return best[1], best[2]


def _flags(cfg):
    flags = 0
    if cfg.get("SCALE_LDS", False):
        flags |= _lib.FLAG_SCALE_LDS
    if cfg.get("XCD_REMAP", False):
        flags |= _lib.FLAG_XCD_REMAP
    swz = cfg.get("LDS_SWIZZLE", "row16")
    if swz not in ("row8", "row16", "pair"):
        raise ValueError("LDS_SWIZZLE must be one of ('row8', 'row16', 'pair')")
    flags |= {"row16": 0, "row8": _lib.FLAG_SWZ8, "pair": _lib.FLAG_SWZPAIR}[swz]
    return flags


def _split_mode(cfg, default):
    mode = cfg.get("SPLIT_MODE", default)
    if mode not in SPLIT_MODES:
        raise ValueError(f"SPLIT_MODE must be one of {tuple(SPLIT_MODES)}")
    return SPLIT_MODES[mode]


def tiled_struct(cfg, k_fixed=0):
    """C config struct for a tiled (or shortk) config dict."""
    tw, tt = int(cfg["BLOCK_W"]), int(cfg["BLOCK_T"])
    ww, wt = cfg.get("WAVES_W"), cfg.get("WAVES_T")
    if ww is None or wt is None:
        waves = default_waves(tw, tt, k_fixed)
        if waves is None:
            raise ValueError(f"no compiled gfx950 kernel for tile {tw}x{tt} (k_fixed={k_fixed})")
        ww, wt = waves
    return _lib.Config(_lib.KIND_TILED, tw, tt, int(ww), int(wt), 1, 1, 1, int(cfg.get("SPLIT", 1)),
                       _split_mode(cfg, "full"), int(cfg.get("GROUP_SIZE_M", 1)), _flags(cfg), k_fixed)


def skinny_struct(cfg):
    """C config struct for a skinny config dict."""
    return _lib.Config(_lib.KIND_SKINNY, int(cfg["BLOCK_W"]), int(cfg["BLOCK_T"]), 1, 1,
                       int(cfg.get("WAVES_K", 8)), int(cfg.get("UNROLL", 1)), 1,
                       int(cfg.get("SPLIT", 1)), _split_mode(cfg, "none"), 1, _flags(cfg), 0)


def ring_struct(cfg, k_fixed=0):
    """C config struct for a ring config dict (K_UNROLL: 128-K groups per
    barrier; WAVES_K: K slices of waves)."""
    return _lib.Config(_lib.KIND_RING, int(cfg["BLOCK_W"]), int(cfg["BLOCK_T"]),
                       int(cfg["WAVES_W"]), int(cfg["WAVES_T"]), int(cfg.get("WAVES_K", 1)),
                       int(cfg.get("K_UNROLL", 1)),
                       int(cfg["STAGES"]),
                       int(cfg.get("SPLIT", 1)), _split_mode(cfg, "none"),
                       int(cfg.get("GROUP_SIZE_M", 1)), _flags(cfg), k_fixed)



# ---------------------------------------------------------------------------
# device state: CU count and split-K workspaces
# ---------------------------------------------------------------------------
_NUM_CUS = {}


class SplitBuffers:
    """Split-K workspace of one (device, stream) pair (reference
    baseline_gluon.py:229-244): COUNTERS uint32 tile counters, zero when
    allocated and left zero by every call, then the fp32 partials.

    Launches on one stream are ordered, so every split-K GEMM on that stream
    can share one workspace; kernels on different streams never share.

    Growth never frees a buffer: a hipGraph captured earlier holds the old
    device address, and torch.cuda.graph() empties the allocator cache at
    every capture, which would hand freed blocks back to the driver and leave
    such a graph writing to unmapped memory.  Replaced buffers are therefore
    retired (kept alive until the process ends); sizes at least double on each
    growth, so the retired total stays below the live size.
    """

    MIN_WS = 1 << 20

    def __init__(self, device):
        self.device = device
        self.ws = None
        self.retired = []

    def get(self, ws_elems):
        import torch
        if self.ws is None or self.ws.numel() < ws_elems:
            size = max(ws_elems, self.MIN_WS, 2 * (self.ws.numel() if self.ws is not None else 0))
            if self.ws is not None:
                self.retired.append(self.ws)
            self.ws = torch.zeros(size, device=self.device, dtype=torch.float32)
        return self.ws


# (device index, stream handle) -> SplitBuffers
_BUFS = {}


def _device_index(dev):
    import torch
    return dev.index if dev.index is not None else torch.cuda.current_device()


def num_cus(dev):
    idx = _device_index(dev)
    n = _NUM_CUS.get(idx)
    if n is None:
        n = _NUM_CUS[idx] = _lib.num_cus(idx)
    return n


def _workspace(dev, ws_elems):
    import torch
    key = (_device_index(dev), torch.cuda.current_stream(dev).cuda_stream)
    bufs = _BUFS.get(key)
    if bufs is None:
        bufs = _BUFS[key] = SplitBuffers(dev)
    return bufs.get(ws_elems)


# shuffled B (C ABI fp8bg_shuffle_b): N/16 x K/128 blocks of 2048 bytes, held
# as a [N/16, K/128, 2048] e4m3 tensor so that its layout shows in its shape
SHUF_BLOCK = 2048


def is_shuffled(B):
    """True for a weight in the shuffled layout ([N/16, K/128, 2048])."""
    return B.dim() == 3 and B.shape[2] == SHUF_BLOCK


def weight_dims(B):
    """(N, K) of a row-major [N, K] or a shuffled weight."""
    if is_shuffled(B):
        return B.shape[0] * 16, B.shape[1] * 128
    return tuple(B.shape)


def shuffle_b(B):
    """Row-major e4m3 B [N, K] (unit column stride, 16-byte row stride) ->
    the shuffled layout, as a new [N/16, K/128, 2048] tensor on B's device."""
    import torch
    n, k = B.shape
    bt = torch.empty((n // 16, k // 128, SHUF_BLOCK), device=B.device, dtype=B.dtype)
    stream = torch.cuda.current_stream(B.device).cuda_stream
    _lib.check(_lib.lib().fp8bg_shuffle_b(B.data_ptr(), B.stride(0), bt.data_ptr(), n, k, stream))
    return bt


def _layout_struct(cstruct, B):
    """The config struct for B's layout: a copy with FLAG_B_SHUFFLED for a
    shuffled B (tiled configurations do not read it: ValueError)."""
    if not is_shuffled(B):
        return cstruct
    if cstruct.kind == _lib.KIND_TILED:
        raise ValueError("a shuffled B needs a skinny or ring configuration")
    c = _lib.Config.from_buffer_copy(cstruct)
    c.flags |= _lib.FLAG_B_SHUFFLED
    return c


def check_operands(M, N, K, B, As, Bs, bias=None, out=None):
    """The kernels take M, N, K and raw pointers; operands whose shapes
    disagree with them would be read or written out of bounds, so they are
    refused here (ValueError) before anything is launched."""
    b_shape = (N // 16, K // 128, SHUF_BLOCK) if is_shuffled(B) else (N, K)
    if (tuple(B.shape) != b_shape or N % 16 or (As is not None and tuple(As.shape) != (M, K // 128))
            or tuple(Bs.shape) != (N // 128, K // 128)
            or (bias is not None and tuple(bias.shape) != (N,))
            or (out is not None and tuple(out.shape) != (M, N))):
        raise ValueError(f"operand shapes disagree with M,N,K={M},{N},{K}: "
                         f"B{tuple(B.shape)} As{None if As is None else tuple(As.shape)} "
                         f"Bs{tuple(Bs.shape)}")


def launch(A, B, As, Bs, cstruct, bias=None, out=None):
    """Enqueue the kernel(s) described by `cstruct` into `out` (allocated
    when None); `bias` is an optional bf16 [N] added in the epilogue."""
    import torch
    M, K = A.shape
    N = weight_dims(B)[0]
    check_operands(M, N, K, B, As, Bs, bias, out)
    cstruct = _layout_struct(cstruct, B)
    dev = A.device
    cus = num_cus(dev)
    plan = _lib.make_plan(M, N, K, cstruct, cus)
    C = torch.empty((M, N), device=dev, dtype=torch.bfloat16) if out is None else out
    ws_ptr, ws_n = None, 0
    if plan.n_split:
        ws = _workspace(dev, plan.ws_elems)
        ws_ptr, ws_n = ws.data_ptr(), ws.numel()
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(_lib.lib().fp8bg_gemm(
        A.data_ptr(), B.data_ptr(),
        As.data_ptr(), As.stride(0), As.stride(1),
        Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
        None if bias is None else bias.data_ptr(),
        C.data_ptr(), M, N, K, ctypes.byref(cstruct), cus,
        ws_ptr, ws_n, stream))
    return C


def quant_act(x2, m, k, eps, column_major_scales):
    """Launch the activation quantiser on a [M, K] bf16 view (unit column stride)."""
    import torch
    dev = x2.device
    q = torch.empty((m, k), device=dev, dtype=torch.float8_e4m3fn)
    if column_major_scales:
        s = torch.empty((k // 128, m), device=dev, dtype=torch.float32).T
    else:
        s = torch.empty((m, k // 128), device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(_lib.lib().fp8bg_quant_act(x2.data_ptr(), x2.stride(0), q.data_ptr(), s.data_ptr(),
                                          s.stride(0), s.stride(1), m, k, ctypes.c_float(eps), stream))
    return q, s


def linear_fused(x2, B, Bs, config, eps, bias=None, out=None, keep_quantized=False):
    """Decode-size linear in one launch: the skinny kernel with the activation
    quantiser fused (C ABI fp8bg_gemm_bf16a).  `x2` is a [M, K] bf16 view with
    unit column stride; `config` a skinny configuration of a compiled
    fused-quantiser instance (SKINNY_QA).
    Returns C, or (C, q, s) with the codes and scales the kernel used when
    keep_quantized is set."""
    import torch
    m, k = x2.shape
    n = weight_dims(B)[0]
    check_operands(m, n, k, B, None, Bs, bias, out)
    dev = x2.device
    cstruct = _layout_struct(_skinny_cached(_freeze(config)), B)
    cus = num_cus(dev)
    plan = _lib.make_plan(m, n, k, cstruct, cus)
    C = torch.empty((m, n), device=dev, dtype=torch.bfloat16) if out is None else out
    ws_ptr, ws_n = None, 0
    if plan.n_split:
        ws = _workspace(dev, plan.ws_elems)
        ws_ptr, ws_n = ws.data_ptr(), ws.numel()
    q = s = None
    if keep_quantized:
        q = torch.empty((m, k), device=dev, dtype=torch.float8_e4m3fn)
        s = torch.empty((m, k // 128), device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(_lib.lib().fp8bg_gemm_bf16a(
        x2.data_ptr(), x2.stride(0), ctypes.c_float(eps),
        B.data_ptr(), Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
        None if bias is None else bias.data_ptr(),
        C.data_ptr(), m, n, k, ctypes.byref(cstruct), cus, ws_ptr, ws_n,
        None if q is None else q.data_ptr(), None if s is None else s.data_ptr(),
        0 if s is None else s.stride(0), 0 if s is None else s.stride(1), stream))
    return (C, q, s) if keep_quantized else C


def fused_config_ok(entry):
    """True when a table entry can run as the fused-quantiser skinny kernel."""
    c = entry["config"]
    return (entry["impl"] == "skinny"
            and (int(c["BLOCK_W"]) // 16, int(c["BLOCK_T"]) // 16, int(c.get("WAVES_K", 8)),
                 int(c.get("UNROLL", 1))) in SKINNY_QA)


def _freeze(config):
    return tuple(sorted(config.items()))


@lru_cache(maxsize=1024)
def _tiled_cached(items, k_fixed):
    return tiled_struct(dict(items), k_fixed)


@lru_cache(maxsize=1024)
def _skinny_cached(items):
    return skinny_struct(dict(items))


@lru_cache(maxsize=1024)
def _ring_cached(items, k_fixed):
    return ring_struct(dict(items), k_fixed)


# ---------------------------------------------------------------------------
# gfx950-native impls
# ---------------------------------------------------------------------------
def tiled(A, B, As, Bs, config, **epilogue):
    """LDS-tiled MFMA kernel with optional tail/full split-K."""
    return launch(A, B, As, Bs, _tiled_cached(_freeze(config), 0), **epilogue)


def skinny(A, B, As, Bs, config, **epilogue):
    """Small-M kernel: operands straight to registers, waves split K."""
    return launch(A, B, As, Bs, _skinny_cached(_freeze(config)), **epilogue)


def ring(A, B, As, Bs, config, **epilogue):
    """Large-tile kernel: direct-to-LDS ring, one barrier per K group.
    K_FIXED=2 selects the K == 256 instance with both groups unrolled.

    M_SPLIT / TAIL: rows [0, M_SPLIT) run on this configuration, filling whole
    waves of workgroups over the CUs, and rows [M_SPLIT, M) run on the TAIL
    entry ({"impl", "config"}) in a second launch.  That replaces a last, mostly
    empty wave of big tiles; with M <= M_SPLIT the whole GEMM runs here."""
    m1 = int(config.get("M_SPLIT", 0))
    if m1 and A.shape[0] > m1 and "TAIL" in config:
        import torch
        from .engine import run
        m, n = A.shape[0], weight_dims(B)[0]
        out = epilogue.get("out")
        C = torch.empty((m, n), device=A.device, dtype=torch.bfloat16) if out is None else out
        head = {k: v for k, v in config.items() if k not in ("M_SPLIT", "TAIL")}
        bias = epilogue.get("bias")
        launch(A[:m1], B, As[:m1], Bs, _ring_cached(_freeze(head), int(head.get("K_FIXED", 0))),
               bias=bias, out=C[:m1])
        run(config["TAIL"], (A[m1:], B, As[m1:], Bs), bias=bias, out=C[m1:])
        return C
    config = {k: v for k, v in config.items() if k not in ("M_SPLIT", "TAIL")}
    return launch(A, B, As, Bs, _ring_cached(_freeze(config), int(config.get("K_FIXED", 0))),
                  **epilogue)


def shortk(A, B, As, Bs, config, **epilogue):
    """K == 256 kernel: both scale groups unrolled, no K loop, no split-K.

    Accepts gfx950 keys (BLOCK_W/BLOCK_T) or the reference's shortk keys
    (BM/BN, kernels/kernel_shortk.py:46-54)."""
    K = A.shape[1]
    if K != 256:
        raise ValueError("shortk requires K=256")
    if "BLOCK_W" not in config:
        tw, tt = nearest_tile(int(config["BN"]), int(config["BM"]), k_fixed=2)
        config = {"BLOCK_W": tw, "BLOCK_T": tt, "GROUP_SIZE_M": int(config.get("GROUP", 1))}
    return launch(A, B, As, Bs, _tiled_cached(_freeze(config), 2), **epilogue)



# ---------------------------------------------------------------------------
# reference (H20) table entries on gfx950 kernels
# ---------------------------------------------------------------------------
def _compat(tw_req, tt_req, split, mode, group, scale_lds=False):
    tw, tt = nearest_tile(tw_req, tt_req)
    cfg = {"BLOCK_W": tw, "BLOCK_T": tt, "SPLIT": int(split), "SPLIT_MODE": mode,
           "GROUP_SIZE_M": int(group), "SCALE_LDS": bool(scale_lds)}
    return _tiled_cached(_freeze(cfg), 0)


def triton(A, B, As, Bs, config, **epilogue):
    """Reference c3 entry (kernels/baseline_triton.py:87-114): full-grid split-K."""
    c = _compat(config["BLOCK_SIZE_N"], config["BLOCK_SIZE_M"], config.get("SPLIT_K", 1), "full",
                config.get("GROUP_SIZE_M", 1))
    return launch(A, B, As, Bs, c, **epilogue)


def gluon(A, B, As, Bs, config, **epilogue):
    """Reference c11 entry (kernels/baseline_gluon.py:259-293): tail split-K."""
    c = _compat(config["BLOCK_W"], config["BLOCK_T"], config.get("SPLIT", 1), "tail",
                config.get("GROUP_SIZE_M", 1))
    return launch(A, B, As, Bs, c, **epilogue)


def v2(A, B, As, Bs, config, **epilogue):
    """Reference v2 entry (kernels/kernel_v2.py:339-376): same schedule as c11."""
    return gluon(A, B, As, Bs, config, **epilogue)


def scale_tma(A, B, As, Bs, config, **epilogue):
    """Reference scale-TMA entry (kernels/kernel_scale_tma.py:356-396).

    Stages As in LDS when As is row-major, and otherwise runs the v2 path,
    mirroring the reference's `As.stride(1) != 1` fallback (:367-369)."""
    c = _compat(config["BLOCK_W"], config["BLOCK_T"], config.get("SPLIT", 1), "tail",
                config.get("GROUP_SIZE_M", 1), scale_lds=As.stride(1) == 1)
    return launch(A, B, As, Bs, c, **epilogue)
