/*
 * fp8bg.h - C ABI of the gfx950 block-scaled FP8 GEMM library (libfp8bg.so).
 *
 * Computes, on one AMD Instinct MI355X (gfx950):
 *
 *     C[M,N] (bf16) = sum_g ( A[:, g] . B[:, g]^T ) * As[m, g] * Bs[n / 128, g]
 *
 * where g runs over the K/128 groups of 128 K elements, A[M,K] and B[N,K] are
 * OCP e4m3 ("float8_e4m3fn") row-major with row stride K, As[M,K/128] and
 * Bs[N/128,K/128] are fp32 with arbitrary element strides, and C is row-major
 * bf16 with row stride N (round-to-nearest-even from the fp32 accumulator).
 * B may instead be given in the shuffled layout (FP8BG_FLAG_B_SHUFFLED).
 *
 * The reference (qiuuuuu622/fp8_gemm_h20) has no C ABI: its kernels are
 * Python-level Triton/Gluon host wrappers with the signature
 *     fn(A, B, As, Bs, config: dict) -> C
 * registered in fp8_gemm_h20/engine.py:5-19.  Each entry point below names the
 * reference interface it replaces.  All pointers are device pointers except
 * the config/plan structs and output scalars; no torch types cross this ABI.
 * Every function is reentrant.  The library's only device memory is the
 * static split-K scratch of fp8bg_gemm_noalloc (FP8BG_SCRATCH_ELEMS fp32 per
 * GPU, part of the loaded code object, held until the process ends).
 */
#ifndef FP8BG_H
#define FP8BG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes (returned by every entry point; 0 = success) ---------- */
#define FP8BG_OK             0
#define FP8BG_ERR_SHAPE      1  /* M<1, N or K not a positive multiple of 128, ... */
#define FP8BG_ERR_CONFIG     2  /* tile/wave/split combination not built or invalid */
#define FP8BG_ERR_WORKSPACE  3  /* split-K workspace missing, misaligned or too small */
#define FP8BG_ERR_ALIGN      4  /* A, B or C not 16-byte aligned */
#define FP8BG_ERR_LAUNCH     5  /* hipLaunchKernel / hip runtime error */
#define FP8BG_ERR_DEVICE     6  /* device query failed */
#define FP8BG_ERR_NULL       7  /* required pointer argument is NULL */
#define FP8BG_ERR_SCRATCH    8  /* split-K workspace beyond FP8BG_SCRATCH_ELEMS (fp8bg_gemm_noalloc) */

/* ABI version returned by fp8bg_version(); bumped on any signature or struct
 * change. */
#define FP8BG_ABI_VERSION 12

/* ---- kernel kinds --------------------------------------------------------- */
/* LDS-tiled kernel: a block_w x block_t workgroup tile, 4 waves in a
 * waves_w x waves_t grid, each 128-K group staged in LDS (double-buffered).
 * Replaces the reference's tiled kernels (kernels/baseline_triton.py:28-81,
 * kernels/baseline_gluon.py:94-211, kernels/kernel_v2.py:94-291). */
#define FP8BG_KIND_TILED  0
/* Small-M kernel: no LDS staging; waves_k waves (2, 4, 8 or 16) split the K groups
 * of one block_w x block_t tile, `unroll` groups in flight per wave, partials
 * summed in fixed wave order.  The reference's SWAP_AB small-M role
 * (kernels/baseline_gluon.py:77-83). */
#define FP8BG_KIND_SKINNY 1
/* LDS-ring kernel: like FP8BG_KIND_TILED, but each 128-K group is copied
 * global -> LDS by direct-to-LDS loads into a `stages`-deep ring (no register
 * staging, one barrier per `unroll` groups); waves_w x waves_t waves (4, 8
 * or 12), times waves_k K slices that split the tile's 128-K groups and sum
 * their partial tiles in fixed slice order.  Requires M*K and N*K below
 * 2^32. */
#define FP8BG_KIND_RING   2

/* ---- split-K modes ------------------------------------------------------ */
/* No split: every tile runs the full K range (config split ignored). */
#define FP8BG_SPLIT_NONE 0
/* Tail split (reference kernels/baseline_gluon.py:274-287): the first
 * tiles - (tiles % num_cus) tiles run whole; only the last partial wave is
 * split over `split` workgroups.  Tiled and ring kernels. */
#define FP8BG_SPLIT_TAIL 1
/* Full split (reference kernels/baseline_triton.py:100-114): every tile is
 * split. */
#define FP8BG_SPLIT_FULL 2
/* In both split modes the fp32 partials go to the caller's workspace and a
 * second kernel on the same stream sums them in fixed split order and writes
 * bf16 (deterministic, replay-safe, no atomics or counters). */
/* Full split reduced inside the GEMM kernel: skinny kernels, and ring
 * kernels with block_t <= 64 and k_fixed 0.  Each split workgroup (skinny),
 * or each wave's part of a split tile (ring), writes its partial with
 * device-scope stores and counts it in its counter; the one that completes
 * the count sums the partials in split order (bitwise the FP8BG_SPLIT_FULL
 * result), writes C and resets the counter.  One launch instead of two (the
 * reference's self-resetting counters, kernels/baseline_gluon.py:194-209,
 * with the summation order fixed).  At most FP8BG_COUNTERS counters: split
 * tiles (skinny) or split tiles x waves_w x waves_t (ring), and partials
 * below 2^31 bytes; a launch beyond either limit takes the FP8BG_SPLIT_FULL
 * reduction instead (plan.launches = 2, the same C bit for bit). */
#define FP8BG_SPLIT_LAST 3
/* Stream-K (ring kernels with k_fixed 0, waves_k 1 and block_w * block_t
 * below 256 * 256; config split ignored): for launches with fewer tiles
 * than CUs.  The tiles x (K/128) units of work are dealt out in equal
 * contiguous runs, about one per CU (plan.stream_units each: at least half
 * a tile, less than a whole one, a multiple of `unroll`), so every CU
 * computes the same number of 128-K groups and a tile is cut between two or
 * three consecutive runs.  A run that crosses a tile boundary computes the
 * next tile's head, then the current tile's tail, with one LDS ring running
 * through both.  The run holding a tile's last group owns it: the other
 * runs store their fp32 partials (device-scope stores) and count
 * themselves in the tile's per-wave counters, and the run that finds, or
 * completes, the full count sums the parts in K order (fixed, so C is the
 * same bit for bit on every call), writes C and resets the counters.  One
 * launch; no run waits for another.  Where no tile would be cut (tiles >=
 * CUs), or the counters (tiles x waves_w x waves_t) exceed FP8BG_COUNTERS,
 * the launch runs whole tiles instead (plan.stream_units = 0), so the mode
 * is valid at any M.  The reference's tail split-K role
 * (kernels/baseline_gluon.py:194-209,274-287), with equal work per CU
 * instead of whole split tiles. */
#define FP8BG_SPLIT_STREAM 4

/* Split-K workspace layout (every split mode): FP8BG_COUNTERS uint32 tile
 * counters, then the fp32 partials.  The counters must be zero before a
 * workspace's first use; every call leaves them zero. */
#define FP8BG_COUNTERS 4096

/* ---- config flags --------------------------------------------------------- */
/* Stage the tile's activation scales As[tile rows, k range] in LDS once per
 * workgroup (reference kernels/kernel_scale_tma.py:160-165); any As strides.
 * Tiled kernel only. */
#define FP8BG_FLAG_SCALE_LDS 0x1
/* Remap workgroup ids so that consecutive tiles run on the same XCD (L2). */
#define FP8BG_FLAG_XCD_REMAP 0x2
/* LDS chunk swizzle of the tiled and ring kernels (chunk c of row r is stored
 * at slot c ^ swz(r)); default swz = (r & 7) ^ ((r >> 3) & 1) (tiled) and
 * (r & 7) ^ 5 ((r >> 3) & 1) (ring), free of bank conflicts for each
 * kernel's MFMA operand reads.  At most one of: */
#define FP8BG_FLAG_SWZ8      0x4   /* swz = r & 7 */
#define FP8BG_FLAG_SWZPAIR   0x8   /* swz = (r >> 1) & 7 */
/* B is in the shuffled layout that fp8bg_shuffle_b writes (skinny and ring
 * kernels; a tiled configuration with it is FP8BG_ERR_CONFIG).  Every kernel
 * gives each MFMA the same operand bytes from either layout, so C is bitwise
 * the same as with the row-major B it was made from. */
#define FP8BG_FLAG_B_SHUFFLED 0x10

/*
 * Kernel configuration: one gfx950 table entry (fp8_gemm_h20/configs/<profile>.json).
 * Replaces the reference's per-entry `config` dict (fp8_gemm_h20/config.py:80-91).
 */
typedef struct fp8bg_config {
    int32_t kind;       /* FP8BG_KIND_* */
    int32_t block_w;    /* weight rows (N) per workgroup tile */
    int32_t block_t;    /* tokens (M) per workgroup tile */
    int32_t waves_w;    /* tiled/ring: waves along N inside the tile */
    int32_t waves_t;    /* tiled/ring: waves along M inside the tile */
    int32_t waves_k;    /* skinny: waves splitting K inside a workgroup (2, 4, 8 or 16);
                           ring: K slices of waves_w x waves_t waves (1, 2 or 4;
                           0 means 1) */
    int32_t unroll;     /* skinny: 128-K groups in flight per wave;
                           ring: 128-K groups per barrier (1, 2 or 4; 0 means 1);
                           K/128/split must be a multiple of it */
    int32_t stages;     /* ring: LDS ring depth in 128-K groups */
    int32_t split;      /* cross-workgroup K split factor, in 128-K groups;
                           normalised to 1 when it does not divide K/128
                           (baseline_gluon.py:274-276) */
    int32_t split_mode; /* FP8BG_SPLIT_* (skinny: NONE, FULL or LAST; tiled:
                           NONE, TAIL or FULL; ring: NONE, TAIL, FULL, LAST
                           when block_t <= 64 and k_fixed is 0, STREAM when
                           k_fixed is 0, waves_k is 1 and block_w * block_t
                           < 256 * 256) */
    int32_t group_t;    /* tiled: token-tile swizzle group (GROUP_SIZE_M
                           semantics, baseline_triton.py:36-45); >= 1 */
    int32_t flags;      /* FP8BG_FLAG_* */
    int32_t k_fixed;    /* tiled/ring: 0 = runtime K loop; 2 = K==256 short-K
                           kernel with no K loop (reference
                           kernels/kernel_shortk.py:11-54) */
} fp8bg_config;

/*
 * Launch plan derived on the host from (M,N,K,config,num_cus).  Pure host
 * arithmetic: CPU-testable without a GPU.
 * Replaces the host-wrapper arithmetic of kernels/baseline_gluon.py:266-287
 * (split normalisation, tail = tiles % num_SMs, n_dp, grid, _bufs sizes).
 */
typedef struct fp8bg_plan {
    int32_t tiles_w;    /* ceil(N / block_w) */
    int32_t tiles_t;    /* ceil(M / block_t) */
    int32_t tiles;      /* tiles_w * tiles_t */
    int32_t split;      /* effective split (1 when not split) */
    int32_t n_dp;       /* tiles computed whole (no reduction) */
    int32_t n_split;    /* tiles split over `split` workgroups */
    int32_t grid;       /* workgroups of the GEMM kernel = n_dp + n_split * split */
    int32_t launches;   /* kernels enqueued: 1, or 2 with the split-K reduction */
    int64_t ws_elems;   /* workspace elements needed (0 if no split):
                           FP8BG_COUNTERS + the fp32 partials */
    int32_t lds_bytes;  /* LDS used per workgroup */
    int32_t threads;    /* threads per workgroup */
    int32_t kernel_id;  /* index of the compiled kernel instance */
    int32_t stream_units; /* FP8BG_SPLIT_STREAM: 128-K groups (tile x group
                           units) per workgroup; 0 when the launch runs whole
                           tiles.  ws_elems then counts FP8BG_COUNTERS plus
                           2 * grid * block_w * block_t fp32 partials. */
} fp8bg_plan;

/* Library ABI version: FP8BG_ABI_VERSION of the build. */
int fp8bg_version(void);

/* Number of compute units of `device` (replaces _num_sms,
 * kernels/baseline_gluon.py:218-226). */
int fp8bg_num_cus(int device, int32_t* num_cus);

/* Validate (M,N,K,config) and fill `plan`.  No device calls. */
int fp8bg_make_plan(int32_t M, int32_t N, int32_t K, const fp8bg_config* cfg,
                    int32_t num_cus, fp8bg_plan* plan);

/* 1 if this kind/tile/wave/k_fixed combination is compiled into the library. */
int fp8bg_config_supported(const fp8bg_config* cfg);

/*
 * The GEMM.  Enqueues the kernel (plus the split-K reduction when the plan
 * splits) on `stream` (a hipStream_t; NULL = default stream) and returns
 * without synchronising.  Replaces the L0 host wrappers
 *   block_fp8_gemm_triton_h20  (kernels/baseline_triton.py:87-114)
 *   block_fp8_gemm_gluon_h20   (kernels/baseline_gluon.py:259-293)
 *   block_fp8_gemm_v2          (kernels/kernel_v2.py:339-376)
 *   block_fp8_gemm_scale_tma   (kernels/kernel_scale_tma.py:356-396)
 *   shortk                     (kernels/kernel_shortk.py:46-54)
 * with the caller owning C (bf16 [M,N], row stride N) and the split-K
 * workspace `ws` (>= plan.ws_elems 4-byte elements, 16-byte aligned, laid out
 * as FP8BG_COUNTERS zero counters then fp32 partials; unused and may be NULL
 * when plan.n_split == 0).  Calls that share `ws` must be ordered (same
 * stream); a captured hipGraph keeps using the `ws` it was captured with, so
 * that buffer must outlive the graph.
 * Scale strides are in elements.  A, B and C must be 16-byte aligned.
 * `bias` (bf16 [N], 8-byte aligned, or NULL) is added in the epilogue exactly
 * as the reference adapter's separate `out + bias` does it
 * (sgl_patch/fp8mm_sglang_patch.py:55-56): C is rounded to bf16, then
 * bf16(C) + bias is evaluated in fp32 and rounded to bf16 again.
 */
int fp8bg_gemm(const void* A, const void* B,
               const float* As, int64_t as_stride_m, int64_t as_stride_k,
               const float* Bs, int64_t bs_stride_n, int64_t bs_stride_k,
               const void* bias, void* C, int32_t M, int32_t N, int32_t K,
               const fp8bg_config* cfg, int32_t num_cus,
               float* ws, int64_t ws_elems,
               void* stream);

/*
 * fp8bg_gemm without a workspace argument, for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Same kernels,
 * plan and results as fp8bg_gemm (bitwise), with the split-K partials in a
 * static per-GPU scratch array of FP8BG_SCRATCH_ELEMS fp32 (16 MiB; every
 * entry of the packaged gfx950 tables fits it, where it is routed).  Calls
 * nothing that allocates: no hipMalloc/hipFree, no library allocator.
 *   - A launch whose plan needs more than FP8BG_SCRATCH_ELEMS workspace
 *     elements returns FP8BG_ERR_SCRATCH before anything is enqueued.
 *   - Runs on the current device; a non-NULL `stream` must belong to it
 *     (else FP8BG_ERR_DEVICE).  The scratch address is looked up once per
 *     device.
 *   - Every call on one GPU shares that GPU's scratch, which keeps the last
 *     split call's partials.  Nothing in it needs clearing: each split call
 *     writes all the partials it reads, and the tile counters of
 *     FP8BG_SPLIT_LAST and FP8BG_SPLIT_STREAM start at zero (the array is
 *     zero when the library loads) and are left zero by every call.  Split
 *     calls that overlap on one GPU (different streams, or threads without
 *     ordering) race on it.
 *   - Safe to call during hipGraph capture, including a process's first
 *     call on a device (tested): the call makes no stream-ordered request
 *     besides its kernel launches, and the graph keeps the scratch address.
 */
#define FP8BG_SCRATCH_ELEMS (1 << 22)
int fp8bg_gemm_noalloc(const void* A, const void* B,
                       const float* As, int64_t as_stride_m, int64_t as_stride_k,
                       const float* Bs, int64_t bs_stride_n, int64_t bs_stride_k,
                       const void* bias, void* C, int32_t M, int32_t N, int32_t K,
                       const fp8bg_config* cfg, int32_t num_cus, void* stream);

/*
 * Per-token-group activation quantisation (stream-ordered, no sync):
 *   for every row m and 128-wide K group g of x (bf16 [M,K], row stride
 *   x_stride_m elements, a multiple of 8; 16-byte aligned):
 *     s[m,g] = max(max_k |x[m,k]|, eps) / 448            (fp32, IEEE division)
 *     q[m,k] = e4m3(x[m,k] / s[m,g])                      (round to nearest even)
 *   q is e4m3 [M,K] row-major (row stride K); s is fp32 [M,K/128] with element
 *   strides (s_stride_m, s_stride_k), so row-major (K/128, 1) and column-major
 *   (1, M) scales are both direct outputs.
 * Produces the operands that the reference's SGLang adapter obtains from
 * sglang_per_token_group_quant_fp8(x, 128, column_major_scales=False,
 * scale_tma_aligned=False) before calling matmul
 * (sgl_patch/fp8mm_sglang_patch.py:51-54); same formula as the reference's
 * test recipe (scripts/validate.py:26-29, clamp_min(eps) then / 448).
 */
int fp8bg_quant_act(const void* x, int64_t x_stride_m, void* q,
                    float* s, int64_t s_stride_m, int64_t s_stride_k,
                    int32_t M, int32_t K, float eps, void* stream);

/*
 * The dense block-FP8 linear for small M in one kernel: bf16 activations
 * X[M,K] (row stride x_stride_m elements, 16-byte rows) are quantised per
 * 1x128 group inside the skinny GEMM kernel and multiplied with B/Bs as
 * fp8bg_gemm does, adding the optional bias.  Replaces the adapter's pair
 * per_token_group_quant_fp8 + matmul (sgl_patch/fp8mm_sglang_patch.py:51-54)
 * for decode-size M.
 *   - cfg must be a compiled skinny configuration with block_t == 16
 *     (else FP8BG_ERR_CONFIG); any M >= 1 is accepted.
 *   - Scales: s = max(amax, eps) / 448 exactly as fp8bg_quant_act, codes
 *     e4m3(x * (1/s)) with round to nearest even.  The reciprocal differs
 *     from fp8bg_quant_act's x / s by at most one e4m3 step on rare values,
 *     so results agree with quantise-then-gemm to the GEMM tolerance, not
 *     bitwise.  eps must be >= 1e-30.
 *   - q_out/s_out (both or neither) receive the codes and scales it used
 *     (s strides in elements); q_out 16-byte aligned.
 *   - ws as for fp8bg_gemm when the configuration splits K.
 */
int fp8bg_gemm_bf16a(const void* X, int64_t x_stride_m, float eps,
                     const void* B, const float* Bs, int64_t bs_stride_n,
                     int64_t bs_stride_k, const void* bias, void* C,
                     int32_t M, int32_t N, int32_t K, const fp8bg_config* cfg,
                     int32_t num_cus, float* ws, int64_t ws_elems,
                     void* q_out, float* s_out, int64_t s_stride_m,
                     int64_t s_stride_k, void* stream);

/*
 * Weight layout for MFMA-friendly loads (no reference counterpart: the
 * reference's adapter keeps B row-major; its survey ranks a pre-shuffled
 * weight format as an optional later step).  Writes the row-major e4m3
 * B[N,K] (row stride b_stride_n bytes, a multiple of 16) into Bt (N*K
 * bytes) as N/16 x K/128 blocks of 2048 bytes, block (b, g) at byte
 * (b * K/128 + g) * 2048, and inside it
 *     Bt[block + 16 l + 1024 h + e] = B[16 b + (l % 16), 128 g + 64 h + 16 (l / 16) + e]
 * for l < 64, h < 2, e < 16: the bytes that lane l of a wave feeds one
 * 16x16x128 MFMA, in lane order, so the kernels load them coalesced and use
 * them without a cross-lane exchange.  Pass Bt with FP8BG_FLAG_B_SHUFFLED in
 * the configuration (Bs unchanged).  N a multiple of 16, K of 128; B, Bt
 * 16-byte aligned; Bt must not overlap B.  Stream-ordered, no sync.
 */
int fp8bg_shuffle_b(const void* B, int64_t b_stride_n, void* Bt, int32_t N, int32_t K, void* stream);

/*
 * Host copy of the kernels' fp32 -> e4m3 conversion (round to nearest even,
 * NaN/|x| >= 480 -> 0x7f|sign), for host-side checks of that arithmetic.
 * No reference counterpart (the reference relies on torch's cast).
 */
int fp8bg_e4m3_encode_host(const float* x, uint8_t* out, int64_t n);

/*
 * The same conversion on the device, done the way both activation
 * quantisers do it: the v_cvt_pk_fp8_f32 instruction (two values per lane)
 * over n floats in device memory; stream-ordered, no sync.  For tests that
 * pin that instruction against fp8bg_e4m3_encode_host.  No reference
 * counterpart.
 */
int fp8bg_e4m3_encode_device(const float* x, uint8_t* out, int64_t n, void* stream);

/*
 * Calibration kernels: what this chip sustains, measured next to the
 * published peaks (no reference counterpart; the measurement plan for this
 * path asks for an MFMA-only, a streaming-read and a streaming-write
 * calibration).
 *
 * fp8bg_calib_mfma: `workgroups` workgroups of 256 threads (4 waves); each
 * wave issues 16 FP8 16x16x128 MFMAs per iteration (65536 flops each), for
 * `iters` iterations (1 .. FP8BG_CALIB_MAX_ITERS).  codes: 32 x 64 int32
 * e4m3 operand words (word e of lane l at [e * 64 + l]); out: workgroups *
 * 256 floats.  With every code byte 0x38 (1.0) each out value is
 * 2048 * iters exactly.
 *
 * fp8bg_calib_mfma_promoted: the same MFMAs as the GEMM kernels issue them,
 * each product from a zero accumulator and promoted at once by four FMAs
 * with the scale scale[lane] (64 floats, 1.0 for the exact result) into 8
 * accumulators; same arguments and result as fp8bg_calib_mfma.  The ratio of
 * the two rates is what the block-scale promotion costs the matrix pipe.
 *
 * fp8bg_calib_read: reads `bytes` (a multiple of 16, src 16-byte aligned)
 * with `workgroups` workgroups of 256 threads and writes workgroups * 256
 * uint32 words whose XOR equals the XOR of all 32-bit words of src.
 *
 * fp8bg_calib_write: fills `bytes` (a multiple of 16, dst 16-byte aligned)
 * with the 32-bit `value`, `workgroups` workgroups of 256 threads issuing
 * 16-byte stores; nontemporal != 0 uses the non-temporal stores the GEMM
 * kernels write C with.
 *
 * fp8bg_calib_launch: an empty kernel of `workgroups` workgroups of 64
 * threads; back to back in a hipGraph, its time per launch is the launch
 * floor of every call.
 */
#define FP8BG_CALIB_MAX_ITERS 8192
int fp8bg_calib_mfma(const int32_t* codes, float* out, int32_t workgroups, int32_t iters,
                     void* stream);
int fp8bg_calib_mfma_promoted(const int32_t* codes, const float* scale, float* out, int32_t workgroups,
                              int32_t iters, void* stream);
int fp8bg_calib_read(const void* src, int64_t bytes, uint32_t* out, int32_t workgroups,
                     void* stream);
int fp8bg_calib_write(void* dst, int64_t bytes, uint32_t value, int32_t workgroups, int32_t nontemporal,
                      void* stream);
int fp8bg_calib_launch(int32_t workgroups, void* stream);

/* Static message for an error code. */
const char* fp8bg_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* FP8BG_H */
