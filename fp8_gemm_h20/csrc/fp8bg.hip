// Block-scaled FP8 GEMM for AMD Instinct MI355X (gfx950): kernels + C ABI.
//
//   C[M,N] (bf16) = sum_g (A[:, g] . B[:, g]^T) * As[m, g] * Bs[n / 128, g]
//
// Math contract: reference fp8_gemm_h20/kernels/baseline_triton.py:16-18 and
// scripts/validate.py:32-34 (fp32 accumulation, one 128-K scale group per
// step, bf16 output).
//
// Common building block (gfx950, wave64): v_mfma_f32_16x16x128_f8f6f4 (OCP
// e4m3 x e4m3 -> fp32).  One instruction covers a whole 128-K scale group of a
// 16x16 output block, so each group's product lands in a fresh fp32 register
// quad that is promoted immediately: acc = fma(p, As[m,g] * Bs[nb,g], acc).
// Weights sit on the MFMA row side and tokens on the column side (the
// reference's SWAP_AB orientation, used for every M): a lane's four outputs
// then share one token and one 128-row weight block, so the promotion factor
// is ONE fp32 scalar per lane per 16x16 block and group.
//
// Operand layout in a lane (both operands identical): row (lane & 15) of a
// 16-row block, bytes [32 * (lane >> 4), +32) of the 128-byte group (LDS-fed
// kernels), or bytes [16 * (lane >> 4), +16) and [64 + 16 * (lane >> 4), +16)
// (fp8bg_skinny, whose operands arrive by coalesced loads and ds_bpermute).
// Since A and B use the same byte -> K assignment, the MFMA reduction covers
// exactly the 128 products of the group whatever order the hardware sums them
// in.
//
// Kernels:
//  * fp8bg_tiled  - LDS-tiled workgroup tile (weights x tokens), 4 waves, a
//                   128-K group staged global -> LDS with 16-byte loads and
//                   double-buffered; optional cross-workgroup split-K (tail
//                   wave or full grid) whose fp32 partials are summed by
//                   fp8bg_split_reduce in fixed split order.
//  * fp8bg_skinny - small-M kernel: no LDS staging; every wave loads its
//                   operands straight from global memory into MFMA registers
//                   and the S waves of a workgroup split the K groups of one
//                   tile among themselves (deep memory-level parallelism for
//                   weight streaming); the S partial tiles are summed through
//                   LDS in fixed wave order.  The QA variant reads bf16
//                   activations and quantises them in registers (the fused
//                   decode linear, fp8bg_gemm_bf16a).
//  * fp8bg_ring   - large-tile kernel: direct global->LDS loads
//                   (global_load_lds_dwordx4) into an ST-stage LDS ring, one
//                   barrier per 128-K group, 4 or 8 waves, the next group's
//                   loads spread over the MFMA stream; C staged through LDS
//                   and written as whole lines; split-K as fp8bg_tiled, or
//                   reduced inside the kernel (fp8bg_ring_last), or
//                   stream-K (fp8bg_ring_sk).
//  * fp8bg_split_reduce - fixed-order sum of split-K partials -> bf16.
//  * fp8bg_quant_act_kernel - bf16 activations -> e4m3 + fp32 group scales.
// Every reduction order is fixed by the configuration, so results are bitwise
// reproducible run to run and under hipGraph replay.  The in-kernel
// reductions (FP8BG_SPLIT_LAST, FP8BG_SPLIT_STREAM) count finished partials
// with relaxed agent-scope atomics on per-tile counters, after the partials'
// device-scope (SC1) stores have completed, and read them with device-scope
// loads; whichever workgroup completes a count sums the partials and resets
// the counter.  No kernel uses fences beyond workgroup scope or spin waits,
// and no workgroup waits for another.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "fp8bg.h"

// Build partition: fp8_gemm_h20/build.py compiles this file once per part,
// in parallel, and links the objects into one library.  Part 1 holds the C
// ABI, the tiled kernel and the small kernels; parts 2-7 the ring and skinny
// launchers (and so their kernel instances), split by list half and B
// layout.  FP8BG_PART 0 (the default) is all of it in one translation unit.
#ifndef FP8BG_PART
#define FP8BG_PART 0
#endif
#define FP8BG_HOST_PART (FP8BG_PART <= 1)

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kGroupK = 128;          // K elements per scale group
constexpr int kRowBytes = kGroupK;    // one fp8 row of a group = 128 bytes
constexpr int kMaxLds = 160 * 1024;   // gfx950 LDS per workgroup
// Shuffled B (FP8BG_FLAG_B_SHUFFLED): one 16-row block of one 128-K group,
// stored in MFMA lane order; byte 16 l + 1024 h + e of block (b, g) is
// B[16 b + (l & 15), 128 g + 64 h + 16 (l >> 4) + e] (l < 64, h < 2, e < 16)
constexpr int kShufBlock = 16 * kGroupK;

// Bs blocks a ring tile of tw weight rows can span: its first row lies at a
// multiple of gcd(tw, 128) inside a 128-row block (96-row tiles span two).
constexpr int ring_bs_blocks(int tw) {
    int g = 128;
    while (tw % g) g /= 2;
    return (128 - g + tw + 127) / 128;
}
// Scale-area DMA instructions per wave and stage of the ring kernel: one
// 64-dword slice per wave carries the tile's As column (tt floats), its Bs
// blocks (ring_bs_blocks floats) and the bias row (tw bf16 = tw / 2 dwords).
constexpr int ring_scale_slices(int tw, int tt, int nwave) {
    return (tt + ring_bs_blocks(tw) + tw / 2 + 64 * nwave - 1) / (64 * nwave);
}
constexpr int kNumXcd = 8;            // MI355X: 8 XCDs, workgroups dealt round-robin
// Word 3 of a gfx9 buffer resource for raw byte-offset loads (no format
// conversion, no swizzle); word 2 holds the size in bytes, loads past it
// return zero.
constexpr int kBufferFlags = 0x00020000;
// Cache-policy operand of buffer loads and stores: SC1, device scope (the
// access is coherent across the XCDs' private L2 caches).
constexpr int kDeviceScope = 16;
// The same operand's NT bit: a non-temporal (streaming) access.
constexpr int kNonTemporal = 2;

struct KArgs {
    const uint8_t* A;      // [M, K] e4m3, row stride K
    const uint8_t* B;      // [N, K] e4m3, row stride K
    const float* As;       // [M, K/128]
    const float* Bs;       // [N/128, K/128]
    uint16_t* C;           // [M, N] bf16, row stride N
    const uint16_t* bias;  // [N] bf16 or nullptr
    float* ws;             // split-K partials [split tile][split][tt][tw]
                           // (FP8BG_SPLIT_LAST: [split tile][split][block][lane] f32x4)
    uint32_t* cnt;         // FP8BG_SPLIT_LAST / _STREAM tile counters (zero between calls)
    int split_last;        // split tiles reduced in the GEMM kernel (selects its instance)
    int kcount;            // 128-K groups per workgroup: K / 128 / split (stream-K:
                           // the units, tile x group, of each workgroup's run)
    uint2 div_split;       // fast_div reciprocals of split and tiles_t
    uint2 div_tiles_t;
    int64_t as_sm, as_sk, bs_sn, bs_sk;
    int M, N, K;
    int tw, tt;            // workgroup tile (weight rows, tokens)
    int tiles_w, tiles_t;
    int n_dp;              // tiles computed whole
    int split;             // workgroups per split tile
    int group_t;           // token-tile swizzle group
    int xcd_remap;
    int scale_lds;
    int swz;               // LDS swizzle mode (see swz())
    // bf16 activations quantised inside the skinny kernel (fp8bg_gemm_bf16a)
    const uint16_t* X;     // [M, K] bf16, row stride ldx elements
    int64_t ldx;
    float eps;
    float eps_s, eps_r;    // eps / 448 and 1 / (eps / 448), IEEE fp32 on the host
    uint8_t* q_out;        // optional [M, K] e4m3 copy of the quantised activations
    float* s_out;          // optional [M, K/128] scales, strides qs_sm, qs_sk
    int64_t qs_sm, qs_sk;
    int stream;            // stream-K launch (FP8BG_SPLIT_STREAM; selects its instance)
};

// Two fp32 -> packed bf16 with gfx950's v_cvt_pk_bf16_f32: round to nearest
// even, overflow to +-inf, subnormals kept (measured against an integer RNE
// over every exponent class, all ties and subnormals).  Any NaN becomes
// 0x7fc0 as in torch; it is made canonical first because the instruction
// keeps a NaN's sign and payload.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const f32x2 v = {__builtin_isnan(a) ? __builtin_nanf("") : a,
                     __builtin_isnan(b) ? __builtin_nanf("") : b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint2 pack_bf16x4(const f32x4& v) {
    uint2 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    return o;
}

// The same for values known not to be NaN: the instruction alone.
__device__ __forceinline__ uint2 pack_bf16x4_nonan(const f32x4& v) {
    const f32x2 lo = {v[0], v[1]}, hi = {v[2], v[3]};
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                      __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2)));
}

// True on every lane when some lane of the wave holds a NaN among the
// tile's accumulators: one unordered compare covers two values.
template <int NW, int NT>
__device__ __forceinline__ bool wave_has_nan(const f32x4 (&acc)[NW][NT]) {
    bool nan = false;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int t = 0; t < NT; ++t)
            nan = nan | __builtin_isunordered(acc[w][t][0], acc[w][t][1]) |
                  __builtin_isunordered(acc[w][t][2], acc[w][t][3]);
    return __builtin_amdgcn_ballot_w64(nan) != 0;
}

// bf16 output of four consecutive columns n .. n+3, with the optional bias
// added the way a separate bf16 `C + bias` does it: C is rounded to bf16
// first, then bf16(C) + bias is evaluated in fp32 and rounded again.
// (out_bf16x4v: the same with the four bias values b already in registers.)
__device__ __forceinline__ uint2 out_bf16x4v(const f32x4& v, bool has_bias, uint2 b) {
    if (!has_bias) return pack_bf16x4(v);
    const uint2 c = pack_bf16x4(v);
    const uint32_t cc[4] = {c.x << 16, c.x & 0xffff0000u, c.y << 16, c.y & 0xffff0000u};
    const uint32_t bb[4] = {b.x << 16, b.x & 0xffff0000u, b.y << 16, b.y & 0xffff0000u};
    f32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = __uint_as_float(cc[i]) + __uint_as_float(bb[i]);
    return pack_bf16x4(r);
}

__device__ __forceinline__ uint2 out_bf16x4(const f32x4& v, const uint16_t* bias, int n) {
    return bias ? out_bf16x4v(v, true, *(const uint2*)(bias + n)) : pack_bf16x4(v);
}

__device__ __forceinline__ f32x4 mfma16x16x128(const i32x8& w, const i32x8& t) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    // cbsz/blgp format 0 = OCP e4m3 for both operands; scale operands 0 =
    // unscaled instruction.
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, t, zero, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ void promote(f32x4& acc, const f32x4& p, float s) {
    acc[0] = __builtin_fmaf(p[0], s, acc[0]);
    acc[1] = __builtin_fmaf(p[1], s, acc[1]);
    acc[2] = __builtin_fmaf(p[2], s, acc[2]);
    acc[3] = __builtin_fmaf(p[3], s, acc[3]);
}

// The first promotion of an accumulator: fma(p, s, +0), bitwise what promote
// gives on a zeroed accumulator (including the sign of zero), without the
// register moves that zero it.
__device__ __forceinline__ void promote_first(f32x4& acc, const f32x4& p, float s) {
    acc[0] = __builtin_fmaf(p[0], s, 0.0f);
    acc[1] = __builtin_fmaf(p[1], s, 0.0f);
    acc[2] = __builtin_fmaf(p[2], s, 0.0f);
    acc[3] = __builtin_fmaf(p[3], s, 0.0f);
}

// 32 operand bytes of one lane: two 16-byte global loads.
__device__ __forceinline__ i32x8 load_op(const uint8_t* p) {
    const i32x4 lo = *(const i32x4*)p;
    const i32x4 hi = *(const i32x4*)(p + 16);
    return (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// n / d for 0 <= n < 2^31 as (mulhi(n, m) + n) >> l with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (the round-up reciprocal method), from
// the pair {m, l} made on the host by fast_div_of(d).
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint2 ml) {
    return (__umulhi(n, ml.x) + n) >> ml.y;
}

inline uint2 fast_div_of(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = (((1ull << 32) * ((1ull << l) - d)) / d) + 1;
    return make_uint2((uint32_t)m, l);
}

// Bijective remap of workgroup ids 0..n-1 so that ids dealt to the same XCD
// (id % 8) receive a contiguous run of logical tiles.
__device__ __forceinline__ int xcd_remap(int pid, int n) {
    const int per = n / kNumXcd, rem = n % kNumXcd;
    const int xcd = pid % kNumXcd, local = pid / kNumXcd;
    return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// LDS row swizzle: 16-byte chunk c of tile row r is stored at chunk slot
// c ^ swz(r).  Operand reads have lanes l .. l+15 read rows r0 .. r0+15 (r0 a
// multiple of 16) at one logical chunk; the slot pattern decides how those 16
// addresses spread over the LDS banks.
//   mode 0: swz = (r & 7) ^ ((r >> 3) & 1)  (16-row pattern: any 16 consecutive
//           rows read at one chunk hit distinct bank groups; measured free of
//           LDS bank conflicts on gfx950 by SQ_LDS_BANK_CONFLICT)
//   mode 1: swz = r & 7                    (8-row period)
//   mode 2: swz = (r >> 1) & 7              (pairs of rows share a slot)
__device__ __forceinline__ int swz(int r, int mode) {
    return mode == 1 ? (r & 7) : mode == 2 ? ((r >> 1) & 7) : ((r & 7) ^ ((r >> 3) & 1));
}

// The ring kernel's swizzle.  Its operand reads give lane l = r + 16 q the
// logical chunks q and q + 4 (the skinny kernel's K order), and a
// ds_read_b128 serves together the eight lanes that agree in l % 8: rows
// k and k + 8 at chunks q = 0 .. 3.  Their eight slots q ^ swz(k) and
// q ^ swz(k + 8) are distinct when swz(k) ^ swz(k + 8) has bit 2 set; with
// mode 0 of swz() (bit 0) every such read took a 2-way conflict (7x the
// SQ_LDS_BANK_CONFLICT cycles, 2.5% slower at M=16384 N=12288 K=2048).
//   mode 0: swz = (r & 7) ^ 5 ((r >> 3) & 1)   (also keeps any 16
//           consecutive rows at one chunk on distinct 16-byte bank groups)
//   modes 1, 2 as swz()
__device__ __forceinline__ int swz_ring(int r, int mode) {
    return mode == 1 ? (r & 7) : mode == 2 ? ((r >> 1) & 7) : ((r & 7) ^ (((r >> 3) & 1) * 5));
}

// Shuffled B in the ring's LDS: MFMA lane l's 16 bytes of a block half sit
// at slot l ^ ((l >> 3) & 7), so the eight lanes that a ds_read_b128 serves
// together (equal l % 8) read eight different bank groups; the DMA lane that
// writes slot i fetches the block's chunk of lane i ^ ((i >> 3) & 7) (the map
// is its own inverse), still 64 contiguous bytes per quad of lanes.
__device__ __forceinline__ int shuf_slot(int l) { return l ^ ((l >> 3) & 7); }

// Grouped tile order (GROUP_SIZE_M semantics, reference
// kernels/baseline_triton.py:36-45): runs of group_t token tiles sweep the
// weight tiles together so their weight rows are reused while cached.
__device__ __forceinline__ void tile_origin(int tile, const KArgs& a, int& w0, int& t0) {
    const int per_group = a.group_t * a.tiles_w;
    const int first_t = (tile / per_group) * a.group_t;
    const int gsize = min(a.tiles_t - first_t, a.group_t);
    const int local = tile % per_group;
    const int pt = first_t + local % gsize;
    const int pw = local / gsize;
    w0 = pw * a.tw;
    t0 = pt * a.tt;
}

// ===========================================================================
// LDS-tiled kernel
// ===========================================================================
template <int TW, int TT, int WW, int WT, int KF>
__global__ __launch_bounds__(kThreads) void fp8bg_tiled(KArgs a) {
    static_assert(WW * WT == kThreads / 64, "4 waves per workgroup");
    constexpr int WTW = TW / WW;               // weight rows per wave
    constexpr int WTT = TT / WT;               // tokens per wave
    constexpr int NW = WTW / 16;               // 16-row weight blocks per wave
    constexpr int NT = WTT / 16;               // 16-token blocks per wave
    static_assert(WTW % 16 == 0 && WTT % 16 == 0 && NW >= 1 && NT >= 1, "wave tile");
    static_assert(TW % 8 == 0 && TT % 8 == 0, "tile rows");
    constexpr int ROWS = TW + TT;              // LDS rows per group buffer
    constexpr int CHUNKS = ROWS * 8;           // 16-byte chunks per group
    constexpr int NLD = (CHUNKS + kThreads - 1) / kThreads;
    constexpr int WCH = TW * 8;                // chunks belonging to weights
    constexpr int BUF = ROWS * kRowBytes;

    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * BUF];
    extern __shared__ float s_as[];            // [TT][kcount] when scale_lds

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wv_w = wave % WW, wv_t = wave / WW;

    // ---- tile decode ----
    const int KG = KF ? KF : (a.K / kGroupK);
    int pid = blockIdx.x;
    int tile, sidx = 0, kcount, k_lo;
    if (pid < a.n_dp) {
        if (a.xcd_remap) pid = xcd_remap(pid, a.n_dp);
        tile = pid;
        k_lo = 0;
        kcount = KG;
    } else {
        const int q = pid - a.n_dp;
        tile = a.n_dp + q / a.split;
        sidx = q % a.split;
        kcount = KG / a.split;
        k_lo = sidx * kcount;
    }
    int w0, t0;
    tile_origin(tile, a, w0, t0);

    // ---- per-thread global->LDS chunk assignment (fixed across groups) ----
    // chunk c: row c/8 of the stacked [weights; tokens] tile, 16-byte column
    // c%8, stored at slot (c%8) ^ swz(row) so that the operand reads (16
    // consecutive lanes = 16 consecutive rows, same chunk) spread over the
    // LDS banks.
    const uint8_t* gptr[NLD];
    int loff[NLD];
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
        const int c = tid + kThreads * j;
        const int row = min(c >> 3, ROWS - 1);
        const int col = c & 7;
        if (kThreads * j < WCH) {
            const int n = min(w0 + row, a.N - 1);
            gptr[j] = a.B + (size_t)n * a.K + col * 16;
        } else {
            const int m = min(t0 + row - TW, a.M - 1);
            gptr[j] = a.A + (size_t)m * a.K + col * 16;
        }
        loff[j] = row * kRowBytes + ((col ^ swz(row, a.swz)) << 4);
    }
    auto gload = [&](int g, i32x4 (&r)[NLD]) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            if (CHUNKS % kThreads == 0 || tid + kThreads * j < CHUNKS)
                r[j] = *(const i32x4*)(gptr[j] + (size_t)g * kGroupK);
        }
    };
    auto sstore = [&](int buf, const i32x4 (&r)[NLD]) {
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            if (CHUNKS % kThreads == 0 || tid + kThreads * j < CHUNKS)
                *(i32x4*)(lds + buf * BUF + loff[j]) = r[j];
        }
    };

    // ---- scales ----
    int tok[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) tok[t] = min(t0 + wv_t * WTT + t * 16 + (lane & 15), a.M - 1);
    int nb[NW];
    const int nblocks = a.N / 128;
#pragma unroll
    for (int w = 0; w < NW; ++w) nb[w] = min((w0 + wv_w * WTW + w * 16) >> 7, nblocks - 1);

    if (a.scale_lds) {
        // Stage As[tile tokens, k_lo .. k_lo+kcount) once; walk memory along
        // whichever As stride is unit so the loads coalesce
        // (reference kernels/kernel_scale_tma.py:160-165).
        const int n_el = TT * kcount;
        if (a.as_sk == 1) {
            for (int e = tid; e < n_el; e += kThreads) {
                const int r = e / kcount, g = e % kcount;
                const int m = min(t0 + r, a.M - 1);
                s_as[r * kcount + g] = a.As[(int64_t)m * a.as_sm + (int64_t)(k_lo + g) * a.as_sk];
            }
        } else {
            for (int e = tid; e < n_el; e += kThreads) {
                const int g = e / TT, r = e % TT;
                const int m = min(t0 + r, a.M - 1);
                s_as[r * kcount + g] = a.As[(int64_t)m * a.as_sm + (int64_t)(k_lo + g) * a.as_sk];
            }
        }
    }

    float sa_n[NT], sb_n[NW];
    auto sload = [&](int g, int i) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (a.scale_lds)
                sa_n[t] = s_as[(tok[t] - t0) * kcount + i];
            else
                sa_n[t] = a.As[(int64_t)tok[t] * a.as_sm + (int64_t)g * a.as_sk];
        }
#pragma unroll
        for (int w = 0; w < NW; ++w) sb_n[w] = a.Bs[(int64_t)nb[w] * a.bs_sn + (int64_t)g * a.bs_sk];
    };

    f32x4 acc[NW][NT];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[w][t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // operand rows are 16-aligned bases + (lane & 15), so swz(row) = swz(lane & 15)
    const int c0 = ((lane >> 4) * 2) ^ swz(lane & 15, a.swz);
    auto opread = [&](int buf, int row) -> i32x8 {
        const unsigned char* base = lds + buf * BUF + row * kRowBytes;
        const i32x4 lo = *(const i32x4*)(base + (c0 << 4));
        const i32x4 hi = *(const i32x4*)(base + ((c0 ^ 1) << 4));
        return (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    i32x4 stage[NLD];
    if (a.scale_lds) __syncthreads();
    gload(k_lo, stage);
    sload(k_lo, 0);
    sstore(0, stage);
    __syncthreads();

#pragma unroll (KF ? KF : 1)
    for (int i = 0; i < kcount; ++i) {
        const int g = k_lo + i;
        const int buf = i & 1;
        float sa[NT], sb[NW];
#pragma unroll
        for (int t = 0; t < NT; ++t) sa[t] = sa_n[t];
#pragma unroll
        for (int w = 0; w < NW; ++w) sb[w] = sb_n[w];
        const bool more = i + 1 < kcount;
        if (more) {
            gload(g + 1, stage);
            sload(g + 1, i + 1);
        }
        i32x8 top[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) top[t] = opread(buf, TW + wv_t * WTT + t * 16 + (lane & 15));
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const i32x8 wop = opread(buf, wv_w * WTW + w * 16 + (lane & 15));
#pragma unroll
            for (int t = 0; t < NT; ++t) promote(acc[w][t], mfma16x16x128(wop, top[t]), sa[t] * sb[w]);
        }
        if (more) sstore(buf ^ 1, stage);
        __syncthreads();
    }

    // ---- epilogue ----
    // Output block (w, t): this lane holds token (lane & 15) and the four
    // consecutive weight rows 4*(lane >> 4) .. +3.
    if (blockIdx.x < a.n_dp) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int m = t0 + wv_t * WTT + t * 16 + (lane & 15);
            if (m >= a.M) continue;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const int n = w0 + wv_w * WTW + w * 16 + (lane >> 4) * 4;
                if (n >= a.N) continue;
                *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(acc[w][t], a.bias, n);
            }
        }
        return;
    }
    // Split tile: publish this K range's fp32 partial, row-major [tt][tw]
    // inside the tile's slab; fp8bg_split_reduce sums the slabs afterwards.
    float* mine = a.ws + ((size_t)(tile - a.n_dp) * a.split + sidx) * (size_t)(TW * TT);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tl = wv_t * WTT + t * 16 + (lane & 15);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int wl = wv_w * WTW + w * 16 + (lane >> 4) * 4;
            *(f32x4*)(mine + tl * TW + wl) = acc[w][t];
        }
    }
}

// ===========================================================================
// LDS-ring kernel: direct global->LDS loads, ST-stage ring, one barrier per group
// ===========================================================================
// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= N only:
// vmcnt in bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] at maximum.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Same, and also wait for every LDS read of this wave (lgkmcnt = 0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lds() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

#define FP8BG_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Compile-time wave role of the ring kernel's main loop (see fp8bg_ring).
template <int R>
struct WaveRole {
    static constexpr int value = R;
};
// whether a ring step issues the loads of the groups ST - KU ahead (also
// used as a compile-time yes/no flag elsewhere)
template <bool B>
struct Loads {
    static constexpr bool value = B;
};
// whether a ring step holds each K slice's first group
template <bool B>
struct First {
    static constexpr bool value = B;
};

// Workgroup tile TW weight rows x TT tokens, WW x WT waves.  Each 128-K group
// of the stacked [weights; tokens] tile (TW + TT rows of 128 bytes) is copied
// global -> LDS by global_load_lds_dwordx4: one instruction moves 64 lanes x
// 16 bytes = 8 rows into a contiguous 1 KB block, lane l writing chunk slot
// l % 8 of row l / 8.  The lane fetches global chunk (l % 8) ^ swz_ring(row),
// so chunk c of a row sits at slot c ^ swz_ring(row): the XOR swizzle that
// spreads the MFMA operand reads (16 consecutive lanes = 16 consecutive rows,
// four chunks across the wave) over the LDS banks.  The group's scales travel the same way: one
// global_load_lds_dword per wave fills a 64-float slice of the stage's scale
// area with the tile's As column (slots 0 .. TT-1) and its Bs values (slots
// TT .. TT + TW/128 - 1).  ST stages form a ring: the loads of group
// i + ST - 1 are issued while group i is computed, with no register staging
// and no VGPR-destination memory loads in the loop, and each group needs one
// barrier.  With KU > 1 a barrier covers KU consecutive groups: the loads of
// groups i + ST - KU .. i + ST - 1 refill the stages of the KU groups computed
// before the barrier, and the second group's LDS reads overlap the first
// group's MFMAs (small tiles spend most of a one-group step waiting for the
// barrier and the first operand reads).  With WK > 1 the workgroup holds WK
// slices of WW x WT waves; slice k computes (and loads) the groups i with
// i % WK == k, in the stages s with s % WK == k, so each slice runs its own
// ring of ST / WK stages and KU / WK groups per barrier.  The slices' partial
// tiles are summed through LDS in fixed slice order at the end: for tiles
// with few workgroups and long K (narrow N at small M), WK times the loads
// and MFMAs in flight without a second launch.
// Whether a ring instance also has an fp8bg_ring_dp kernel: the instances
// whose last group can write C itself (see group_last below).
constexpr bool ring_has_dp(int TW, int TT, int KF, int KU, int WK) {
    return KU == 1 && WK == 1 && KF == 0 && TW * TT >= 128 * 128;
}

// Whether a ring instance also has an fp8bg_ring_last kernel (split-K
// reduced inside the GEMM kernel, FP8BG_SPLIT_LAST): the token tiles of
// decode and small-M sizes, where few tiles leave most CUs idle.
constexpr bool ring_has_last(int TT, int KF) { return TT <= 64 && KF == 0; }

// Whether a ring instance also has an fp8bg_ring_sk kernel (stream-K,
// FP8BG_SPLIT_STREAM): one K slice, a runtime K loop, and accumulators
// ((TW / WW) x (TT / WT) / 64 VGPRs per wave) that leave room for the two
// more sets of them the fixup loads: at most 64 with two waves per SIMD or
// fewer, 32 with three (larger ones spill).
constexpr bool ring_has_sk(int TW, int TT, int WW, int WT, int KF, int WK) {
    return KF == 0 && WK == 1 && (TW / WW) * (TT / WT) / 64 <= (WW * WT > 8 ? 32 : 64);
}

// The ring kernel's body.  DPO: every workgroup of the launch is a whole
// (data-parallel) tile, none computes a K split.  BSH: B in the shuffled
// layout (kShufBlock); its 16-row blocks reach LDS in MFMA lane order, so
// each wave reads a weight operand as two lane-linear 16-byte loads.
// SK: stream-K (FP8BG_SPLIT_STREAM).  The launch's tiles x K-groups units
// are dealt out in equal contiguous runs of a.kcount units, one run per
// workgroup (per <= K/128: a run touches at most two tiles).  The ring runs
// straight through the run: the loads of the second tile's first groups are
// issued while the first tile's last groups compute, so the pipeline never
// drains between them.  A run that starts inside tile a and ends inside
// tile a + 1 computes tile a + 1's head first and tile a's tail last; the
// workgroup holding a tile's tail owns it and, finishing last, normally
// finds the other parts of the tile stored already.
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK, bool DPO, bool LAST,
          bool BSH = false, bool SK = false>
__device__ __forceinline__ void ring_body(const KArgs& a) {
    constexpr int NWAVE = WW * WT;                // waves of one K slice
    constexpr int WTW = TW / WW;
    constexpr int WTT = TT / WT;
    constexpr int NW = WTW / 16;
    constexpr int NT = WTT / 16;
    constexpr int ROWS = TW + TT;
    constexpr int NBLK = ROWS / 8;                // 1 KB operand blocks (8 rows) per group
    constexpr int NJ = (NBLK + NWAVE - 1) / NWAVE; // blocks per wave per group
    constexpr int NSC = ring_scale_slices(TW, TT, NWAVE);
    constexpr int NDMA = NJ + NSC;                // + the scale slices
    constexpr int OPS = ROWS * kRowBytes;         // operand bytes per stage
    constexpr int SCALES = NSC * NWAVE * 64;      // scale slots per stage
    constexpr int STAGE = OPS + SCALES * 4;
    static_assert(WTW % 16 == 0 && WTT % 16 == 0 && NW >= 1 && NT >= 1, "wave tile");
    static_assert(ROWS % 8 == 0 && NJ >= 1 && NJ * NWAVE - NBLK < NBLK, "DMA blocks per wave");
    constexpr int NBS = ring_bs_blocks(TW);       // Bs blocks the tile spans
    static_assert(TT + NBS + TW / 2 <= SCALES, "scale slots");
    // epilogue: 16 output rows of a wave at a time, staged in LDS
    constexpr int ROWB = WTW * 2;                 // bf16 bytes of one wave row
    constexpr int CPR = ROWB / 16;                // 16-byte chunks per wave row
    static_assert(NWAVE * WTT * ROWB <= ST * STAGE, "epilogue regions inside the ring");
    static_assert(WTW <= 128 && 128 % WTW == 0, "wave weight rows inside one Bs block");
    static_assert(KU >= 1 && ST >= 2 * KU && NDMA * (ST - 2 * KU) / WK < 64, "ring depth");
    static_assert(KF == 0 || KF % KU == 0, "groups per barrier");
    static_assert(WK >= 1 && ST % WK == 0 && KU % WK == 0 && (WK == 1 || KF == 0), "K slices");
    static_assert((WK - 1) * TW * TT * 4 <= ST * STAGE, "slice reduction inside the ring");
    static_assert(ST * STAGE <= kMaxLds, "LDS");

    __shared__ __attribute__((aligned(1024))) unsigned char lds[ST * STAGE];

    const int lane = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = wave_all / NWAVE;              // K slice
    const int wave = wave_all % NWAVE;            // wave inside the slice
    const int wv_w = wave % WW, wv_t = wave / WW;

    // ---- tile decode ----
    const int KG = KF ? KF : (a.K / kGroupK);
    int pid = blockIdx.x;
    int tile, sidx = 0, kcount, k_lo;
    // stream-K: the workgroup's place in the unit order (sk_w), the units of
    // the tile it computes first (n1; kcount when the run stays in one
    // tile), and the tile it computes second with that tile's first group
    int sk_w = 0, n1 = 0, tile2 = 0, k_lo2 = 0;
    if constexpr (SK) {
        static_assert(ring_has_sk(TW, TT, WW, WT, KF, WK), "stream-K instance");
        sk_w = a.xcd_remap ? xcd_remap(pid, (int)gridDim.x) : pid;
        const int u0 = sk_w * a.kcount;
        const int u1 = min(u0 + a.kcount, a.tiles_w * a.tiles_t * KG);
        const int ta = u0 / KG, tb = (u1 - 1) / KG;
        kcount = u1 - u0;
        if (ta == tb) {
            tile = ta;
            k_lo = u0 - ta * KG;
            n1 = kcount;
        } else {
            // tile tb's head (groups 0 .. n1 - 1) first, then tile ta's tail
            tile = tb;
            k_lo = 0;
            n1 = u1 - tb * KG;
            tile2 = ta;
            k_lo2 = u0 - ta * KG;
        }
    } else if (pid < a.n_dp) {
        if (a.xcd_remap) pid = xcd_remap(pid, a.n_dp);
        tile = pid;
        k_lo = 0;
        kcount = KG;
    } else {
        const int q = pid - a.n_dp;
        tile = a.n_dp + q / a.split;
        sidx = q % a.split;
        kcount = KG / a.split;
        k_lo = sidx * kcount;
    }
    int w0, t0;
    tile_origin(tile, a, w0, t0);
    int w0b = w0, t0b = t0;                       // stream-K: the second tile's origin
    if (SK && n1 < kcount) tile_origin(tile2, a, w0b, t0b);
    // weight origin of the tile being computed (its Bs block), changed
    // between a stream-K run's two tiles
    int w0c = w0;

    // ---- DMA sources: operand block b holds rows 8b .. 8b+7; wave w moves
    // blocks w * NJ .. w * NJ + NJ - 1.  When the NBLK blocks do not divide
    // evenly among the waves, the indices past NBLK wrap to the first blocks:
    // those are loaded twice, by two waves, into the same LDS bytes with the
    // same data, so every wave issues NJ loads per group and the vmcnt
    // bookkeeping stays uniform. ----
    // The operand loads go through buffer resources of A and B (byte
    // offsets below 2^32: the host refuses M*K or N*K beyond that): the
    // lane's fixed offset is the VGPR offset and the group's advance the
    // SGPR offset, so a group issues no per-lane address arithmetic.
    const __amdgpu_buffer_rsrc_t rsA =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.A, (short)0, (int)((uint32_t)a.M * (uint32_t)a.K), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsB =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.B, (short)0, (int)((uint32_t)a.N * (uint32_t)a.K), kBufferFlags);
    // (shuffled B: operand block b of the weights is half b % 2 of the
    // tile's 16-row block b / 2, copied as it lies, 16 bytes per lane)
    bool from_b[NJ];
    uint32_t soff[NJ];
    uint32_t soff2[SK ? NJ : 1];                  // stream-K: the second tile's
    int dblk[NJ];
    auto op_off = [&](int j, int w0_, int t0_) -> uint32_t {
        const int b = dblk[j];
        const int row = 8 * b + (lane >> 3);
        const int chunk = (lane & 7) ^ swz_ring(row, a.swz);
        if (from_b[j] && BSH)
            return (uint32_t)min((w0_ >> 4) + (b >> 1), (a.N >> 4) - 1) * (uint32_t)(a.K / kGroupK) *
                       (uint32_t)kShufBlock +
                   (b & 1) * (kShufBlock / 2) + shuf_slot(lane) * 16;
        if (from_b[j]) return (uint32_t)min(w0_ + row, a.N - 1) * (uint32_t)a.K + chunk * 16;
        return (uint32_t)min(t0_ + row - TW, a.M - 1) * (uint32_t)a.K + chunk * 16;
    };
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int b_raw = wave * NJ + j;
        const int b = b_raw < NBLK ? b_raw : b_raw - NBLK;
        dblk[j] = b;
        from_b[j] = 8 * b < TW;                   // wave-uniform
        soff[j] = op_off(j, w0, t0);
        if constexpr (SK) soff2[j] = op_off(j, w0b, t0b);
    }
    // scale slot q = 64 * (h * NWAVE + wave) + lane of slice h: As of token
    // t0 + q, then Bs of weight block w0 / 128 + (q - TT) for the NBS blocks
    // the tile spans, then bias dword (q - TT - NBS) = columns w0 + 2 (q - TT
    // - NBS) and the next one (the same every group); spare slots, and the
    // bias slots without a bias, reload As[0, g] (never read).  Stream-K
    // adds the bias where it writes C, from global memory.
    const float* sc_base[NSC];
    const float* sc_base2[SK ? NSC : 1];
    int64_t sc_step[NSC];
    auto sc_src = [&](int h, int w0_, int t0_) -> const float* {
        const int q = 64 * (h * NWAVE + wave) + lane;
        if (q < TT) {
            // slot r * NT + t of a wave's WTT-token range holds token
            // t * 16 + r: a lane's NT scales (token r of each 16-token
            // block) are contiguous, one or two 16-byte reads per group
            const int ql = q % WTT;
            const int tok = q - ql + (ql % NT) * 16 + ql / NT;
            return a.As + (int64_t)min(t0_ + tok, a.M - 1) * a.as_sm;
        }
        if (q < TT + NBS) return a.Bs + (int64_t)min(w0_ / 128 + (q - TT), a.N / 128 - 1) * a.bs_sn;
        if (!SK && q < TT + NBS + TW / 2 && a.bias)
            return (const float*)(a.bias + min(w0_ + 2 * (q - TT - NBS), a.N - 2));
        return a.As;
    };
#pragma unroll
    for (int h = 0; h < NSC; ++h) {
        const int q = 64 * (h * NWAVE + wave) + lane;
        sc_base[h] = sc_src(h, w0, t0);
        if constexpr (SK) sc_base2[h] = sc_src(h, w0b, t0b);
        sc_step[h] = q < TT ? a.as_sk : q < TT + NBS ? a.bs_sk : (!SK && q < TT + NBS + TW / 2 && a.bias) ? 0 : a.as_sk;
    }
    // g: the 128-K group of the tile (stream-K: the unit of the run, in the
    // order the run computes them, the second tile's from n1 on)
    auto dma_block = [&](int j, int g, int stage) {
        uint32_t off = soff[j];
        if constexpr (SK) {
            const bool second = g >= n1;          // wave-uniform
            off = second ? soff2[j] : soff[j];
            g = second ? k_lo2 + (g - n1) : k_lo + g;
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(from_b[j] ? rsB : rsA,
                                                 FP8BG_LDS_PTR(lds + stage * STAGE + dblk[j] * 1024), 16,
                                                 off,
                                                 (uint32_t)g * (BSH && from_b[j] ? kShufBlock : kGroupK), 0,
                                                 0);
    };
    auto dma_scales = [&](int g, int stage) {
        bool second = false;
        if constexpr (SK) {
            second = g >= n1;
            g = second ? k_lo2 + (g - n1) : k_lo + g;
        }
#pragma unroll
        for (int h = 0; h < NSC; ++h)
            __builtin_amdgcn_global_load_lds(
                (const void*)((SK && second ? sc_base2[h] : sc_base[h]) + (int64_t)g * sc_step[h]),
                FP8BG_LDS_PTR(lds + stage * STAGE + OPS + (h * NWAVE + wave) * 256), 4, 0, 0);
    };
    auto dma = [&](int g, int stage) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) dma_block(j, g, stage);
        dma_scales(g, stage);
    };

    // The first barrier step initialises the accumulators (promote_first):
    // every path through the loops below starts with a First<true> step, so
    // nothing zeroes them (a zeroing branch for one-step launches would be
    // merged into every path by the compiler).
    f32x4 acc[NW][NT];

    // Operand reads: lane l = r + 16 q reads row r0 + r of a 16-row block at
    // chunks q and q + 4 (K bytes [16 q, +16) and [64 + 16 q, +16): the order
    // of the skinny kernel and of the shuffled layout, so that every kernel
    // feeds each MFMA the same bytes from either B layout).  The lane's two
    // byte offsets inside a stage are fixed; the block's row r0 (wave-
    // uniform) becomes the read's immediate offset, so a group adds only the
    // stage base to the two lane offsets.  The weights of a shuffled B sit in
    // lane order, permuted by shuf_slot: bytes 16 shuf_slot(l) and 1024 + the
    // same of their block.
    const int sw_l = swz_ring(lane & 15, a.swz);
    const uint32_t lane_lo = (lane & 15) * kRowBytes + (((lane >> 4) ^ sw_l) << 4);
    const uint32_t lane_hi = (lane & 15) * kRowBytes + ((((lane >> 4) + 4) ^ sw_l) << 4);
    auto opread = [&](const unsigned char* st, int r0) -> i32x8 {
        const i32x4 lo = *(const i32x4*)(st + lane_lo + r0 * kRowBytes);
        const i32x4 hi = *(const i32x4*)(st + lane_hi + r0 * kRowBytes);
        return (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    const uint32_t wlane_lo = BSH ? 16 * shuf_slot(lane) : lane_lo;
    const uint32_t wlane_hi = BSH ? kShufBlock / 2 + 16 * shuf_slot(lane) : lane_hi;
    auto wread = [&](const unsigned char* st, int r0) -> i32x8 {
        const i32x4 lo = *(const i32x4*)(st + wlane_lo + r0 * kRowBytes);
        const i32x4 hi = *(const i32x4*)(st + wlane_hi + r0 * kRowBytes);
        return (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // Every step but the last issues its loads unconditionally so the vmcnt
    // bookkeeping is the same in every iteration: group indices past the
    // range are clamped to the last group (an L2 hit), and such a load lands
    // in a stage that no later step reads (the stage of group g is read only
    // by group g, and a clamped index g is past the last group).  The last
    // step's loads would all be clamped; it is peeled off without them (no
    // wait counts the loads issued after the ones it waits for).
    const int g_last = k_lo + kcount - 1;
    // the group (stream-K: the unit of the run) that step slot v loads
    auto load_idx = [&](int v) { return SK ? min(v, kcount - 1) : min(k_lo + v, g_last); };
    for (int s = ks; s < ST - KU; s += WK) dma(load_idx(s), s);

    // One 128-K group: stage i % ST is computed while the loads of group
    // g_next are spread over its token blocks (operand block j before token
    // block j * NT / (2 NJ), the scale slices before token block NT / 2).
    // Issued together right after the barrier, the waves' loads queue at the
    // address unit and hold back the first MFMAs; spread out, they overlap
    // the MFMA stream.
    // Wave priorities on the 256x256 tile: the two waves sharing a SIMD
    // (token halves 0 and 1) would otherwise share the matrix pipe oldest
    // first, the older one finishing its group long before the younger one
    // and then idling at the barrier while the pipe runs one wave.  The
    // younger wave takes priority for the first token blocks of each group
    // and the older one for the rest (about 2% faster; no effect on smaller
    // tiles, so they keep one role).
    constexpr bool kPrio = WT == 2 && TW * TT >= 256 * 256;
    auto group = [&](int i, int g_next, int s_next, auto role, auto load, auto first) {
        constexpr int R = decltype(role)::value;
        constexpr bool LD = decltype(load)::value;
        constexpr bool FIRST = decltype(first)::value;
        const unsigned char* st = lds + (i % ST) * STAGE;
        const float* sc = (const float*)(st + OPS);
        // The group's first operands are read in the order the first token
        // block's MFMAs consume them (token block 0, then weight blocks 0..NW-1),
        // fenced so the LDS serves them in that order: the first MFMA waits
        // for four reads, not for all of them (about 1% fewer cycles on the
        // largest tiles, up to 4% on the mid-size ones).
        i32x8 top = opread(st, TW + wv_t * WTT);
        __builtin_amdgcn_sched_barrier(0);
        i32x8 wop[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            wop[w] = wread(st, wv_w * WTW + w * 16);
            __builtin_amdgcn_sched_barrier(0);
        }
        const float sb = sc[TT + (w0c % 128 + wv_w * WTW) / 128];
        float sa[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) sa[t] = sc[wv_t * WTT + (lane & 15) * NT + t];
        __builtin_amdgcn_sched_barrier(0);
        // Software pipeline over token blocks: block t's products go into
        // their own registers, and each MFMA is followed by the four
        // promotion FMAs of the previous block's product for the same weight
        // block, which run on the VALU while the MFMA occupies the matrix
        // pipe; block t + 1's operand is read from LDS one block ahead (for
        // block 0, right after its first MFMA).  The scheduling fences keep
        // this order (the default schedule promotes each product right after
        // its own MFMA and stalls on it).
        f32x4 prev[NW];
        float s_prev = 0.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            i32x8 top_next = top;
            if (t > 0 && t + 1 < NT) top_next = opread(st, TW + wv_t * WTT + (t + 1) * 16);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                if (LD && (j * NT) / (2 * NJ) == t) dma_block(j, g_next, s_next);
            if (LD && t == NT / 2) dma_scales(g_next, s_next);
            if (kPrio && t == 0) {
                if (R) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            if (kPrio && t == NT / 2 + 1) {
                if (R) __builtin_amdgcn_s_setprio(0);
                else __builtin_amdgcn_s_setprio(1);
            }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 cur[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                cur[w] = mfma16x16x128(wop[w], top);
                if (t > 0) {
                    if (FIRST) promote_first(acc[w][t - 1], prev[w], s_prev);
                    else promote(acc[w][t - 1], prev[w], s_prev);
                }
                if (t == 0 && w == 0 && NT > 1) {
                    __builtin_amdgcn_sched_barrier(0);
                    top_next = opread(st, TW + wv_t * WTT + 16);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int w = 0; w < NW; ++w) prev[w] = cur[w];
            s_prev = sa[t] * sb;
            top = top_next;
        }
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            if (FIRST) promote_first(acc[w][NT - 1], prev[w], s_prev);
            else promote(acc[w][NT - 1], prev[w], s_prev);
        }
    };

    // Tiles with one group per barrier write C from the last group itself
    // (tiles without a K split): its step issues no loads, so the stage of
    // the group before (read by every wave before the barrier, and the
    // target of no later load) is idle, and token block t's C rows are
    // final once its products are promoted.  Each wave stages them in its
    // own 16-row slice of the idle stage (reused block after block: a wave's
    // LDS operations run in order) and stores them while the MFMAs of the
    // later blocks run, instead of after a barrier at the end:
    // 1-5% faster on tiles from 128x128 up (smaller ones, whose epilogue is
    // short, do not gain), bitwise the same output.  Only fp8bg_ring_dp (the
    // kernel of launches without split tiles) takes this path: beside the
    // split tiles' end epilogue the large tiles' registers spill.  The
    // products are promoted right after their own MFMAs here (no second set
    // of product registers).
    constexpr bool kEarlyC = ring_has_dp(TW, TT, KF, KU, WK) && DPO;
    static_assert(!kEarlyC || NWAVE * 16 * ROWB <= STAGE, "C staging inside the idle stage");
    // Packing of a finished token block: with a bias, C is rounded, the bias
    // added and the sum rounded again (every value canonicalised); without
    // one, a single wave-wide unordered compare per block decides whether
    // any value needs NaN canonicalisation at all, and otherwise the
    // conversion instruction alone packs it.
    auto group_last = [&](int i, auto has_bias) __attribute__((always_inline)) {
        constexpr bool HB = decltype(has_bias)::value;
        const unsigned char* st = lds + (i % ST) * STAGE;
        const float* sc = (const float*)(st + OPS);
        unsigned char* reg = lds + ((i + ST - 1) % ST) * STAGE + wave * (16 * ROWB);
        const uint16_t* bl = (const uint16_t*)(st + OPS + (TT + NBS) * 4);
        i32x8 top = opread(st, TW + wv_t * WTT);
        i32x8 wop[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) wop[w] = wread(st, wv_w * WTW + w * 16);
        const float sb = sc[TT + (w0c % 128 + wv_w * WTW) / 128];
        const int r = lane & 15, qd = lane >> 4;
        // byte offsets of the lane's C chunks inside a 16-row block
        constexpr int HC = (16 * CPR + 63) / 64;
        uint32_t voff[HC];
#pragma unroll
        for (int h = 0; h < HC; ++h) {
            const int idx = lane + 64 * h;
            const int row = idx / CPR, n = w0 + wv_w * WTW + (idx % CPR) * 8;
            voff[h] = row < 16 && n < a.N ? (uint32_t)(row * a.N + n) * 2u : 0x80000000u;
        }
        float sa[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) sa[t] = sc[wv_t * WTT + r * NT + t];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float s_t = sa[t] * sb;
            i32x8 top_next = top;
            if (t + 1 < NT) top_next = opread(st, TW + wv_t * WTT + (t + 1) * 16);
#pragma unroll
            for (int w = 0; w < NW; ++w) promote(acc[w][t], mfma16x16x128(wop[w], top), s_t);
            top = top_next;
            // rows of token block t: chunk c of row r at slot c ^ (r % CPR)
            const int mb = t0 + wv_t * WTT + t * 16;        // wave-uniform
            uint2 pk[NW];
            if constexpr (HB) {
#pragma unroll
                for (int w = 0; w < NW; ++w)
                    pk[w] = out_bf16x4v(acc[w][t], true, *(const uint2*)(bl + wv_w * WTW + w * 16 + qd * 4));
            } else {
                bool nan = false;
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    pk[w] = pack_bf16x4_nonan(acc[w][t]);
                    nan = nan | __builtin_isunordered(acc[w][t][0], acc[w][t][1]) |
                          __builtin_isunordered(acc[w][t][2], acc[w][t][3]);
                }
                if (__builtin_amdgcn_ballot_w64(nan) != 0) {
                    asm volatile("" ::: "memory");    // stays a branch: not computed speculatively
#pragma unroll
                    for (int w = 0; w < NW; ++w) pk[w] = pack_bf16x4(acc[w][t]);
                }
            }
#pragma unroll
            for (int w = 0; w < NW; ++w)
                *(uint2*)(reg + r * ROWB + (((2 * w + (qd >> 1)) ^ (r % CPR)) << 4) + (qd & 1) * 8) = pk[w];
            // The block's 16 rows through a buffer resource based at row mb
            // and sized to the rows that exist (below 2^31 bytes: the host
            // checks 32 N): rows past M, and columns past N (offset 2^31),
            // fall outside it and are dropped.
            // (both wave-uniform; readfirstlane says so to the compiler,
            // which otherwise builds the resource per lane in a loop)
            const int rows = __builtin_amdgcn_readfirstlane(min(max(a.M - mb, 0), 16));
            const uint64_t cbase = (uint64_t)(a.C + (size_t)mb * a.N);
            const uint64_t cb = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(cbase >> 32)) << 32) |
                                (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)cbase);
            const __amdgpu_buffer_rsrc_t crs =
                __builtin_amdgcn_make_buffer_rsrc((void*)cb, (short)0, rows * a.N * 2, kBufferFlags);
#pragma unroll
            for (int h = 0; h < HC; ++h) {
                const int idx = lane + 64 * h;
                const int row = idx / CPR, c = idx % CPR;
                if (row >= 16) continue;
                const i32x4 v = *(const i32x4*)(reg + row * ROWB + ((c ^ (row % CPR)) << 4));
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), crs, voff[h], 0,
                                                       kNonTemporal);
            }
        }
    };

    // One barrier step: groups i .. i + KU - 1, with (load) or without the
    // loads of groups i + ST - KU .. i + ST - 1.
    auto step = [&](int i, auto role, auto load, auto first) {
        // Groups i .. i + KU - 1 are complete once at most the DMA
        // instructions of the ST - 2 KU later groups are outstanding (vmcnt
        // retires in issue order; a wave loads only its slice's groups, 1 in
        // WK); this wave's LDS reads of the KU groups before have all
        // returned.
        wait_vmcnt_lds<NDMA * (ST - 2 * KU) / WK>();
        // All waves' blocks of those stages have landed, and every wave is
        // done reading the stages of groups i - KU .. i - 1, which are
        // refilled next.  The empty asm statements keep the compiler from
        // moving LDS reads or writes across the barrier.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int uk = 0; uk < KU / WK; ++uk) {
            // group i + ST - KU + u refills the stage of group i - KU + u;
            // both belong to this wave's slice
            const int u = uk * WK + ks;
            const int g = i + ST - KU + u;
            if (decltype(first)::value && uk == 0)
                group(i + u, load_idx(g), g % ST, role, load, First<true>{});
            else
                group(i + u, load_idx(g), g % ST, role, load, First<false>{});
        }
    };
    // Stream-K: the end of one tile's part of a run (groups g_begin ..
    // g_end - 1 of tile tile_), per wave.  A part covering the whole tile
    // writes C.  Otherwise the tile's parts come from consecutive runs (2 or
    // 3: the host keeps a run at least half a tile long), and the part
    // holding the tile's last group is the owner.  Every other part stores
    // its fp32 partial with device-scope stores (coherent across the XCDs'
    // L2s), waits for them and counts itself in the tile's per-wave counter.
    // The owner first reads the counter: when all the other parts are
    // counted it sums the tile without storing its own partial; otherwise it
    // stores and counts itself too, and the part whose count completes the
    // tile sums it.  The sum runs in K order over the parts (each part's
    // value from its partial, or its own registers), so C does not depend on
    // which part sums; that part writes C with the bias and resets the
    // counter.  No wave waits for another.  Partial slots: 2 w + 1 holds the
    // part of run w that is its second tile's head, 2 w the other part.
    auto sk_finish = [&](int tile_, int w0_, int t0_, int g_begin, int g_end, int own_slot)
        __attribute__((always_inline)) {
        const int r = lane & 15, qd = lane >> 4;
        auto write_c = [&]() {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const int m = t0_ + wv_t * WTT + t * 16 + r, n = w0_ + wv_w * WTW + w * 16 + qd * 4;
                    if (m < a.M && n < a.N) *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(acc[w][t], a.bias, n);
                }
        };
        if (g_begin == 0 && g_end == KG) {
            write_c();
            return;
        }
        const int tkg = tile_ * KG;
        const int wa = tkg / a.kcount, wb = (tkg + KG - 1) / a.kcount;
        const int parts = wb - wa + 1;            // 2 or 3
        const int pos = sk_w - wa;                // this part's place in K order
        const uint32_t others = (uint32_t)(parts - 1);
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.ws, (short)0, 0x7fffffff, kBufferFlags);
        auto part_off = [&](int slot, int w, int t) -> uint32_t {
            return ((((uint32_t)slot * NWAVE + wave) * (NW * NT) + (uint32_t)(w * NT + t)) * 64u + lane) * 16u;
        };
        auto store_part = [&]() {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[w][t]), wrs,
                                                           part_off(own_slot, w, t), 0, kDeviceScope);
            asm volatile("" ::: "memory");
            wait_vmcnt<0>();
            asm volatile("" ::: "memory");
        };
        uint32_t* cnt = a.cnt + tile_ * NWAVE + wave;
        uint32_t seen = 0;
        bool sum_here;
        if (g_end == KG) {
            if (lane == 0) seen = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sum_here = __builtin_amdgcn_readfirstlane(seen) == others;
            if (!sum_here) {
                store_part();
                if (lane == 0) seen = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sum_here = __builtin_amdgcn_readfirstlane(seen) == others;
            }
        } else {
            store_part();
            if (lane == 0) seen = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sum_here = __builtin_amdgcn_readfirstlane(seen) == others;
        }
        if (!sum_here) return;
        asm volatile("" ::: "memory");
        // the other parts in K order: o0, then o1 (three parts)
        const int p0 = pos == 0 ? 1 : 0, p1 = pos <= 1 ? 2 : 1;
        auto slot_of = [&](int p) { return 2 * (wa + p) + (p == 0 && wa * a.kcount < tkg ? 1 : 0); };
        const int s0 = slot_of(p0), s1 = slot_of(p1);
        f32x4 o0[NW][NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int w = 0; w < NW; ++w)
                o0[w][t] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, part_off(s0, w, t), 0, kDeviceScope));
        if (parts == 3) {
            f32x4 o1[NW][NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w)
                    o1[w][t] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, part_off(s1, w, t), 0, kDeviceScope));
            // (P0 + P1) + P2, with this part's own value in its place
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    if (pos == 2)
                        acc[w][t] = (o0[w][t] + o1[w][t]) + acc[w][t];
                    else
                        acc[w][t] = (acc[w][t] + o0[w][t]) + o1[w][t];
                }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w) acc[w][t] = acc[w][t] + o0[w][t];
        }
        write_c();
        if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // The last step is peeled off outside the loop (a second copy inside the
    // loop body would make the large tiles spill).
    // a uniform branch around two copies of the loop, so the priority
    // switches are immediates inside straight-line code
    if constexpr (SK) {
        // the first tile's steps, its part's end, then the second tile's
        // steps; the ring's loads run on across the tiles (load_idx counts
        // the run's units)
        if (kcount > KU) {
            step(0, WaveRole<0>{}, Loads<true>{}, First<true>{});
            int i = KU;
            for (; i < n1 && i + KU < kcount; i += KU) step(i, WaveRole<0>{}, Loads<true>{}, First<false>{});
            if (n1 < kcount) {
                sk_finish(tile, w0, t0, 0, n1, 2 * sk_w + 1);
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[w][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
                w0c = w0b;
                for (; i + KU < kcount; i += KU) step(i, WaveRole<0>{}, Loads<true>{}, First<false>{});
            }
            step(kcount - KU, WaveRole<0>{}, Loads<false>{}, First<false>{});
        } else {
            step(0, WaveRole<0>{}, Loads<false>{}, First<true>{});
        }
    } else if constexpr (kEarlyC) {
        // the last step is dispatched after the loop, and the C-writing one
        // returns right away (a path that rejoined the epilogue would keep
        // the epilogue's registers alive through it)
        // (the host launches fp8bg_ring_dp, and the ring kernels that have
        // this path take it, only where a tile has more than one step)
        auto main_loop = [&](auto role) {
            step(0, role, Loads<true>{}, First<true>{});
            for (int i = KU; i + KU < kcount; i += KU) step(i, role, Loads<true>{}, First<false>{});
        };
        if (kPrio && wv_t) {
            main_loop(WaveRole<1>{});
        } else {
            main_loop(WaveRole<0>{});
        }
        if (DPO || blockIdx.x < a.n_dp) {
            // vmcnt(0): the clamped loads of deeper rings land here, so none
            // writes the LDS after this workgroup has returned
            wait_vmcnt_lds<0>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (kPrio) __builtin_amdgcn_s_setprio(0);
            if (a.bias)
                group_last(kcount - 1, Loads<true>{});
            else
                group_last(kcount - 1, Loads<false>{});
            return;
        }
        if (kPrio && wv_t) {
            step(kcount - KU, WaveRole<1>{}, Loads<false>{}, First<false>{});
        } else {
            step(kcount - KU, WaveRole<0>{}, Loads<false>{}, First<false>{});
        }
    } else {
        auto main_loop = [&](auto role) {
            if (kcount > KU) {
                step(0, role, Loads<true>{}, First<true>{});
#pragma unroll (KF > 2 * KU ? KF / KU - 2 : 1)
                for (int i = KU; i + KU < kcount; i += KU) step(i, role, Loads<true>{}, First<false>{});
                step(kcount - KU, role, Loads<false>{}, First<false>{});
            } else {
                step(0, role, Loads<false>{}, First<true>{});
            }
        };
        if (kPrio && wv_t) {
            main_loop(WaveRole<1>{});
        } else {
            main_loop(WaveRole<0>{});
        }
    }
    if (kPrio) __builtin_amdgcn_s_setprio(0);
    // The clamped loads of the last ST - 2 KU groups are still in flight: they
    // must land before the LDS is reused below or handed to another workgroup.
    wait_vmcnt<0>();
    if constexpr (SK) {
        if (n1 < kcount)
            sk_finish(tile2, w0b, t0b, k_lo2, KG, 2 * sk_w);
        else
            sk_finish(tile, w0, t0, k_lo, k_lo + kcount, 2 * sk_w);
        return;
    }

    // ---- epilogue ----
    const bool dp = blockIdx.x < a.n_dp;
    const int r = lane & 15, qd = lane >> 4;
    // The bias row sits in the last group's scale area: read it before the
    // LDS is reused.
    uint2 bv[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) bv[w] = (uint2){0u, 0u};
    if (dp) {
        const uint16_t* bl = (const uint16_t*)(lds + ((kcount - 1) % ST) * STAGE + OPS +
                                               (TT + NBS) * 4);
#pragma unroll
        for (int w = 0; w < NW; ++w)
            bv[w] = *(const uint2*)(bl + wv_w * WTW + w * 16 + qd * 4);
    }
    if (WK > 1) {
        // slices 1 .. WK-1 park their partial tiles in the (now free) ring;
        // slice 0 adds them in slice order
        f32x4* red = (f32x4*)lds;
        wait_vmcnt_lds<0>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (ks > 0) {
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    red[(((ks - 1) * NWAVE + wave) * NW * NT + w * NT + t) * 64 + lane] = acc[w][t];
        }
        wait_vmcnt_lds<0>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (ks == 0) {
            for (int k2 = 1; k2 < WK; ++k2)
#pragma unroll
                for (int w = 0; w < NW; ++w)
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const f32x4 v = red[(((k2 - 1) * NWAVE + wave) * NW * NT + w * NT + t) * 64 + lane];
                        acc[w][t][0] += v[0];
                        acc[w][t][1] += v[1];
                        acc[w][t][2] += v[2];
                        acc[w][t][3] += v[3];
                    }
        }
        if (ks > 0) return;
    }
    // with K slices, slice 0 stages C after the parked partial tiles, so it
    // needs no barrier between adding them and writing C
    constexpr int kCOff = (WK - 1) * TW * TT * 4;
    static_assert(kCOff + NWAVE * WTT * ROWB <= ST * STAGE, "C staging after the partial tiles");
    if (dp) {
        // bf16 C through LDS: once every wave has passed the barrier below the
        // whole ring is free, and each wave of slice 0 writes its WTT x WTW
        // tile into its own region (row-major, chunk c of row r at slot
        // c ^ (r % CPR)), reads it back as whole 16-byte chunks and stores
        // full 128-byte lines with non-temporal stores (C is not re-read).
        if (WK == 1) {
            wait_vmcnt_lds<0>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        unsigned char* region = lds + kCOff + wave * (WTT * ROWB);
        auto stage_c = [&](auto pack) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const int row = t * 16 + r;
                    *(uint2*)(region + row * ROWB + (((2 * w + (qd >> 1)) ^ (row % CPR)) << 4) +
                              (qd & 1) * 8) = pack(acc[w][t], bv[w]);
                }
        };
        // Three copies of the packing loop, picked once per wave: with a
        // bias; without, for a wave with no NaN accumulator (the conversion
        // instruction alone); and without, canonicalising NaN.
        if (a.bias)
            stage_c([](const f32x4& v, uint2 b) { return out_bf16x4v(v, true, b); });
        else if (!wave_has_nan(acc))
            stage_c([](const f32x4& v, uint2) { return pack_bf16x4_nonan(v); });
        else
            stage_c([](const f32x4& v, uint2) { return pack_bf16x4(v); });
#pragma unroll
        for (int h = 0; h < (WTT * CPR + 63) / 64; ++h) {
            const int idx = lane + 64 * h;
            const int row = idx / CPR, c = idx % CPR;
            if (row >= WTT) continue;
            const i32x4 v = *(const i32x4*)(region + row * ROWB + ((c ^ (row % CPR)) << 4));
            const int m = t0 + wv_t * WTT + row, n = w0 + wv_w * WTW + c * 8;
            if (m < a.M && n < a.N)
                __builtin_nontemporal_store(v, (i32x4*)(a.C + (size_t)m * a.N + n));
        }
        return;
    }
    if (ks > 0) return;
    if constexpr (LAST) {
        // Split-K reduced in this kernel (the reference's last-arriver
        // reduction, kernels/baseline_gluon.py:194-209), per wave: each wave
        // stores its WTT x WTW part of the tile's partial with device-scope
        // stores (coherent across the XCDs' L2s), waits for them, and counts
        // them in the counter of its part; the wave that completes the count
        // sums the part over the splits in split order (fp8bg_split_reduce's
        // order, so C is bitwise the two-kernel result), writes C and resets
        // the counter.  No wave waits for another and no barrier is needed.
        const int stile = tile - a.n_dp;
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.ws, (short)0, 0x7fffffff, kBufferFlags);
        auto part_off = [&](int sp, int t, int w) -> uint32_t {
            const int tl = wv_t * WTT + t * 16 + r, wl = wv_w * WTW + w * 16 + qd * 4;
            return ((uint32_t)(stile * a.split + sp) * (uint32_t)(TW * TT) + (uint32_t)(tl * TW + wl)) * 4u;
        };
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int w = 0; w < NW; ++w)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[w][t]), wrs,
                                                       part_off(sidx, t, w), 0, kDeviceScope);
        asm volatile("" ::: "memory");
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        uint32_t* cnt = a.cnt + stile * NWAVE + wave;
        uint32_t arrived = 0;
        if (lane == 0) arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane(arrived) != (uint32_t)(a.split - 1)) return;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                f32x4 sum = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, part_off(0, t, w), 0, kDeviceScope));
                for (int sp = 1; sp < a.split; ++sp) {
                    const f32x4 v = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, part_off(sp, t, w), 0, kDeviceScope));
                    sum[0] += v[0];
                    sum[1] += v[1];
                    sum[2] += v[2];
                    sum[3] += v[3];
                }
                const int m = t0 + wv_t * WTT + t * 16 + r, n = w0 + wv_w * WTW + w * 16 + qd * 4;
                if (m < a.M && n < a.N) *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(sum, a.bias, n);
            }
        if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    float* mine = a.ws + ((size_t)(tile - a.n_dp) * a.split + sidx) * (size_t)(TW * TT);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int tl = wv_t * WTT + t * 16 + (lane & 15);
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int wl = wv_w * WTW + w * 16 + (lane >> 4) * 4;
            *(f32x4*)(mine + tl * TW + wl) = acc[w][t];
        }
    }
}

template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, false>(a);
}

// The same with the split-K reduction inside the kernel (FP8BG_SPLIT_LAST),
// for the instances ring_has_last names: a kernel of its own, so that the
// other launches do not carry its epilogue.
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_last(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, true>(a);
}

// The same for launches without split tiles: with no epilogue path left
// beside the last group's C writes, the 256x256 tile takes them too (in the
// kernel above its registers would spill at the loop's end).
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_dp(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, true, false>(a);
}

// Stream-K (FP8BG_SPLIT_STREAM), for the instances ring_has_sk names.
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_sk(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, false, false, true>(a);
}
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_sk_bs(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, false, true, true>(a);
}

// The three ring kernels for a shuffled B (FP8BG_FLAG_B_SHUFFLED).
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_bs(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, false, true>(a);
}
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_last_bs(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, false, true, true>(a);
}
template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK>
__global__ __launch_bounds__(64 * WW * WT * WK)
__attribute__((amdgpu_waves_per_eu((WW * WT * WK + 3) / 4, (WW * WT * WK + 3) / 4)))
void fp8bg_ring_dp_bs(KArgs a) {
    ring_body<TW, TT, WW, WT, ST, KF, KU, WK, true, false, true>(a);
}

// An activation group's scale s = RN(x / 448) and its reciprocal RN(1 / s),
// x = max(amax, eps), for the activation quantisers: in the few-token one
// two IEEE division sequences (or a branch around them) would sit on each
// group's dependent chain, in the standalone one they cost VALU time.  x is
// either eps, whose s and 1/s the host computes once, or the bf16 amax
// itself (in the fused kernel at least eps >= 1e-30 > 2^-100; the standalone
// one takes this pair only where s >= 2^-60).  For a finite bf16 x of
// at least 2^-100, s is the product with RN(1/448) corrected by one FMA of
// its exact remainder, and 1/s is v_rcp_f32 (within 1 ulp) refined by one
// Newton step.  Both equal the correctly rounded quotients there: the
// quotient was checked for all 32,639 positive finite bf16 x, and the Newton
// step from every start value within 2 ulp of RN(1/s) for every s of that
// range (tests/fastdiv_check.c).  From 2^-100 on, no remainder or
// intermediate is subnormal.
__device__ __forceinline__ void act_scale_reciprocal_fast(float x, float& s, float& r) {
#pragma clang fp contract(off)
    constexpr float kInv448 = 1.0f / 448.0f;
    const float q0 = x * kInv448;
    s = __builtin_fmaf(__builtin_fmaf(-q0, 448.0f, x), kInv448, q0);
    const float r0 = __builtin_amdgcn_rcpf(s);
    r = __builtin_fmaf(__builtin_fmaf(-s, r0, 1.0f), r0, r0);
}

// ===========================================================================
// Small-M kernel: operands straight from global memory, waves split K
// ===========================================================================
// With QA the token operand is quantised in registers from bf16 activations:
// the quad of lanes holding one token's 128-K group reduces its amax by two
// DPP permutations, s = max(amax, eps) / 448 and each value becomes
// e4m3(x * (1 / s)) through v_cvt_pk_fp8_f32 (round to nearest even; the
// same code as the integer encoder for every non-NaN input).  The
// reciprocal replaces the standalone quantiser's division: one multiply per
// value instead of a division sequence, which is what makes the fused path
// cheaper than a separate kernel.
// MODE bits: the fused quantiser, and the in-kernel split-K reduction
// (FP8BG_SPLIT_LAST).  The reduction is compiled only into its own instances:
// its epilogue, even when not taken, costs the common instances registers
// (skinny<2,1,8,1> 80 -> 86 VGPRs, one workgroup per CU fewer).
// kSkinnyQuantFew: the fused quantiser for launches with at most 4 tokens
// (16-token tiles, so one token tile).  The general quantiser gives each lane
// 32 values of one of the tile's 16 tokens: with M = 1 only 4 lanes hold real
// ones, and every wave of every workgroup runs the full per-value chain.
// Here the real tokens' 128 values of a group are spread over the whole wave
// (lane l: token l / 16, values 8 (l % 16) .. + 7); the amax is an unsigned
// max of the bf16 magnitude bits (exact, and NaN propagates: its magnitude
// bits exceed infinity's) over the token's 16 lanes by DPP row rotations;
// the codes go back to the MFMA operand layout through the wave's own slice
// of the reduction LDS.  Same scales and codes as the general path, so the
// host may take it for any launch with M <= 4.
// kSkinnyFewTokens: fp8 tokens for launches with at most 8 of them.  Rows of
// the 16-token operand at or past M feed only outputs that are never stored,
// so one 16-byte load per lane covers the group of rows 0..7 (lane l: row
// l >> 3, chunk l & 7): half the L1 accesses of the two loads that cover 16
// rows, which at M <= 8 cost as much as the weights' own loads.  The same
// eight ds_bpermute passes give MFMA lane (r, q) chunks q and 4 + q of row
// r & 7; bitwise the same C as the general path.  Taken on tiles of 16 and
// 32 weight rows (see the skinny launcher).
// kSkinnyBShuf: B in the shuffled layout (FP8BG_FLAG_B_SHUFFLED): the 2 KB
// of a 16-row block's 128-K group are stored in MFMA lane order, so lane l's
// loads at bytes 16 l and 1024 + 16 l of the block are its operand as they
// arrive, and the weights need no ds_bpermute.
// kSkinnyDirectTokens: fp8 tokens loaded in the MFMA layout, for launches with at
// most two tokens and row-major B (see the skinny launcher).  Rows of the 16-token operand at or past M
// reach no stored output, so lane (r, q) loads row min(r, M - 1)'s chunks q
// and 4 + q itself and the tokens need no ds_bpermute; with one token its
// scale of a group is one value for the wave (v_readlane), else the lane's
// row's scale comes by ds_bpermute as in the general path.  Bitwise the same
// C as the general path.
constexpr int kSkinnyQuant = 1, kSkinnyLast = 2, kSkinnyQuantFew = 4, kSkinnyFewTokens = 8,
              kSkinnyBShuf = 16, kSkinnyDirectTokens = 32;
template <int NWB, int NTB, int S, int U, int MODE>
__global__ __launch_bounds__(64 * S) void fp8bg_skinny(KArgs a) {
    constexpr int TW = 16 * NWB, TT = 16 * NTB, NB = NWB * NTB;
    constexpr bool QA = MODE & kSkinnyQuant, LAST = MODE & kSkinnyLast;
    constexpr bool QF = MODE & kSkinnyQuantFew;
    constexpr bool FT = MODE & kSkinnyFewTokens;
    constexpr bool BSH = MODE & kSkinnyBShuf;
    constexpr bool DT = MODE & kSkinnyDirectTokens;
    static_assert(!DT || (!QA && !FT && NTB == 1), "the direct token load takes one 16-token tile of fp8 tokens");
    static_assert(!QF || (QA && NTB == 1), "the few-token quantiser takes one 16-token tile");
    static_assert(!FT || (!QA && NTB == 1), "the few-token load takes one 16-token tile of fp8 tokens");
    __shared__ f32x4 red[S][NB][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;

    // Tokens vary fastest, so the workgroups that share weight rows are
    // adjacent (and, with xcd_remap, on one XCD's L2).
    // With a cross-workgroup split (full mode only) workgroup pid computes
    // K range pid % split of tile pid / split.
    // (divisions by the split and by tiles_t through host-computed
    // reciprocals: the decode's first loads wait on this arithmetic)
    // The fields are read up front and the tile decoded without branches,
    // so the argument loads issue together instead of one round per branch.
    const int pid = blockIdx.x;
    const int split = a.split, tiles_t = a.tiles_t, remap = a.xcd_remap;
    const int tiles = a.tiles_w * tiles_t;
    const int kcount = a.kcount;
    const uint2 div_split = a.div_split, div_tiles_t = a.div_tiles_t;
    const int q_split = (int)fast_div(pid, div_split);
    const int tile = split > 1 ? q_split : remap ? xcd_remap(pid, tiles) : pid;
    const int sidx = split > 1 ? pid - q_split * split : 0;
    const int pw = (int)fast_div(tile, div_tiles_t), pt = tile - pw * tiles_t;
    const int w0 = pw * TW, t0 = pt * TT;
    const int k_lo = sidx * kcount;

    // Operand loads are coalesced: lane l reads row l >> 2 of a 16-row block,
    // 16-byte chunks (l & 3) and 4 + (l & 3) of the 128-byte group, so a quad
    // of lanes reads 64 contiguous bytes of ONE row (one L1 access; a quad
    // spread over four rows costs four, and the L1's access rate, not HBM,
    // then bounds the kernel).  ds_bpermute hands MFMA lane (r, q) the data
    // of loading lane 4 r + q: row r, chunks q and 4 + q (K bytes [16 q, +16)
    // and [64 + 16 q, +16)).  Weights and tokens use this one byte -> K
    // assignment, so each MFMA still reduces exactly its group's 128 products.
    const int lr = lane >> 2, lc = lane & 3;
    const int op_src = (4 * r + q) << 2;
    // The Bs block of the whole tile (where TW divides 128 the tile's rows
    // share one; a 48-row tile may reach into the next block, whose scales
    // come from a second pointer, and each 16-row block takes the scale of
    // the block holding its rows) and the As rows, read with one load per
    // batch: lane l takes group slot u of token row l >> 2 (row-major As: a
    // quad reads 4 nearby floats of one row) or u = l >> 4 of row l & 15
    // (column-major As), and lane (r, q) gets its row's scale of slot u by
    // ds_bpermute.
    constexpr bool kTwoBs = 128 % TW != 0;
    static_assert(TW <= 128 && (TW % 16) == 0, "a skinny tile spans at most two 128-row Bs blocks");
    const bool as_cm = a.as_sm == 1;
    const int sa_row = as_cm ? (lane & 15) : lr, sa_u = as_cm ? (lane >> 4) : lc;
    const float* bsp = a.Bs + (int64_t)(w0 >> 7) * a.bs_sn;
    const float* bsp2 = kTwoBs ? a.Bs + (int64_t)min((w0 + TW - 1) >> 7, a.N / 128 - 1) * a.bs_sn : bsp;
    // shuffled B: block (b, g) of 16 rows and one group at (b K/128 + g) 2 KB
    const int KGB = a.K / kGroupK;
    const uint8_t* wp[NWB];
#pragma unroll
    for (int w = 0; w < NWB; ++w)
        wp[w] = BSH ? a.B + (size_t)min((w0 >> 4) + w, (a.N >> 4) - 1) * KGB * kShufBlock + 16 * lane
                    : a.B + (size_t)min(w0 + 16 * w + lr, a.N - 1) * a.K + 16 * lc;
    const uint8_t* tp[NTB];
    const float* asp[NTB];
    const uint16_t* xp[NTB];
#pragma unroll
    for (int t = 0; t < NTB; ++t) {
        if (QF) {
            // few-token quantiser: lane l reads token l / 16, values 8 (l % 16) ..
            xp[t] = a.X + (size_t)min(q, a.M - 1) * a.ldx + 8 * r;
        } else if (QA) {
            // loading lane l: token l >> 2, values [16 (l & 3), +16) and
            // [64 + 16 (l & 3), +16) (a quad holds the token's whole group)
            xp[t] = a.X + (size_t)min(t0 + 16 * t + lr, a.M - 1) * a.ldx + 16 * lc;
        } else {
            // (the launch's only token tile starts at row 0)
            tp[t] = DT   ? a.A + (size_t)min(r, a.M - 1) * a.K + 16 * q
                    : FT ? a.A + (size_t)min(t0 + (lane >> 3), a.M - 1) * a.K + 16 * (lane & 7)
                         : a.A + (size_t)min(t0 + 16 * t + lr, a.M - 1) * a.K + 16 * lc;
            asp[t] = a.As + (int64_t)min(t0 + 16 * t + sa_row, a.M - 1) * a.as_sm;
        }
    }
    // few-token quantiser: the codes of token r of a group, for the lanes of
    // token r (r < 4), in this wave's slice of the reduction LDS (in order:
    // a wave's LDS accesses execute in issue order)
    unsigned char* qstage = (unsigned char*)&red[wave][0][0];
    // side outputs of the fused quantiser come from the first weight tile
    const bool qa_write = QA && a.q_out != nullptr && pw == 0;

    f32x4 acc[NWB][NTB];
#pragma unroll
    for (int w = 0; w < NWB; ++w)
#pragma unroll
        for (int t = 0; t < NTB; ++t) acc[w][t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // This wave's groups: k_lo + wave + S*j, j = 0 .. J-1, in batches of U.
    // Where the doubled operand registers fit (kPipe), the next batch's loads
    // are issued before the current batch is computed, so a wave has two
    // batches of weight bytes in flight instead of one round trip per batch
    // (the accumulation order, and so the result, is the same either way).
    const int J = wave < kcount ? (kcount - 1 - wave) / S + 1 : 0;
    struct Batch {
        i32x4 wl[U][NWB][2], tl[QA ? 1 : U][QA ? 1 : NTB][2];   // as loaded (coalesced)
        i32x8 tv[U][NTB];                                       // quantised tokens (QA)
        i32x4 xr[QA ? U : 1][QA ? NTB : 1][QF ? 1 : 4];
        float sa[U][NTB];                                       // token scales (QA)
        float sar[NTB], sbr, sbr2;                              // lane-indexed scales
    };
    // Loads are issued unconditionally (a group index past the wave's last
    // group is clamped to it; compute skips those), so they form straight-
    // line code and each batch's computation waits only for its own loads.
    auto group = [&](int j) __attribute__((always_inline)) { return k_lo + wave + S * min(j, J - 1); };
    auto load = [&](Batch& b, int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t go = (size_t)group(j0 + u) * kGroupK;
            const size_t gw = BSH ? (size_t)group(j0 + u) * kShufBlock : go;
#pragma unroll
            for (int w = 0; w < NWB; ++w) {
                b.wl[u][w][0] = *(const i32x4*)(wp[w] + gw);
                b.wl[u][w][1] = *(const i32x4*)(wp[w] + gw + (BSH ? kShufBlock / 2 : 64));
            }
#pragma unroll
            for (int t = 0; t < NTB; ++t) {
                if (QF) {
                    b.xr[u][t][0] = *(const i32x4*)(xp[t] + go);
                } else if (QA) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        b.xr[u][t][c] = *(const i32x4*)(xp[t] + go + 8 * (c & 1) + 64 * (c >> 1));
                } else {
                    b.tl[u][t][0] = *(const i32x4*)(tp[t] + go);
                    if (!FT) b.tl[u][t][1] = *(const i32x4*)(tp[t] + go + 64);
                }
            }
        }
        b.sbr = bsp[(int64_t)group(j0 + min(lane, U - 1)) * a.bs_sk];
        if constexpr (kTwoBs) b.sbr2 = bsp2[(int64_t)group(j0 + min(lane, U - 1)) * a.bs_sk];
        if (!QA) {
#pragma unroll
            for (int t = 0; t < NTB; ++t) b.sar[t] = asp[t][(int64_t)group(j0 + min(sa_u, U - 1)) * a.as_sk];
        }
    };
    // MFMA operand of lane (r, q) from the coalesced loads of a 16-row block
    // (few-token load: chunk q of row r & 7 sits in loading lane 8 (r & 7) + q,
    // chunk 4 + q in lane 8 (r & 7) + 4 + q)
    const int few_src = (8 * (r & 7) + q) << 2;
    auto gather_few = [&](const i32x4& v) __attribute__((always_inline)) {
        i32x8 o;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            o[d] = __builtin_amdgcn_ds_bpermute(few_src, v[d]);
            o[4 + d] = __builtin_amdgcn_ds_bpermute(few_src + 16, v[d]);
        }
        return o;
    };
    auto gather = [&](const i32x4 (&v)[2]) __attribute__((always_inline)) {
        i32x8 o;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            o[d] = __builtin_amdgcn_ds_bpermute(op_src, v[0][d]);
            o[4 + d] = __builtin_amdgcn_ds_bpermute(op_src, v[1][d]);
        }
        return o;
    };
    auto compute = [&](Batch& b, int j0) __attribute__((always_inline)) {
        if constexpr (QF) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (j0 + u < J) {
                    const int g = k_lo + wave + S * (j0 + u);
                    const i32x4 xv = b.xr[u][0][0];
                    // max of the 8 magnitudes (bf16 bits), then over the
                    // token's 16 lanes: rotations by 1, 2, 4, 8 in the row
                    uint32_t mx = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t d = (uint32_t)xv[i] & 0x7fff7fffu;
                        mx = max(mx, max(d & 0xffffu, d >> 16));
                    }
                    mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0x121, 0xf, 0xf, false));
                    mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0x122, 0xf, 0xf, false));
                    mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0x124, 0xf, 0xf, false));
                    mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0x128, 0xf, 0xf, false));
                    const bool nan = mx > 0x7f80u;
                    // s = max(amax, eps) / 448 and 1/s without a division:
                    // eps's pair from the host, an infinite amax gives
                    // (inf, 0), any other amax >= eps the exact fast pair
                    const float amax = __uint_as_float(mx << 16);
                    float sf, rf;
                    act_scale_reciprocal_fast(amax, sf, rf);
                    const bool inf = mx == 0x7f80u, above = amax >= a.eps;
                    const float sc = nan ? __builtin_nanf("") : inf ? amax : above ? sf : a.eps_s;
                    const float rcp = nan ? __builtin_nanf("") : inf ? 0.0f : above ? rf : a.eps_r;
                    int o[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t lo = (uint32_t)xv[2 * i], hi = (uint32_t)xv[2 * i + 1];
                        int d = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(lo << 16) * rcp,
                                                                __uint_as_float(lo & 0xffff0000u) * rcp, 0, false);
                        d = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(hi << 16) * rcp,
                                                            __uint_as_float(hi & 0xffff0000u) * rcp, d, true);
                        o[i] = d;
                    }
                    asm volatile("" ::: "memory");
                    *(uint2*)(qstage + q * kGroupK + 8 * r) = make_uint2((uint32_t)o[0], (uint32_t)o[1]);
                    asm volatile("" ::: "memory");
                    i32x8 tv = {0, 0, 0, 0, 0, 0, 0, 0};
                    float sa = 0.f;
                    // lane (r, q) takes codes [16 q, +16) and [64 + 16 q, +16)
                    // of token r and its scale (held by lanes 16 r .. 16 r + 15)
                    const float sc_r = __shfl(sc, 16 * (r & 3));
                    if (r < 4) {
                        const i32x4 lo = *(const i32x4*)(qstage + r * kGroupK + 16 * q);
                        const i32x4 hi = *(const i32x4*)(qstage + r * kGroupK + 64 + 16 * q);
                        tv = (i32x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        sa = sc_r;
                    }
                    asm volatile("" ::: "memory");
                    b.tv[u][0] = tv;
                    b.sa[u][0] = sa;
                    if (qa_write && q < a.M) {
                        uint8_t* qd = a.q_out + (size_t)q * a.K + (size_t)g * kGroupK + 8 * r;
                        *(uint2*)qd = make_uint2((uint32_t)o[0], (uint32_t)o[1]);
                        if (r == 0) a.s_out[q * a.qs_sm + g * a.qs_sk] = sc;
                    }
                }
            }
        } else if (QA) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (j0 + u < J) {
                    const int g = k_lo + wave + S * (j0 + u);
#pragma unroll
                    for (int t = 0; t < NTB; ++t) {
                        float v[32];
#pragma unroll
                        for (int c = 0; c < 4; ++c)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                v[8 * c + 2 * i] = __uint_as_float((uint32_t)b.xr[u][t][c][i] << 16);
                                v[8 * c + 2 * i + 1] = __uint_as_float((uint32_t)b.xr[u][t][c][i] & 0xffff0000u);
                            }
                        // the quad of lanes 4 lr .. 4 lr + 3 holds token lr's
                        // group: amax as an unsigned max of the bf16 magnitude
                        // bits (exact; a NaN's exceed infinity's), over the
                        // quad by two DPP quad permutations
                        uint32_t mx = 0;
#pragma unroll
                        for (int c = 0; c < 4; ++c)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const uint32_t d = (uint32_t)b.xr[u][t][c][i] & 0x7fff7fffu;
                                mx = max(mx, max(d & 0xffffu, d >> 16));
                            }
                        mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0xb1, 0xf, 0xf, false));
                        mx = max(mx, (uint32_t)__builtin_amdgcn_mov_dpp((int)mx, 0x4e, 0xf, 0xf, false));
                        const bool nan = mx > 0x7f80u;
                        const float sc = nan ? __builtin_nanf("") : fmaxf(__uint_as_float(mx << 16), a.eps) / 448.0f;
                        const float rcp = 1.0f / sc;
                        i32x8 o;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            int d = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * i] * rcp, v[4 * i + 1] * rcp, 0, false);
                            d = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * i + 2] * rcp, v[4 * i + 3] * rcp, d, true);
                            o[i] = d;
                        }
                        // codes and scale in the loading layout (gathered
                        // into the MFMA layout with the weights)
                        b.tv[u][t] = o;
                        b.sa[u][t] = sc;
                        const int m = t0 + 16 * t + lr;
                        if (qa_write && m < a.M) {
                            uint8_t* qd = a.q_out + (size_t)m * a.K + (size_t)g * kGroupK + 16 * lc;
                            *(i32x4*)qd = (i32x4){o[0], o[1], o[2], o[3]};
                            *(i32x4*)(qd + 64) = (i32x4){o[4], o[5], o[6], o[7]};
                            if (lc == 0) a.s_out[m * a.qs_sm + g * a.qs_sk] = sc;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (j0 + u < J) {
                const float sb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.sbr), u));
                const float sb2 =
                    kTwoBs ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.sbr2), u)) : sb;
                i32x8 tv[NTB];
                float sa[NTB];
#pragma unroll
                for (int t = 0; t < NTB; ++t) {
                    if constexpr (QF) {
                        tv[t] = b.tv[u][t];
                        sa[t] = b.sa[u][t];
                    } else if constexpr (QA) {
                        const i32x8 o = b.tv[u][t];
                        tv[t] = gather({(i32x4){o[0], o[1], o[2], o[3]}, (i32x4){o[4], o[5], o[6], o[7]}});
                        sa[t] = __int_as_float(__builtin_amdgcn_ds_bpermute(op_src, __float_as_int(b.sa[u][t])));
                    } else {
                        const int src = as_cm ? r + 16 * u : 4 * r + u;
                        if constexpr (DT) {
                            // one token: slot u of row 0 sits in lane 16 u
                            // (column-major As) or u
                            tv[t] = (i32x8){b.tl[u][t][0][0], b.tl[u][t][0][1], b.tl[u][t][0][2],
                                            b.tl[u][t][0][3], b.tl[u][t][1][0], b.tl[u][t][1][1],
                                            b.tl[u][t][1][2], b.tl[u][t][1][3]};
                            sa[t] = a.M == 1 ? __int_as_float(__builtin_amdgcn_readlane(
                                                   __float_as_int(b.sar[t]), as_cm ? 16 * u : u))
                                             : __int_as_float(__builtin_amdgcn_ds_bpermute(
                                                   src << 2, __float_as_int(b.sar[t])));
                        } else {
                            tv[t] = FT ? gather_few(b.tl[u][t][0]) : gather(b.tl[u][t]);
                            sa[t] = __int_as_float(
                                __builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(b.sar[t])));
                        }
                    }
                }
#pragma unroll
                for (int w = 0; w < NWB; ++w) {
                    const i32x8 wv = BSH ? (i32x8){b.wl[u][w][0][0], b.wl[u][w][0][1], b.wl[u][w][0][2],
                                                   b.wl[u][w][0][3], b.wl[u][w][1][0], b.wl[u][w][1][1],
                                                   b.wl[u][w][1][2], b.wl[u][w][1][3]}
                                         : gather(b.wl[u][w]);
                    // (wave-uniform: the block of this 16-row block's rows)
                    const float sbw = kTwoBs && ((w0 + 16 * w) >> 7) != (w0 >> 7) ? sb2 : sb;
#pragma unroll
                    for (int t = 0; t < NTB; ++t) promote(acc[w][t], mfma16x16x128(wv, tv[t]), sa[t] * sbw);
                }
            }
        }
    };
    // operand VGPRs of one batch: weights, tokens (and their bf16 source);
    // two batches and the accumulators must leave room for the rest
    // (16 waves per workgroup leave 128 VGPRs per wave, fewer waves 256;
    // the 48-row tiles' second Bs scale takes more: 48x64 spills at 160)
    constexpr int kBatchRegs = U * (NWB + NTB + (QF ? 1 : QA ? 2 * NTB : 0)) * 8;
    constexpr bool kPipe = 2 * kBatchRegs + 4 * NWB * NTB <= (S >= 16 ? 72 : kTwoBs ? 150 : 160);
    if (J > 0) {
        if constexpr (kPipe) {
            // batches alternate between b0 and b1; the wave's last batch is
            // computed on an early exit, so no load sits under a branch
            Batch b0, b1;
            load(b0, 0);
            for (int j0 = 0;; j0 += 2 * U) {
                if (j0 + U >= J) {
                    compute(b0, j0);
                    break;
                }
                load(b1, j0 + U);
                compute(b0, j0);
                if (j0 + 2 * U >= J) {
                    compute(b1, j0 + U);
                    break;
                }
                load(b0, j0 + 2 * U);
                compute(b1, j0 + U);
            }
        } else {
            for (int j0 = 0; j0 < J; j0 += U) {
                Batch b;
                load(b, j0);
                compute(b, j0);
            }
        }
    }

    // FP8BG_SPLIT_LAST partials: block b of split sidx of tile, one f32x4 per
    // lane (byte offsets below 2^31: the host checks the plan)
    [[maybe_unused]] const __amdgpu_buffer_rsrc_t ws_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.ws, (short)0, 0x7fffffff, kBufferFlags);
    [[maybe_unused]] auto last_off = [&](int tl_, int sp, int b) -> uint32_t {
        return (uint32_t)((((tl_ * a.split + sp) * NB + b) * 64 + lane) * 16);
    };

    // Fixed-order sum of the S wave partials through LDS.
#pragma unroll
    for (int w = 0; w < NWB; ++w)
#pragma unroll
        for (int t = 0; t < NTB; ++t) red[wave][w * NTB + t][lane] = acc[w][t];
    __syncthreads();
    for (int b = wave; b < NB; b += S) {
        f32x4 s = red[0][b][lane];
#pragma unroll
        for (int k = 1; k < S; ++k) {
            const f32x4 v = red[k][b][lane];
            s[0] += v[0];
            s[1] += v[1];
            s[2] += v[2];
            s[3] += v[3];
        }
        const int w = b / NTB, t = b % NTB;
        const int tl = 16 * t + r, wl = 16 * w + 4 * q;
        if constexpr (LAST) {
            // device-scope store (coherent across the XCDs' L2s): the tile's
            // last workgroup may run on another XCD
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, s), ws_rsrc,
                                                   last_off(tile, sidx, b), 0, kDeviceScope);
        } else if (a.split > 1) {
            float* mine = a.ws + ((size_t)tile * a.split + sidx) * (size_t)(TW * TT);
            *(f32x4*)(mine + tl * TW + wl) = s;
        } else {
            const int m = t0 + tl, n = w0 + wl;
            if (m < a.M && n < a.N) *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(s, a.bias, n);
        }
    }
    if constexpr (LAST) {
        // The tile's partials are summed by the workgroup that completes its
        // count (the reference's last-arriver reduction, kernels/
        // baseline_gluon.py:194-209): every workgroup's partial stores have
        // completed (vmcnt 0, at device scope) before its count, so the last
        // one's device-scope loads, issued after its count returned, see them
        // all.  Device-scope stores and loads instead of release / acquire
        // fences: on this chip an agent-scope fence writes back or
        // invalidates the XCD's whole L2.  The sum runs
        // in split order, as fp8bg_split_reduce's; the counter is left at
        // zero for the next call (and for hipGraph replays).  The flag lives
        // in red[], whose reads all precede the barrier below.
        int* is_last = (int*)&red[0][0][0];
        asm volatile("" ::: "memory");
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            *is_last = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (uint32_t)(a.split - 1);
        __syncthreads();
        if (!*is_last) return;
        for (int b = wave; b < NB; b += S) {
            f32x4 s = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, last_off(tile, 0, b), 0, kDeviceScope));
            for (int k = 1; k < a.split; ++k) {
                const f32x4 v = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, last_off(tile, k, b), 0, kDeviceScope));
                s[0] += v[0];
                s[1] += v[1];
                s[2] += v[2];
                s[3] += v[3];
            }
            const int w = b / NTB, t = b % NTB;
            const int m = t0 + 16 * t + r, n = w0 + 16 * w + 4 * q;
            if (m < a.M && n < a.N) *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(s, a.bias, n);
        }
        if (threadIdx.x == 0) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

#if FP8BG_HOST_PART
// ===========================================================================
// Split-K reduction: one workgroup per split tile, fixed split order.
// ===========================================================================
// `parts` workgroups share one split tile, each taking every parts-th run of
// kThreads * 4 elements, so a small tail of split tiles still spreads over
// the whole GPU.
__global__ __launch_bounds__(kThreads) void fp8bg_split_reduce(KArgs a, int skinny_order, int parts) {
    const int stile = blockIdx.x / parts, part = blockIdx.x % parts;
    int w0, t0;
    if (skinny_order) {
        w0 = (stile / a.tiles_t) * a.tw;
        t0 = (stile % a.tiles_t) * a.tt;
    } else {
        tile_origin(a.n_dp + stile, a, w0, t0);
    }
    const int tile_el = a.tw * a.tt;
    const float* base = a.ws + (size_t)stile * a.split * tile_el;
    for (int e = (part * kThreads + threadIdx.x) * 4; e < tile_el; e += parts * kThreads * 4) {
        const int tl = e / a.tw, wl = e % a.tw;
        const int m = t0 + tl, n = w0 + wl;
        if (m >= a.M || n >= a.N) continue;
        f32x4 s = *(const f32x4*)(base + e);
        for (int k = 1; k < a.split; ++k) {
            const f32x4 v = *(const f32x4*)(base + (size_t)k * tile_el + e);
            s[0] += v[0];
            s[1] += v[1];
            s[2] += v[2];
            s[3] += v[3];
        }
        *(uint2*)(a.C + (size_t)m * a.N + n) = out_bf16x4(s, a.bias, n);
    }
}

// ===========================================================================
// Per-token-group activation quantisation (bf16 -> e4m3 + fp32 scale)
// ===========================================================================
// fp32 -> OCP e4m3 ("fn") code, round to nearest even, matching torch's
// float -> float8_e4m3fn cast: NaN and |x| >= 480 (which would round past the
// largest finite 448) give 0x7f with the sign; subnormals are multiples of
// 2^-9.  Pure integer/float arithmetic, identical on host and device.
__host__ __device__ inline uint32_t e4m3_from_f32(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 24) & 0x80u;
    u &= 0x7fffffffu;
    if (u >= 0x43f00000u) return sign | 0x7fu;          // NaN, inf, |x| >= 480
    if (u < 0x3c800000u) {                               // |x| < 2^-6: subnormal grid
        float a;
        __builtin_memcpy(&a, &u, 4);
        return sign | (uint32_t)__builtin_rintf(a * 512.0f);   // 0 .. 8 (8 = 2^-6)
    }
    const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);  // RNE to 3 mantissa bits
    return sign | ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
}

// Row-major e4m3 B [N, K] (row stride ldb bytes) -> the shuffled layout
// (kShufBlock): thread c of the grid-stride loop writes the 16 bytes at
// 16 c, so the stores are contiguous; each reads 16 bytes of one row.
__global__ __launch_bounds__(kThreads) void fp8bg_shuffle_b_kernel(const uint8_t* b, int64_t ldb,
                                                                   uint8_t* bt, int64_t chunks, int kg) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks; c += stride) {
        const int64_t blk = c >> 7;                      // 128 chunks per block
        const int in = (int)(c & 127), h = in >> 6, l = in & 63;
        const int64_t nb = blk / kg, g = blk - nb * kg;
        const int64_t row = 16 * nb + (l & 15);
        const int64_t col = 128 * g + 64 * h + 16 * (l >> 4);
        *(i32x4*)(bt + 16 * c) = *(const i32x4*)(b + row * ldb + col);
    }
}

struct QArgs {
    const uint16_t* x;     // bf16 [M, K], row stride ldx elements
    uint8_t* q;            // e4m3 [M, K], row stride K
    float* s;              // fp32 [M, K/128], strides s_sm, s_sk
    int64_t ldx, s_sm, s_sk;
    int M, K;
    float eps;
    float eps_s, eps_r;    // eps / 448 and 1 / (eps / 448), IEEE fp32 on the host
};

// v / s for a bf16 value v and a scale s >= 2^-60 (or +inf), given
// r = RN(1 / s): the product corrected by one FMA of its exact remainder.
// It equals the IEEE quotient for every bf16 mantissa against every fp32
// scale mantissa (tests/divscale_check.c, all 2^31 pairs of one binade
// each).  Powers of two scale every step exactly wherever the quotient can
// round to a nonzero e4m3 code (|v / s| >= 2^-11 with s >= 2^-60 keeps v,
// the product and the remainder's granularity in the normal range); smaller
// quotients give a signed zero code either way.  An infinite s takes v * 0
// (+-0, or NaN for an infinite v, as the division gives), and the sign is
// v's (-0 / s is -0).
__device__ __forceinline__ float div_by_scale(float v, float s, float r) {
#pragma clang fp contract(off)
    const float q0 = v * r;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, s, v), r, q0);
    return s == __builtin_inff() ? q0 : __builtin_copysignf(q1, v);
}

// 16 lanes per 128-element group, 8 elements (16 bytes) per lane.
__global__ __launch_bounds__(kThreads) void fp8bg_quant_act_kernel(QArgs a) {
    const int kg = a.K / kGroupK;
    const int64_t group = (int64_t)blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    if (group >= (int64_t)a.M * kg) return;              // whole 16-lane groups exit together
    const int m = (int)(group / kg), g = (int)(group % kg);
    const int col = g * kGroupK + sub * 8;
    const i32x4 raw = *(const i32x4*)(a.x + m * a.ldx + col);
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float((uint32_t)raw[i] << 16);
        v[2 * i + 1] = __uint_as_float((uint32_t)raw[i] & 0xffff0000u);
    }
    // amax as an unsigned max of the bf16 magnitude bits over the group's 16
    // lanes (exact; a NaN's bits exceed infinity's, so a NaN anywhere makes
    // the group's scale NaN, as max/clamp do in the reference recipe)
    uint32_t mx = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = (uint32_t)raw[i] & 0x7fff7fffu;
        mx = max(mx, max(d & 0xffffu, d >> 16));
    }
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, d, 16));
    const bool nan = mx > 0x7f80u, inf = mx == 0x7f80u;
    const float amax = __uint_as_float(mx << 16);
    // The scale and its reciprocal without a division (the bf16 amax's exact
    // pair, eps's pair from the host, (inf, 0) for an infinite amax), and
    // each value's quotient without one, where every lane's scale is at
    // least 2^-60 (NaN fails the compare); otherwise the divisions.
    float sf, rf;
    act_scale_reciprocal_fast(amax, sf, rf);
    const bool above = amax >= a.eps;
    const float scale_f = nan ? __builtin_nanf("") : inf ? amax : above ? sf : a.eps_s;
    float scale;
    uint2 o;
    if (__builtin_amdgcn_ballot_w64(!(scale_f >= 0x1p-60f)) == 0) {
        scale = scale_f;
        const float rs = inf ? 0.0f : above ? rf : a.eps_r;
        float qv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[i] = div_by_scale(v[i], scale, rs);
        o.x = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
            qv[2], qv[3], __builtin_amdgcn_cvt_pk_fp8_f32(qv[0], qv[1], 0, false), true);
        o.y = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(
            qv[6], qv[7], __builtin_amdgcn_cvt_pk_fp8_f32(qv[4], qv[5], 0, false), true);
    } else {
        scale = nan ? __builtin_nanf("") : fmaxf(amax, a.eps) / 448.0f;
        o.x = e4m3_from_f32(v[0] / scale) | (e4m3_from_f32(v[1] / scale) << 8) |
              (e4m3_from_f32(v[2] / scale) << 16) | (e4m3_from_f32(v[3] / scale) << 24);
        o.y = e4m3_from_f32(v[4] / scale) | (e4m3_from_f32(v[5] / scale) << 8) |
              (e4m3_from_f32(v[6] / scale) << 16) | (e4m3_from_f32(v[7] / scale) << 24);
    }
    *(uint2*)(a.q + (int64_t)m * a.K + col) = o;
    if (sub == 0) a.s[m * a.s_sm + g * a.s_sk] = scale;
}

// fp32 -> e4m3 with the instruction the quantisers use (v_cvt_pk_fp8_f32),
// two values per lane, grid-stride (fp8bg_e4m3_encode_device).
__global__ __launch_bounds__(kThreads) void fp8bg_e4m3_cvt_kernel(const float* x, uint8_t* out, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * p < n; p += stride) {
        const int64_t i = 2 * p;
        const bool pair = i + 1 < n;
        const uint32_t d = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x[i], pair ? x[i + 1] : 0.0f, 0, false);
        out[i] = (uint8_t)d;
        if (pair) out[i + 1] = (uint8_t)(d >> 8);
    }
}

#endif  // FP8BG_HOST_PART

// ---------------------------------------------------------------------------
// Compiled instances
// ---------------------------------------------------------------------------
// tiled: (block_w, block_t, waves_w, waves_t, k_fixed)
#define FP8BG_TILED(X)                                                         \
    X(64, 16, 4, 1, 0) X(128, 16, 4, 1, 0) X(256, 16, 4, 1, 0)                 \
    X(64, 32, 4, 1, 0) X(128, 32, 4, 1, 0) X(256, 32, 4, 1, 0)                 \
    X(64, 64, 4, 1, 0) X(128, 64, 4, 1, 0) X(256, 64, 4, 1, 0)                 \
    X(128, 64, 2, 2, 0) X(128, 128, 2, 2, 0) X(128, 128, 4, 1, 0)              \
    X(256, 128, 4, 1, 0) X(256, 128, 2, 2, 0) X(128, 256, 2, 2, 0)             \
    X(64, 16, 4, 1, 2) X(128, 16, 4, 1, 2) X(64, 32, 4, 1, 2)                  \
    X(128, 32, 4, 1, 2) X(128, 64, 4, 1, 2) X(128, 128, 2, 2, 2)               \
    X(256, 128, 4, 1, 2)

// skinny: (weight 16-blocks, token 16-blocks, waves splitting K, groups in flight)
// (the 48-row tiles: N = 12288 in 256 of them, one per CU)
#define FP8BG_SKINNY(X)                                                        \
    X(1, 1, 4, 1) X(1, 1, 4, 2) X(1, 1, 8, 1) X(1, 1, 8, 2) X(1, 1, 8, 4)      \
    X(2, 1, 4, 1) X(2, 1, 4, 2) X(2, 1, 8, 1) X(2, 1, 8, 2) X(2, 1, 8, 4)      \
    X(4, 1, 4, 1) X(4, 1, 4, 2) X(4, 1, 8, 1) X(4, 1, 8, 2) X(4, 1, 8, 4)      \
    X(1, 2, 4, 2) X(1, 2, 8, 1) X(1, 2, 8, 2)                                  \
    X(2, 2, 4, 2) X(2, 2, 8, 1) X(2, 2, 8, 2)                                  \
    X(4, 2, 4, 2) X(4, 2, 8, 1) X(4, 2, 8, 2)                                  \
    X(1, 4, 4, 2) X(1, 4, 8, 1) X(1, 4, 8, 2)                                  \
    X(2, 4, 4, 2) X(2, 4, 8, 1) X(2, 4, 8, 2)                                  \
    X(4, 4, 4, 1) X(4, 4, 8, 1) X(4, 4, 4, 2)                                  \
    X(1, 1, 4, 4) X(2, 1, 4, 4) X(4, 1, 4, 4)                                  \
    X(1, 1, 16, 1) X(1, 1, 16, 2) X(2, 1, 16, 1) X(2, 1, 16, 2) X(4, 1, 16, 1) \
    X(1, 2, 16, 1) X(2, 2, 16, 1) X(1, 4, 16, 1)                               \
    X(3, 1, 4, 1) X(3, 1, 4, 2) X(3, 1, 8, 1) X(3, 1, 8, 2)                    \
    X(3, 2, 4, 2) X(3, 2, 8, 1) X(3, 2, 8, 2)                                  \
    X(3, 4, 4, 1) X(3, 4, 8, 1) X(3, 4, 4, 2)                                  \
    X(3, 1, 16, 1) X(3, 2, 16, 1)                                              \
    X(1, 1, 2, 1) X(2, 1, 2, 1)

// ring: (block_w, block_t, waves_w, waves_t, stages, k_fixed, groups per barrier,
//        K slices)
#define FP8BG_RING_A(X) \
    X(256, 128, 4, 1, 3, 0, 1, 1) X(256, 128, 2, 2, 3, 0, 1, 1) \
    X(128, 128, 2, 2, 4, 0, 1, 1) X(128, 128, 4, 1, 4, 0, 1, 1) \
    X(128, 128, 2, 2, 3, 0, 1, 1) X(128, 64, 2, 2, 4, 0, 1, 1) \
    X(128, 64, 4, 1, 4, 0, 1, 1) X(128, 64, 2, 2, 3, 0, 1, 1) \
    X(64, 64, 4, 1, 4, 0, 1, 1) X(256, 64, 4, 1, 3, 0, 1, 1) \
    X(128, 32, 4, 1, 4, 0, 1, 1) X(256, 256, 4, 2, 2, 0, 1, 1) \
    X(256, 128, 4, 2, 3, 0, 1, 1) X(256, 128, 4, 2, 2, 0, 1, 1) \
    X(128, 256, 2, 4, 2, 0, 1, 1) X(256, 128, 4, 1, 2, 2, 1, 1) \
    X(128, 128, 2, 2, 2, 2, 1, 1) X(64, 64, 4, 1, 8, 0, 1, 1) \
    X(128, 64, 4, 1, 6, 0, 1, 1) X(128, 32, 4, 1, 7, 0, 1, 1) \
    X(128, 128, 2, 2, 2, 0, 1, 1) X(192, 256, 3, 4, 2, 0, 1, 1) \
    X(192, 128, 6, 2, 2, 0, 1, 1) X(192, 128, 6, 2, 3, 0, 1, 1) \
    X(192, 128, 3, 4, 3, 0, 1, 1)

#define FP8BG_RING_B(X) \
    X(192, 64, 6, 2, 4, 0, 1, 1) X(64, 64, 4, 1, 4, 0, 2, 1) \
    X(64, 64, 4, 1, 8, 0, 2, 1) X(64, 64, 4, 1, 8, 0, 4, 1) \
    X(128, 64, 4, 1, 4, 0, 2, 1) X(128, 64, 4, 1, 6, 0, 2, 1) \
    X(128, 32, 4, 1, 4, 0, 2, 1) X(128, 32, 4, 1, 7, 0, 2, 1) \
    X(128, 64, 2, 2, 4, 0, 2, 1) X(192, 64, 6, 2, 4, 0, 2, 1) \
    X(64, 64, 4, 1, 4, 0, 2, 2) X(64, 64, 4, 1, 8, 0, 2, 2) \
    X(64, 64, 4, 1, 8, 0, 4, 2) X(64, 64, 4, 1, 8, 0, 4, 4) \
    X(128, 64, 4, 1, 6, 0, 2, 2) X(128, 32, 4, 1, 4, 0, 2, 2) \
    X(128, 128, 4, 2, 2, 0, 1, 1) X(128, 128, 4, 2, 3, 0, 1, 1) \
    X(128, 128, 4, 2, 4, 0, 2, 1) X(256, 160, 4, 2, 2, 0, 1, 1) \
    X(256, 192, 4, 2, 2, 0, 1, 1) X(128, 160, 2, 2, 3, 0, 1, 1) \
    X(128, 96, 2, 2, 4, 0, 1, 1) X(64, 64, 2, 2, 8, 0, 4, 1)                   \
    X(96, 64, 3, 1, 4, 0, 2, 1) X(96, 128, 3, 2, 3, 0, 1, 1)
#define FP8BG_RING(X) FP8BG_RING_A(X) FP8BG_RING_B(X)

// skinny with the fused activation quantiser: the 16-, 32- and 64-token
// tiles ((4, 1, 8, 4), (4, 1, 4, 4), (4, 1, 16, 1), (2, 4, 8, 2), (1, 4, 16, 1)
// and the 4 x 4 tiles left out: with the bf16 staging they need more VGPRs
// than their wave count leaves)
#define FP8BG_SKINNY_QA(X)                                                     \
    X(1, 1, 4, 1) X(1, 1, 4, 2) X(1, 1, 8, 1) X(1, 1, 8, 2) X(1, 1, 8, 4)      \
    X(2, 1, 4, 1) X(2, 1, 4, 2) X(2, 1, 8, 1) X(2, 1, 8, 2) X(2, 1, 8, 4)      \
    X(4, 1, 4, 1) X(4, 1, 4, 2) X(4, 1, 8, 1) X(4, 1, 8, 2)                    \
    X(1, 2, 4, 2) X(1, 2, 8, 1) X(1, 2, 8, 2)                                  \
    X(2, 2, 4, 2) X(2, 2, 8, 1) X(2, 2, 8, 2)                                  \
    X(4, 2, 4, 2) X(4, 2, 8, 1) X(4, 2, 8, 2)                                  \
    X(1, 4, 4, 2) X(1, 4, 8, 1) X(1, 4, 8, 2)                                  \
    X(2, 4, 4, 2) X(2, 4, 8, 1)                                                \
    X(1, 1, 4, 4) X(2, 1, 4, 4)                                                \
    X(1, 1, 16, 1) X(1, 1, 16, 2) X(2, 1, 16, 1) X(2, 1, 16, 2)                \
    X(1, 2, 16, 1) X(2, 2, 16, 1)                                              \
    X(3, 1, 4, 1) X(3, 1, 4, 2) X(3, 1, 8, 1) X(3, 1, 8, 2)                    \
    X(3, 2, 4, 2) X(3, 2, 8, 1) X(3, 2, 8, 2) X(3, 1, 16, 1)                   \
    X(1, 1, 2, 1) X(2, 1, 2, 1)

// Launchers, one per compiled instance and B layout; the skinny and ring
// ones pick the kernel variant at run time.  The arguments travel by pointer
// so that a launcher compiled in another part of the build (external
// functions of plain types, below) can fill the table of part 1.
typedef void (*LaunchFn)(dim3 grid, size_t shm, hipStream_t s, const void* a);
struct Instance {
    int kind, tw, tt, ww, wt, wk, unroll, stages, kf, threads;
    LaunchFn launch;       // row-major B
    LaunchFn launch_bs;    // shuffled B (FP8BG_FLAG_B_SHUFFLED); null: not supported
};

template <int TW, int TT, int WW, int WT, int KF>
void tiled_launch(dim3 g, size_t shm, hipStream_t s, const void* a) {
    hipLaunchKernelGGL((fp8bg_tiled<TW, TT, WW, WT, KF>), g, dim3(kThreads), shm, s, *(const KArgs*)a);
}

// BM: the B-layout MODE bit (0 or kSkinnyBShuf).
// (launches with at most 8 tokens on 16-token tiles of 16 or 32 weight rows
// take the few-token load; on 64-row tiles it measured 15% slower cold at
// (12288, 2048) M = 4 and 8, and 1-3% faster on the others)
template <int NW, int NT, int S, int U, int BM>
void skinny_launch(dim3 g, size_t shm, hipStream_t s, const void* av) {
    const KArgs& a = *(const KArgs*)av;
    constexpr int kFewTok = NT == 1 && NW <= 2 ? kSkinnyFewTokens : 0;
    constexpr int kDirectTok = NT == 1 ? kSkinnyDirectTokens : 0;
    // direct token loads at M <= 2 with row-major B, where the tokens' and
    // the weights' ds_bpermute bound the call (7-15% faster warm at M = 1 and
    // 2 on the larger decode shapes, within 3% cold); at M = 4 their extra L1
    // accesses already cost as much as they save, and with a shuffled B
    // (no weight gather left) at any M
    constexpr int kDirectTokensMax = BM == kSkinnyBShuf ? 0 : 2;
    if (a.split_last)
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, BM | kSkinnyLast>), g, dim3(64 * S), shm, s, a);
    else if (kDirectTok && a.M <= kDirectTokensMax)
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, BM | kDirectTok>), g, dim3(64 * S), shm, s, a);
    else if (kFewTok && a.M <= 8)
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, BM | kFewTok>), g, dim3(64 * S), shm, s, a);
    else
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, BM>), g, dim3(64 * S), shm, s, a);
}

// (launches with at most 4 tokens on 16-token tiles take the few-token
// quantiser: same codes and scales, a fraction of the per-value work)
template <int NW, int NT, int S, int U, int BM>
void skinny_qa_launch(dim3 g, size_t shm, hipStream_t s, const void* av) {
    const KArgs& a = *(const KArgs*)av;
    constexpr int kQ = BM | kSkinnyQuant;
    if constexpr (NT == 1) {
        if (a.M <= 4) {
            if (a.split_last)
                hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, kQ | kSkinnyQuantFew | kSkinnyLast>), g,
                                   dim3(64 * S), shm, s, a);
            else
                hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, kQ | kSkinnyQuantFew>), g, dim3(64 * S),
                                   shm, s, a);
            return;
        }
    }
    if (a.split_last)
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, kQ | kSkinnyLast>), g, dim3(64 * S), shm, s, a);
    else
        hipLaunchKernelGGL((fp8bg_skinny<NW, NT, S, U, kQ>), g, dim3(64 * S), shm, s, a);
}

template <int TW, int TT, int WW, int WT, int ST, int KF, int KU, int WK, bool BSH>
void ring_launch(dim3 g, size_t shm, hipStream_t s, const void* av) {
    const KArgs& a = *(const KArgs*)av;
    const dim3 block(64 * WW * WT * WK);
    if constexpr (ring_has_sk(TW, TT, WW, WT, KF, WK)) {
        if (a.stream) {
            if constexpr (BSH)
                hipLaunchKernelGGL((fp8bg_ring_sk_bs<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            else
                hipLaunchKernelGGL((fp8bg_ring_sk<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            return;
        }
    }
    if constexpr (ring_has_last(TT, KF)) {
        if (a.split_last) {
            if constexpr (BSH)
                hipLaunchKernelGGL((fp8bg_ring_last_bs<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            else
                hipLaunchKernelGGL((fp8bg_ring_last<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            return;
        }
    }
    if constexpr (ring_has_dp(TW, TT, KF, KU, WK)) {
        if (a.n_dp == (int)g.x && a.kcount > KU) {
            if constexpr (BSH)
                hipLaunchKernelGGL((fp8bg_ring_dp_bs<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            else
                hipLaunchKernelGGL((fp8bg_ring_dp<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
            return;
        }
    }
    if constexpr (BSH)
        hipLaunchKernelGGL((fp8bg_ring_bs<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
    else
        hipLaunchKernelGGL((fp8bg_ring<TW, TT, WW, WT, ST, KF, KU, WK>), g, block, shm, s, a);
}

}  // namespace

// The launchers' external names (L: rm = row-major B, bs = shuffled B), and
// for each part either their definitions (the part that compiles them, or
// all in part 0) or their declarations (part 1, whose table takes them).
#define FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, L) \
    fp8bg_ring_##L##_##TW##_##TT##_##WW##_##WT##_##ST##_##KF##_##KU##_##WK
#define FP8BG_SKINNY_FN(NW, NT, S, U, L) fp8bg_skinny_##L##_##NW##_##NT##_##S##_##U
#define FP8BG_SKINNY_QA_FN(NW, NT, S, U, L) fp8bg_skinny_qa_##L##_##NW##_##NT##_##S##_##U
#define FP8BG_LAUNCH_ARGS dim3 g, size_t shm, hipStream_t s, const void* a
// (linked across the parts, not exported from the library)
#define FP8BG_LAUNCHER __attribute__((visibility("hidden"))) void

#define FP8BG_RING_DEF_RM(TW, TT, WW, WT, ST, KF, KU, WK)                            \
    FP8BG_LAUNCHER FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, rm)(FP8BG_LAUNCH_ARGS) {      \
        ring_launch<TW, TT, WW, WT, ST, KF, KU, WK, false>(g, shm, s, a);            \
    }
#define FP8BG_RING_DEF_BS(TW, TT, WW, WT, ST, KF, KU, WK)                            \
    FP8BG_LAUNCHER FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, bs)(FP8BG_LAUNCH_ARGS) {      \
        ring_launch<TW, TT, WW, WT, ST, KF, KU, WK, true>(g, shm, s, a);             \
    }
#define FP8BG_RING_DECL_RM(TW, TT, WW, WT, ST, KF, KU, WK) \
    FP8BG_LAUNCHER FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, rm)(FP8BG_LAUNCH_ARGS);
#define FP8BG_RING_DECL_BS(TW, TT, WW, WT, ST, KF, KU, WK) \
    FP8BG_LAUNCHER FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, bs)(FP8BG_LAUNCH_ARGS);
#define FP8BG_SKINNY_DEF_RM(NW, NT, S, U) \
    FP8BG_LAUNCHER FP8BG_SKINNY_FN(NW, NT, S, U, rm)(FP8BG_LAUNCH_ARGS) { skinny_launch<NW, NT, S, U, 0>(g, shm, s, a); }
#define FP8BG_SKINNY_DEF_BS(NW, NT, S, U)                                              \
    FP8BG_LAUNCHER FP8BG_SKINNY_FN(NW, NT, S, U, bs)(FP8BG_LAUNCH_ARGS) {                        \
        skinny_launch<NW, NT, S, U, kSkinnyBShuf>(g, shm, s, a);                       \
    }
#define FP8BG_SKINNY_DECL_RM(NW, NT, S, U) FP8BG_LAUNCHER FP8BG_SKINNY_FN(NW, NT, S, U, rm)(FP8BG_LAUNCH_ARGS);
#define FP8BG_SKINNY_DECL_BS(NW, NT, S, U) FP8BG_LAUNCHER FP8BG_SKINNY_FN(NW, NT, S, U, bs)(FP8BG_LAUNCH_ARGS);
#define FP8BG_SKINNY_QA_DEF_RM(NW, NT, S, U)                                           \
    FP8BG_LAUNCHER FP8BG_SKINNY_QA_FN(NW, NT, S, U, rm)(FP8BG_LAUNCH_ARGS) {                     \
        skinny_qa_launch<NW, NT, S, U, 0>(g, shm, s, a);                               \
    }
#define FP8BG_SKINNY_QA_DEF_BS(NW, NT, S, U)                                           \
    FP8BG_LAUNCHER FP8BG_SKINNY_QA_FN(NW, NT, S, U, bs)(FP8BG_LAUNCH_ARGS) {                     \
        skinny_qa_launch<NW, NT, S, U, kSkinnyBShuf>(g, shm, s, a);                    \
    }
#define FP8BG_SKINNY_QA_DECL_RM(NW, NT, S, U) FP8BG_LAUNCHER FP8BG_SKINNY_QA_FN(NW, NT, S, U, rm)(FP8BG_LAUNCH_ARGS);
#define FP8BG_SKINNY_QA_DECL_BS(NW, NT, S, U) FP8BG_LAUNCHER FP8BG_SKINNY_QA_FN(NW, NT, S, U, bs)(FP8BG_LAUNCH_ARGS);

#if FP8BG_PART == 0 || FP8BG_PART == 2
FP8BG_RING_A(FP8BG_RING_DEF_RM)
#elif FP8BG_PART == 1
FP8BG_RING_A(FP8BG_RING_DECL_RM)
#endif
#if FP8BG_PART == 0 || FP8BG_PART == 3
FP8BG_RING_A(FP8BG_RING_DEF_BS)
#elif FP8BG_PART == 1
FP8BG_RING_A(FP8BG_RING_DECL_BS)
#endif
#if FP8BG_PART == 0 || FP8BG_PART == 4
FP8BG_RING_B(FP8BG_RING_DEF_RM)
#elif FP8BG_PART == 1
FP8BG_RING_B(FP8BG_RING_DECL_RM)
#endif
#if FP8BG_PART == 0 || FP8BG_PART == 5
FP8BG_RING_B(FP8BG_RING_DEF_BS)
#elif FP8BG_PART == 1
FP8BG_RING_B(FP8BG_RING_DECL_BS)
#endif
#if FP8BG_PART == 0 || FP8BG_PART == 6
FP8BG_SKINNY(FP8BG_SKINNY_DEF_RM)
FP8BG_SKINNY_QA(FP8BG_SKINNY_QA_DEF_RM)
#elif FP8BG_PART == 1
FP8BG_SKINNY(FP8BG_SKINNY_DECL_RM)
FP8BG_SKINNY_QA(FP8BG_SKINNY_QA_DECL_RM)
#endif
#if FP8BG_PART == 0 || FP8BG_PART == 7
FP8BG_SKINNY(FP8BG_SKINNY_DEF_BS)
FP8BG_SKINNY_QA(FP8BG_SKINNY_QA_DEF_BS)
#elif FP8BG_PART == 1
FP8BG_SKINNY(FP8BG_SKINNY_DECL_BS)
FP8BG_SKINNY_QA(FP8BG_SKINNY_QA_DECL_BS)
#endif

// Everything below is part 1 (and part 0): the instance tables, the host
// planning code, the small kernels and the C ABI.
#if FP8BG_HOST_PART
namespace {

#define FP8BG_TILED_ENTRY(TW, TT, WW, WT, KF) \
    {FP8BG_KIND_TILED, TW, TT, WW, WT, 1, 1, 1, KF, kThreads, tiled_launch<TW, TT, WW, WT, KF>, nullptr},
#define FP8BG_SKINNY_ENTRY(NW, NT, S, U)                            \
    {FP8BG_KIND_SKINNY, 16 * NW, 16 * NT, 1, 1, S, U, 1, 0, 64 * S, \
     FP8BG_SKINNY_FN(NW, NT, S, U, rm), FP8BG_SKINNY_FN(NW, NT, S, U, bs)},
#define FP8BG_RING_ENTRY(TW, TT, WW, WT, ST, KF, KU, WK)                        \
    {FP8BG_KIND_RING, TW, TT, WW, WT, WK, KU, ST, KF, 64 * WW * WT * WK,        \
     FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, rm), FP8BG_RING_FN(TW, TT, WW, WT, ST, KF, KU, WK, bs)},
const Instance kInstances[] = {FP8BG_TILED(FP8BG_TILED_ENTRY) FP8BG_SKINNY(FP8BG_SKINNY_ENTRY)
                                   FP8BG_RING(FP8BG_RING_ENTRY)};
#define FP8BG_SKINNY_QA_ENTRY(NW, NT, S, U)                         \
    {FP8BG_KIND_SKINNY, 16 * NW, 16 * NT, 1, 1, S, U, 1, 0, 64 * S, \
     FP8BG_SKINNY_QA_FN(NW, NT, S, U, rm), FP8BG_SKINNY_QA_FN(NW, NT, S, U, bs)},
const Instance kQaInstances[] = {FP8BG_SKINNY_QA(FP8BG_SKINNY_QA_ENTRY)};
#undef FP8BG_TILED_ENTRY
#undef FP8BG_SKINNY_ENTRY
#undef FP8BG_SKINNY_QA_ENTRY
#undef FP8BG_RING_ENTRY
constexpr int kNumInstances = sizeof(kInstances) / sizeof(kInstances[0]);
constexpr int kNumQaInstances = sizeof(kQaInstances) / sizeof(kQaInstances[0]);

// Workgroups per split tile in the reduction: enough for about two per CU,
// at most one per kThreads * 4 elements of the tile.
int reduce_parts(const fp8bg_plan& p, const Instance& k, int num_cus) {
    const int max_parts = max(1, k.tw * k.tt / (kThreads * 4));
    const int want = (2 * num_cus + p.n_split - 1) / p.n_split;
    return max(1, min(want, max_parts));
}

int find_qa_instance(const fp8bg_config* c) {
    for (int i = 0; i < kNumQaInstances; ++i) {
        const Instance& k = kQaInstances[i];
        if (c->kind == FP8BG_KIND_SKINNY && k.tw == c->block_w && k.tt == c->block_t &&
            k.wk == c->waves_k && k.unroll == c->unroll && c->k_fixed == 0)
            return i;
    }
    return -1;
}

int find_instance(const fp8bg_config* c) {
    for (int i = 0; i < kNumInstances; ++i) {
        const Instance& k = kInstances[i];
        if (k.kind != c->kind || k.tw != c->block_w || k.tt != c->block_t) continue;
        if (k.kind == FP8BG_KIND_TILED && k.ww == c->waves_w && k.wt == c->waves_t &&
            k.kf == c->k_fixed)
            return i;
        if (k.kind == FP8BG_KIND_SKINNY && k.wk == c->waves_k && k.unroll == c->unroll &&
            c->k_fixed == 0)
            return i;
        if (k.kind == FP8BG_KIND_RING && k.ww == c->waves_w && k.wt == c->waves_t &&
            k.stages == c->stages && k.kf == c->k_fixed && k.unroll == max(c->unroll, 1) &&
            k.wk == max(c->waves_k, 1))
            return i;
    }
    return -1;
}

}  // namespace

// ===========================================================================
// Calibration kernels (measurement only): the MFMA issue rate and the
// streaming-read and streaming-write rates this chip sustains, next to the
// published peaks.
// ===========================================================================
namespace {

constexpr int kCalibMfmaPerIter = 16;

// Each wave issues kCalibMfmaPerIter FP8 16x16x128 MFMAs per iteration from
// register operands into 4 independent accumulators (so no MFMA waits for
// the previous one's result).  The empty asm statements make the operands
// opaque each iteration, so nothing is hoisted or folded.  With every code
// 0x38 (1.0) each output element of an accumulator grows by 128 per MFMA:
// out = 4 * 128 * (kCalibMfmaPerIter / 4) * iters, exact in fp32 for the
// iteration counts the entry point accepts.
__global__ __launch_bounds__(256) void fp8bg_calib_mfma_kernel(const int32_t* codes, float* out,
                                                               int iters) {
    const int lane = threadIdx.x & 63;
    i32x8 a[2], b[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[0][e] = codes[(0 * 8 + e) * 64 + lane];
        a[1][e] = codes[(1 * 8 + e) * 64 + lane];
        b[0][e] = codes[(2 * 8 + e) * 64 + lane];
        b[1][e] = codes[(3 * 8 + e) * 64 + lane];
    }
    f32x4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
        asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]));
#pragma unroll
        for (int u = 0; u < kCalibMfmaPerIter; ++u)
            acc[u & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                a[u & 1], b[(u >> 1) & 1], acc[u & 3], 0, 0, 0, 0, 0, 0);
    }
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0][0] + acc[1][0] + acc[2][0] + acc[3][0];
}

// The same MFMAs as the GEMM kernels take them: each product starts from a
// zero accumulator and is promoted at once by four FMAs with a scale read
// at run time (1.0), into 8 accumulators; the FMAs of one product follow
// the next MFMA, as in the ring kernel's loop.  out = 2048 * iters as
// above.  Its rate against fp8bg_calib_mfma_kernel's is what the block-scale
// promotion costs the matrix pipe.  A product from a zero accumulator is a
// pure function of its operands, so the empty asm before each MFMA gives
// the compiler a new A operand every time: without it, the 16 MFMAs of an
// iteration fold into the 4 distinct (A, B) pairs.
__global__ __launch_bounds__(256) void fp8bg_calib_promote_kernel(const int32_t* codes,
                                                                  const float* scale, float* out,
                                                                  int iters) {
    const int lane = threadIdx.x & 63;
    i32x8 a[2], b[2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[0][e] = codes[(0 * 8 + e) * 64 + lane];
        a[1][e] = codes[(1 * 8 + e) * 64 + lane];
        b[0][e] = codes[(2 * 8 + e) * 64 + lane];
        b[1][e] = codes[(3 * 8 + e) * 64 + lane];
    }
    float sc = scale[lane];
    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
        asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(b[0]), "+v"(b[1]), "+v"(sc));
#pragma unroll
        for (int u = 0; u < kCalibMfmaPerIter; ++u) {
            asm volatile("" : "+v"(a[u & 1]));
            promote(acc[u & 7], mfma16x16x128(a[u & 1], b[(u >> 1) & 1]), sc);
        }
    }
    float r = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) r += acc[c][0];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = r;
}

// Grid-stride read of n16 16-byte words, four loads in flight per lane,
// XOR-folded; one 32-bit word per thread is written.
__global__ __launch_bounds__(256) void fp8bg_calib_read_kernel(const i32x4* src, int64_t n16,
                                                               uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    i32x4 x = {0, 0, 0, 0};
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const i32x4 v0 = src[i];
        const i32x4 v1 = src[i + stride];
        const i32x4 v2 = src[i + 2 * stride];
        const i32x4 v3 = src[i + 3 * stride];
        x ^= v0 ^ v1 ^ v2 ^ v3;
    }
    for (; i < n16; i += stride) x ^= src[i];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (uint32_t)(x[0] ^ x[1] ^ x[2] ^ x[3]);
}

// An empty kernel: back to back in a hipGraph, its per-launch time is the
// launch floor every call of the path pays.
__global__ void fp8bg_calib_empty_kernel() {}

// Grid-stride write of n16 16-byte words of `value`, four stores in flight
// per lane; NT selects the non-temporal stores that the GEMM kernels use for
// C, whose lines are not read again.
template <bool NT>
__global__ __launch_bounds__(256) void fp8bg_calib_write_kernel(i32x4* dst, int64_t n16, uint32_t value) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const i32x4 v = {(int)value, (int)value, (int)value, (int)value};
    auto put = [&](int64_t j) __attribute__((always_inline)) {
        if constexpr (NT)
            __builtin_nontemporal_store(v, dst + j);
        else
            dst[j] = v;
    };
    for (; i + 3 * stride < n16; i += 4 * stride) {
        put(i);
        put(i + stride);
        put(i + 2 * stride);
        put(i + 3 * stride);
    }
    for (; i < n16; i += stride) put(i);
}

}  // namespace

extern "C" {

int fp8bg_version(void) { return FP8BG_ABI_VERSION; }

const char* fp8bg_strerror(int code) {
    switch (code) {
        case FP8BG_OK: return "ok";
        case FP8BG_ERR_SHAPE: return "invalid shape: need M>=1 and N, K positive multiples of 128";
        case FP8BG_ERR_CONFIG: return "invalid or uncompiled kernel configuration";
        case FP8BG_ERR_WORKSPACE: return "split-K workspace missing or too small";
        case FP8BG_ERR_ALIGN: return "A, B and C must be 16-byte aligned";
        case FP8BG_ERR_LAUNCH: return "HIP kernel launch failed";
        case FP8BG_ERR_DEVICE: return "HIP device query failed";
        case FP8BG_ERR_NULL: return "required pointer argument is NULL";
        case FP8BG_ERR_SCRATCH:
            return "split-K workspace larger than the library scratch (FP8BG_SCRATCH_ELEMS fp32)";
        default: return "unknown fp8bg error";
    }
}

int fp8bg_num_cus(int device, int32_t* num_cus) {
    if (!num_cus) return FP8BG_ERR_NULL;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || v < 1)
        return FP8BG_ERR_DEVICE;
    *num_cus = v;
    return FP8BG_OK;
}

int fp8bg_config_supported(const fp8bg_config* cfg) {
    return cfg != nullptr && find_instance(cfg) >= 0;
}

int fp8bg_make_plan(int32_t M, int32_t N, int32_t K, const fp8bg_config* cfg, int32_t num_cus,
                    fp8bg_plan* plan) {
    if (!cfg || !plan) return FP8BG_ERR_NULL;
    if (M < 1 || N < 128 || K < 128 || N % 128 || K % 128) return FP8BG_ERR_SHAPE;
    const int ki = find_instance(cfg);
    if (ki < 0) return FP8BG_ERR_CONFIG;
    if (cfg->split < 1 || cfg->group_t < 1 || num_cus < 1) return FP8BG_ERR_CONFIG;
    if (cfg->split_mode < FP8BG_SPLIT_NONE || cfg->split_mode > FP8BG_SPLIT_STREAM) return FP8BG_ERR_CONFIG;
    if (cfg->flags & ~(FP8BG_FLAG_SCALE_LDS | FP8BG_FLAG_XCD_REMAP | FP8BG_FLAG_SWZ8 |
                       FP8BG_FLAG_SWZPAIR | FP8BG_FLAG_B_SHUFFLED))
        return FP8BG_ERR_CONFIG;
    if ((cfg->flags & FP8BG_FLAG_SWZ8) && (cfg->flags & FP8BG_FLAG_SWZPAIR)) return FP8BG_ERR_CONFIG;
    const int kg = K / 128;
    const Instance& k = kInstances[ki];
    if (k.kf && kg != k.kf) return FP8BG_ERR_CONFIG;
    if ((cfg->flags & FP8BG_FLAG_B_SHUFFLED) && !k.launch_bs) return FP8BG_ERR_CONFIG;
    const bool skinny = k.kind == FP8BG_KIND_SKINNY;
    const bool ring = k.kind == FP8BG_KIND_RING;
    if ((skinny || ring) && (cfg->flags & FP8BG_FLAG_SCALE_LDS)) return FP8BG_ERR_CONFIG;
    // the ring kernel addresses A and B with 32-bit byte offsets, and 16 rows
    // of C with 31-bit ones
    if (ring && ((int64_t)M * K > 0xffffffffLL || (int64_t)N * K > 0xffffffffLL ||
                 (int64_t)N * 32 > 0x7fffffffLL))
        return FP8BG_ERR_SHAPE;

    const bool stream = cfg->split_mode == FP8BG_SPLIT_STREAM;
    if (stream && !(ring && ring_has_sk(k.tw, k.tt, k.ww, k.wt, k.kf, k.wk))) return FP8BG_ERR_CONFIG;
    int split = (cfg->split_mode == FP8BG_SPLIT_NONE || k.kf || stream) ? 1 : cfg->split;
    if (kg % split) split = 1;  // reference baseline_gluon.py:274-276
    const bool last = cfg->split_mode == FP8BG_SPLIT_LAST;
    if (last && !skinny && !(ring && ring_has_last(k.tt, k.kf))) return FP8BG_ERR_CONFIG;
    if (skinny && split > 1 && cfg->split_mode == FP8BG_SPLIT_TAIL) return FP8BG_ERR_CONFIG;
    const int64_t tiles_w = (N + k.tw - 1) / k.tw;
    const int64_t tiles_t = ((int64_t)M + k.tt - 1) / k.tt;
    const int64_t tiles = tiles_w * tiles_t;
    int64_t n_split = 0;
    if (split > 1) n_split = cfg->split_mode == FP8BG_SPLIT_TAIL ? tiles % num_cus : tiles;
    if (n_split == 0) split = 1;
    // the in-kernel reduction: one counter per split tile (skinny) or per
    // wave of a split tile (ring), partial byte offsets below 2^31; beyond
    // that the split tiles take the two-kernel reduction, which sums the same
    // partials in the same order (bitwise the same C), so a table entry of
    // this mode stays valid at any M
    const bool in_kernel = last && n_split > 0 &&
                           n_split * (ring ? k.ww * k.wt : 1) <= FP8BG_COUNTERS &&
                           n_split * split * (int64_t)k.tw * k.tt * 4 <= 0x7fffffffLL;
    // a ring kernel computing KU groups per barrier needs whole multiples of
    // KU in every workgroup's K range (kg / split divides kg)
    if (ring && (kg / split) % k.unroll) return FP8BG_ERR_CONFIG;
    int64_t n_dp = tiles - n_split;
    int64_t grid = n_dp + n_split * split;
    if (grid > 0x7fffffff) return FP8BG_ERR_SHAPE;
    // Stream-K: tiles x K-groups units dealt out in runs of `per` units, one
    // run per workgroup, about one run per CU.  A run is at least half a tile
    // (so at most three runs share a tile) and at most one tile less a group
    // (so it touches at most two tiles); a multiple of the groups per
    // barrier.  Where that leaves no tile cut (tiles >= CUs), or the
    // counters (one per tile and wave) or the partials' 31-bit offsets do
    // not fit, the launch runs whole tiles instead, so a table entry of this
    // mode stays valid at any M.
    int64_t stream_units = 0, ws_stream = 0;
    if (stream) {
        const int ku = k.unroll;
        const int64_t units = tiles * kg;
        int64_t per = (units + num_cus - 1) / num_cus;
        per = max(per, (int64_t)(kg / 2));
        per = (per + ku - 1) / ku * ku;
        const int64_t sk_grid = (units + per - 1) / per;
        const int64_t parts = 2 * sk_grid * (int64_t)k.tw * k.tt;
        if (per < kg && tiles * k.ww * k.wt <= FP8BG_COUNTERS && parts * 4 <= 0x7fffffffLL) {
            stream_units = per;
            ws_stream = FP8BG_COUNTERS + parts;
            n_dp = 0;
            n_split = tiles;
            grid = sk_grid;
        }
    }
    int64_t lds;
    if (skinny) {
        lds = (int64_t)k.wk * (k.tw / 16) * (k.tt / 16) * 64 * 16;
    } else if (ring) {
        const int nwave = k.ww * k.wt;
        lds = (int64_t)k.stages * ((k.tw + k.tt) * 128 +
                                   ring_scale_slices(k.tw, k.tt, nwave) * nwave * 64 * 4);
    } else {
        lds = 2LL * (k.tw + k.tt) * 128;
        if (cfg->flags & FP8BG_FLAG_SCALE_LDS) lds += (int64_t)k.tt * kg * 4;
    }
    if (lds > kMaxLds) return FP8BG_ERR_CONFIG;

    plan->tiles_w = (int32_t)tiles_w;
    plan->tiles_t = (int32_t)tiles_t;
    plan->tiles = (int32_t)tiles;
    plan->split = split;
    plan->n_dp = (int32_t)n_dp;
    plan->n_split = (int32_t)n_split;
    plan->grid = (int32_t)grid;
    plan->launches = n_split && !in_kernel && !stream_units ? 2 : 1;
    plan->ws_elems = stream_units ? ws_stream
                     : n_split    ? FP8BG_COUNTERS + n_split * split * (int64_t)k.tw * k.tt
                                  : 0;
    plan->lds_bytes = (int32_t)lds;
    plan->threads = k.threads;
    plan->kernel_id = ki;
    plan->stream_units = (int32_t)stream_units;
    return FP8BG_OK;
}

}  // extern "C"

namespace {

// The GEMM enqueue shared by fp8bg_gemm (caller's workspace) and
// fp8bg_gemm_noalloc (the library's static scratch): plan, checks, the GEMM
// kernel and, for split tiles, the fixed-order reduction.  `ws_check`
// validates the workspace size once the plan is known (it may refuse).
template <typename WsCheck>
int gemm_enqueue(const void* A, const void* B, const float* As, int64_t as_stride_m,
                 int64_t as_stride_k, const float* Bs, int64_t bs_stride_n, int64_t bs_stride_k,
                 const void* bias, void* C, int32_t M, int32_t N, int32_t K,
                 const fp8bg_config* cfg, int32_t num_cus, void* stream, WsCheck ws_check) {
    if (!A || !B || !As || !Bs || !C) return FP8BG_ERR_NULL;
    if (((uintptr_t)bias) & 7) return FP8BG_ERR_ALIGN;
    fp8bg_plan p;
    const int rc = fp8bg_make_plan(M, N, K, cfg, num_cus, &p);
    if (rc != FP8BG_OK) return rc;
    if ((((uintptr_t)A) | ((uintptr_t)B) | ((uintptr_t)C)) & 15) return FP8BG_ERR_ALIGN;
    float* ws = nullptr;
    if (p.n_split > 0) {
        const int wrc = ws_check(p.ws_elems, &ws);
        if (wrc != FP8BG_OK) return wrc;
    }

    const Instance& k = kInstances[p.kernel_id];
    KArgs a = {};
    a.A = (const uint8_t*)A;
    a.B = (const uint8_t*)B;
    a.As = As;
    a.Bs = Bs;
    a.C = (uint16_t*)C;
    a.bias = (const uint16_t*)bias;
    // workspace: the tile counters, then the partials
    a.cnt = (uint32_t*)ws;
    a.ws = ws ? ws + FP8BG_COUNTERS : nullptr;
    a.stream = p.stream_units > 0;
    a.split_last = p.n_split > 0 && p.launches == 1 && !a.stream;  // FP8BG_SPLIT_LAST within its limits
    a.as_sm = as_stride_m;
    a.as_sk = as_stride_k;
    a.bs_sn = bs_stride_n;
    a.bs_sk = bs_stride_k;
    a.M = M;
    a.N = N;
    a.K = K;
    a.tw = k.tw;
    a.tt = k.tt;
    a.tiles_w = p.tiles_w;
    a.tiles_t = p.tiles_t;
    a.n_dp = p.n_dp;
    a.split = p.split;
    a.kcount = a.stream ? p.stream_units : (K / kGroupK) / p.split;
    a.div_split = fast_div_of((uint32_t)p.split);
    a.div_tiles_t = fast_div_of((uint32_t)p.tiles_t);
    a.group_t = cfg->group_t;
    a.xcd_remap = (cfg->flags & FP8BG_FLAG_XCD_REMAP) ? 1 : 0;
    a.scale_lds = (cfg->flags & FP8BG_FLAG_SCALE_LDS) ? 1 : 0;
    a.swz = (cfg->flags & FP8BG_FLAG_SWZ8) ? 1 : (cfg->flags & FP8BG_FLAG_SWZPAIR) ? 2 : 0;
    const size_t shm = a.scale_lds ? (size_t)k.tt * (K / 128) * sizeof(float) : 0;
    hipStream_t s = (hipStream_t)stream;
    ((cfg->flags & FP8BG_FLAG_B_SHUFFLED) ? k.launch_bs : k.launch)(dim3(p.grid), shm, s, &a);
    if (hipGetLastError() != hipSuccess) return FP8BG_ERR_LAUNCH;
    if (p.launches == 2) {
        const int parts = reduce_parts(p, k, num_cus);
        hipLaunchKernelGGL(fp8bg_split_reduce, dim3(p.n_split * parts), dim3(kThreads), 0, s, a,
                           k.kind == FP8BG_KIND_SKINNY ? 1 : 0, parts);
        if (hipGetLastError() != hipSuccess) return FP8BG_ERR_LAUNCH;
    }
    return FP8BG_OK;
}

// Split-K scratch of fp8bg_gemm_noalloc: one copy per GPU, held until the
// process ends.  In host code `scratch` names a host-side stand-in, not a
// device address; kernels receive the per-device address that
// hipGetSymbolAddress returns, looked up once per device with that device
// current and kept in scratch_ptr.  Its layout is the workspace's:
// FP8BG_COUNTERS tile counters, then the partials.  The counters must start
// at zero: they do because the array is zero-filled when the code object
// loads, and every in-kernel reduction (FP8BG_SPLIT_LAST, _STREAM) resets
// each counter it completes, so every call leaves them zero.  The partials
// need no clearing: every split call writes each partial it reads.
static __device__ __align__(256) float scratch[FP8BG_SCRATCH_ELEMS];

constexpr int kMaxDevices = 64;
std::atomic<float*> scratch_ptr[kMaxDevices];
std::mutex scratch_mu;

// Device address of `scratch` on the device of `stream` (which must be the
// current device).
int scratch_address(void* stream, float** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FP8BG_ERR_DEVICE;
    if (stream) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev)
            return FP8BG_ERR_DEVICE;
    }
    float* p = scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(scratch_mu);
        p = scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* q = nullptr;
            if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return FP8BG_ERR_DEVICE;
            p = (float*)q;
            scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return FP8BG_OK;
}

}  // namespace

extern "C" {

int fp8bg_gemm(const void* A, const void* B, const float* As, int64_t as_stride_m,
               int64_t as_stride_k, const float* Bs, int64_t bs_stride_n, int64_t bs_stride_k,
               const void* bias, void* C, int32_t M, int32_t N, int32_t K,
               const fp8bg_config* cfg, int32_t num_cus, float* ws, int64_t ws_elems,
               void* stream) {
    return gemm_enqueue(A, B, As, as_stride_m, as_stride_k, Bs, bs_stride_n, bs_stride_k, bias, C,
                        M, N, K, cfg, num_cus, stream, [&](int64_t need, float** out) {
                            if (!ws || ws_elems < need || (((uintptr_t)ws) & 15))
                                return FP8BG_ERR_WORKSPACE;
                            *out = ws;
                            return FP8BG_OK;
                        });
}

int fp8bg_gemm_noalloc(const void* A, const void* B, const float* As, int64_t as_stride_m,
                       int64_t as_stride_k, const float* Bs, int64_t bs_stride_n,
                       int64_t bs_stride_k, const void* bias, void* C, int32_t M, int32_t N,
                       int32_t K, const fp8bg_config* cfg, int32_t num_cus, void* stream) {
    return gemm_enqueue(A, B, As, as_stride_m, as_stride_k, Bs, bs_stride_n, bs_stride_k, bias, C,
                        M, N, K, cfg, num_cus, stream, [&](int64_t need, float** out) {
                            if (need > FP8BG_SCRATCH_ELEMS) return FP8BG_ERR_SCRATCH;
                            return scratch_address(stream, out);
                        });
}

int fp8bg_gemm_bf16a(const void* X, int64_t x_stride_m, float eps, const void* B, const float* Bs,
                     int64_t bs_stride_n, int64_t bs_stride_k, const void* bias, void* C, int32_t M,
                     int32_t N, int32_t K, const fp8bg_config* cfg, int32_t num_cus, float* ws,
                     int64_t ws_elems, void* q_out, float* s_out, int64_t s_stride_m,
                     int64_t s_stride_k, void* stream) {
    if (!X || !B || !Bs || !C || !cfg) return FP8BG_ERR_NULL;
    if ((q_out == nullptr) != (s_out == nullptr)) return FP8BG_ERR_NULL;
    const int qi = find_qa_instance(cfg);
    if (qi < 0) return FP8BG_ERR_CONFIG;
    // 1 / (max(amax, eps) / 448) stays finite
    if (!(eps >= 1e-30f) || !(eps < 3.4e38f)) return FP8BG_ERR_CONFIG;
    fp8bg_plan p;
    const int rc = fp8bg_make_plan(M, N, K, cfg, num_cus, &p);
    if (rc != FP8BG_OK) return rc;
    if (x_stride_m < K) return FP8BG_ERR_SHAPE;
    if ((((uintptr_t)X) | ((uintptr_t)B) | ((uintptr_t)C) | ((uintptr_t)q_out)) & 15 ||
        (x_stride_m % 8) || (((uintptr_t)bias) & 7) || (((uintptr_t)s_out) & 3))
        return FP8BG_ERR_ALIGN;
    if (p.n_split > 0 && (!ws || ws_elems < p.ws_elems || (((uintptr_t)ws) & 15)))
        return FP8BG_ERR_WORKSPACE;

    const Instance& k = kQaInstances[qi];
    KArgs a = {};
    a.B = (const uint8_t*)B;
    a.Bs = Bs;
    a.C = (uint16_t*)C;
    a.bias = (const uint16_t*)bias;
    a.cnt = (uint32_t*)ws;
    a.ws = ws ? ws + FP8BG_COUNTERS : nullptr;
    a.split_last = p.n_split > 0 && p.launches == 1;  // FP8BG_SPLIT_LAST within its limits
    a.bs_sn = bs_stride_n;
    a.bs_sk = bs_stride_k;
    a.M = M;
    a.N = N;
    a.K = K;
    a.tw = k.tw;
    a.tt = k.tt;
    a.tiles_w = p.tiles_w;
    a.tiles_t = p.tiles_t;
    a.n_dp = p.n_dp;
    a.split = p.split;
    a.kcount = (K / kGroupK) / p.split;
    a.div_split = fast_div_of((uint32_t)p.split);
    a.div_tiles_t = fast_div_of((uint32_t)p.tiles_t);
    a.group_t = cfg->group_t;
    a.xcd_remap = (cfg->flags & FP8BG_FLAG_XCD_REMAP) ? 1 : 0;
    a.X = (const uint16_t*)X;
    a.ldx = x_stride_m;
    a.eps = eps;
    a.eps_s = eps / 448.0f;
    a.eps_r = 1.0f / a.eps_s;
    a.q_out = (uint8_t*)q_out;
    a.s_out = s_out;
    a.qs_sm = s_stride_m;
    a.qs_sk = s_stride_k;
    hipStream_t s = (hipStream_t)stream;
    ((cfg->flags & FP8BG_FLAG_B_SHUFFLED) ? k.launch_bs : k.launch)(dim3(p.grid), 0, s, &a);
    if (hipGetLastError() != hipSuccess) return FP8BG_ERR_LAUNCH;
    if (p.n_split > 0 && !a.split_last) {
        const int parts = reduce_parts(p, k, num_cus);
        hipLaunchKernelGGL(fp8bg_split_reduce, dim3(p.n_split * parts), dim3(kThreads), 0, s, a, 1,
                           parts);
        if (hipGetLastError() != hipSuccess) return FP8BG_ERR_LAUNCH;
    }
    return FP8BG_OK;
}

int fp8bg_quant_act(const void* x, int64_t x_stride_m, void* q, float* s, int64_t s_stride_m,
                    int64_t s_stride_k, int32_t M, int32_t K, float eps, void* stream) {
    if (!x || !q || !s) return FP8BG_ERR_NULL;
    if (M < 1 || K < 128 || K % 128 || x_stride_m < K) return FP8BG_ERR_SHAPE;
    if (!(eps > 0.f) || !(eps < 3.4e38f)) return FP8BG_ERR_CONFIG;
    // 16-byte loads of x rows and 8-byte stores of q
    if ((((uintptr_t)x) & 15) || (x_stride_m % 8) || (((uintptr_t)q) & 7) || (((uintptr_t)s) & 3))
        return FP8BG_ERR_ALIGN;
    const int64_t groups = (int64_t)M * (K / 128);
    const int64_t blocks = (groups + kThreads / 16 - 1) / (kThreads / 16);
    if (blocks > 0x7fffffff) return FP8BG_ERR_SHAPE;
    QArgs a;
    a.x = (const uint16_t*)x;
    a.q = (uint8_t*)q;
    a.s = s;
    a.ldx = x_stride_m;
    a.s_sm = s_stride_m;
    a.s_sk = s_stride_k;
    a.M = M;
    a.K = K;
    a.eps = eps;
    a.eps_s = eps / 448.0f;
    a.eps_r = 1.0f / a.eps_s;
    hipLaunchKernelGGL(fp8bg_quant_act_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                       (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_shuffle_b(const void* B, int64_t b_stride_n, void* Bt, int32_t N, int32_t K, void* stream) {
    if (!B || !Bt) return FP8BG_ERR_NULL;
    if (N < 16 || N % 16 || K < 128 || K % 128 || b_stride_n < K) return FP8BG_ERR_SHAPE;
    if ((((uintptr_t)B) | ((uintptr_t)Bt) | (uintptr_t)b_stride_n) & 15) return FP8BG_ERR_ALIGN;
    const uint8_t* b = (const uint8_t*)B;
    const uint8_t* bt = (const uint8_t*)Bt;
    // the output must not overlap the rows it reads (no in-place shuffle)
    const uint8_t* b_end = b + (int64_t)(N - 1) * b_stride_n + K;
    if (bt < b_end && b < bt + (int64_t)N * K) return FP8BG_ERR_SHAPE;
    const int64_t chunks = (int64_t)N * K / 16;
    const int64_t want = (chunks + kThreads - 1) / kThreads;
    const int64_t blocks = want < 4096 ? want : 4096;
    hipLaunchKernelGGL(fp8bg_shuffle_b_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                       (hipStream_t)stream, b, b_stride_n, (uint8_t*)Bt, chunks, K / 128);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_calib_mfma(const int32_t* codes, float* out, int32_t workgroups, int32_t iters,
                     void* stream) {
    if (!codes || !out) return FP8BG_ERR_NULL;
    if (workgroups < 1 || iters < 1 || iters > FP8BG_CALIB_MAX_ITERS) return FP8BG_ERR_SHAPE;
    if ((((uintptr_t)codes) & 3) || (((uintptr_t)out) & 3)) return FP8BG_ERR_ALIGN;
    hipLaunchKernelGGL(fp8bg_calib_mfma_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                       (hipStream_t)stream, (const int32_t*)codes, out, iters);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_calib_mfma_promoted(const int32_t* codes, const float* scale, float* out, int32_t workgroups,
                              int32_t iters, void* stream) {
    if (!codes || !scale || !out) return FP8BG_ERR_NULL;
    if (workgroups < 1 || iters < 1 || iters > FP8BG_CALIB_MAX_ITERS) return FP8BG_ERR_SHAPE;
    if ((((uintptr_t)codes) & 3) || (((uintptr_t)scale) & 3) || (((uintptr_t)out) & 3)) return FP8BG_ERR_ALIGN;
    hipLaunchKernelGGL(fp8bg_calib_promote_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                       (hipStream_t)stream, (const int32_t*)codes, scale, out, iters);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_calib_read(const void* src, int64_t bytes, uint32_t* out, int32_t workgroups,
                     void* stream) {
    if (!src || !out) return FP8BG_ERR_NULL;
    if (bytes < 16 || bytes % 16 || workgroups < 1) return FP8BG_ERR_SHAPE;
    if ((((uintptr_t)src) & 15) || (((uintptr_t)out) & 3)) return FP8BG_ERR_ALIGN;
    hipLaunchKernelGGL(fp8bg_calib_read_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                       (hipStream_t)stream, (const i32x4*)src, bytes / 16, out);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_calib_write(void* dst, int64_t bytes, uint32_t value, int32_t workgroups, int32_t nontemporal,
                      void* stream) {
    if (!dst) return FP8BG_ERR_NULL;
    if (bytes < 16 || bytes % 16 || workgroups < 1) return FP8BG_ERR_SHAPE;
    if (((uintptr_t)dst) & 15) return FP8BG_ERR_ALIGN;
    if (nontemporal)
        hipLaunchKernelGGL(fp8bg_calib_write_kernel<true>, dim3((unsigned)workgroups), dim3(256), 0,
                           (hipStream_t)stream, (i32x4*)dst, bytes / 16, value);
    else
        hipLaunchKernelGGL(fp8bg_calib_write_kernel<false>, dim3((unsigned)workgroups), dim3(256), 0,
                           (hipStream_t)stream, (i32x4*)dst, bytes / 16, value);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_calib_launch(int32_t workgroups, void* stream) {
    if (workgroups < 1) return FP8BG_ERR_SHAPE;
    hipLaunchKernelGGL(fp8bg_calib_empty_kernel, dim3((unsigned)workgroups), dim3(64), 0, (hipStream_t)stream);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

int fp8bg_e4m3_encode_host(const float* x, uint8_t* out, int64_t n) {
    if (!x || !out || n < 0) return FP8BG_ERR_NULL;
    for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)e4m3_from_f32(x[i]);
    return FP8BG_OK;
}

int fp8bg_e4m3_encode_device(const float* x, uint8_t* out, int64_t n, void* stream) {
    if (!x || !out) return FP8BG_ERR_NULL;
    if (n < 0) return FP8BG_ERR_SHAPE;
    if (n == 0) return FP8BG_OK;
    const int64_t blocks = std::min<int64_t>(((n + 1) / 2 + kThreads - 1) / kThreads, 65536);
    hipLaunchKernelGGL(fp8bg_e4m3_cvt_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, x,
                       out, n);
    return hipGetLastError() == hipSuccess ? FP8BG_OK : FP8BG_ERR_LAUNCH;
}

}  // extern "C"

#endif  // FP8BG_HOST_PART
