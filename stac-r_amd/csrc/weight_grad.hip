// Weight gradient from the saved factors: dW = (G^T C) Q^T + G^T R_s, dbias = sum_t G.
//
// Restates stacr/layers.py:172-198.  Accumulation is fp32 and dW is rounded once to the weight
// dtype (the reference rounds the d_out x r product and the low-rank term to G's dtype before
// adding its fp32 sparse correction; one rounding at the end is the more accurate of the two).
// Residual codes are dequantized as QuantizedValues.dequantize(fp32) does (stacr/quant.py:17-21,
// 40-46): products use the exact integer code and the per-tensor fp32 scale multiplies each
// segment's sum when it is added to the accumulator.
//
// Two launches:
//   k_dw_plan  for every block of TB token rows and every input-feature part: the block's residual
//              entries bucketed by input feature (in rounds of <= 4096 entries) and cut into equal
//              runs of P entries, one run per thread of the streaming kernel, plus the list of
//              features whose entries cross a run boundary.  Done once, shared by all o-slabs.
//   k_dw_fused one streaming pass over G.  A workgroup owns 16 output features (an "o-slab") and
//              one part of <= 1024 input features.  Per block of token rows it
//                * accumulates M = G^T [C | 1] in registers (packed bf16/fp16 dot products, or
//                  fp32 FMAs), which also yields dbias;
//                * walks its run of bucketed entries, summing v * G[t, o-slab] per feature in
//                  registers, and adds each feature's sum into an LDS accumulator S[i][o]; a sum
//                  that continues a feature from the previous run goes to a slot instead, and the
//                  slots are added (in run order) after a barrier;
//              then reduces M over its threads and writes dW = M Q^T + S for its tile.
// Within a feature, entries follow the bucket order, which is ascending row order: each entry's
// place is its feature's bucket start plus the number of the feature's entries in earlier rows of
// the round, counted from a per-feature row bitmap, so the sparse term is the same bit for bit on
// every run.  (A round holding the same (row, feature) twice, which no valid input does, falls back
// to places handed out by an LDS counter in arrival order.)
#include <type_traits>

#include "internal.h"

using namespace stacr;

namespace {

constexpr int kOSlab = 16;          // output features per workgroup
constexpr int kMaxISlab = 1024;     // input features per part: S = 1024 x 16 fp32 = 64 KiB of LDS
constexpr int kBwdThreads = 1024;   // 16 waves: four per SIMD, so memory and LDS latency overlap
constexpr int kPlanThreads = 512;   // the planner: two input features per thread
constexpr int kRoundMax = 4096;     // residual entries bucketed per round (16-bit G; 2048 for fp32)
constexpr int kMinPiece = 8;        // shortest piece (entries)
constexpr int kMaxGroups = 256;     // piece groups of the widest configuration
// A round's n entries are cut into pieces of P = clamp(ceil(n / groups), kMinPiece, 255) entries:
// a feature with <= P entries is one piece, a longer ("heavy") one ceil(count / P) pieces.  Heavy
// features hold > P entries each, so there are < n / P <= groups of them, and their pieces number
// < 2 n / P <= 2 groups.  Pieces in all: < 2 groups + the features of the part.
constexpr int kSlotCap = 2 * kMaxGroups;                  // partial sums of heavy pieces
constexpr int kHeavyCap = kMaxGroups;                     // heavy features per round
constexpr int kTaskCap = kMaxISlab + kSlotCap;            // pieces per round
constexpr uint32_t kDirect = 0xffffu;                     // piece slot: add straight into S
constexpr int kTaskPT = (kTaskCap + kBwdThreads - 1) / kBwdThreads;  // staged pieces per thread
constexpr int kHdrRing = 256;                             // block headers held in LDS
static_assert(kHeavyCap <= kBwdThreads, "one heavy record per thread");
// the matrix-core streaming kernel (k_dw_fused_mfma)
constexpr int kMCols = 32;            // column features per round (two 16-column tiles)
constexpr int kMTB = 512;             // token rows per block
constexpr int kMPitch = kMTB + 8;     // elements per Bt row
constexpr int kMGRows = kMTB + 1;     // G tile rows: the block's kMTB rows, then a row of zeros
constexpr int kMSlotCap = 64;         // partial sums of heavy pieces
constexpr int kMHdrRing = 64;         // block headers held in LDS
constexpr int kMTaskCap = kMaxISlab + kMSlotCap + kMCols;
constexpr int kMTaskPT = (kMTaskCap + kBwdThreads - 1) / kBwdThreads;
static_assert(kMCols * kMPitch <= 0x8000, "a column entry's tile element fits 15 bits");

// S row i holds the 16 outputs as four 16-byte chunks; chunk q sits at position q ^ (i & 3), which
// spreads rows over the LDS banks while keeping every chunk 16-byte aligned.
constexpr int kAccPitch = kOSlab;
__device__ __forceinline__ int s_index(int i, int o)
{
    return i * kOSlab + ((((o >> 2) ^ i) & 3) << 2) + (o & 3);
}

template <int DT, int R>
struct GradCfg {
    using T = typename Act<DT>::T;
    static constexpr bool k16 = sizeof(T) == 2;
    // output features per thread: keeps the M accumulator at <= 72 fp32 registers
    static constexpr int OT = k16 ? (R <= 8 ? 4 : 2) : (R <= 8 ? 2 : 1);
    static constexpr int OG = kOSlab / OT;             // threads sharing one token row
    static constexpr int TP = kBwdThreads / OG;        // token-row pairs per block
    static constexpr int TB = 2 * TP;                  // token rows per block
    static constexpr int VB = OT * (int)sizeof(T);     // G bytes per thread per row
    static constexpr int NV = OT * (R + 1);            // accumulator values per thread
    static constexpr int CW = R * (int)sizeof(T) / 4;  // 32-bit words of one (padded) C row
    static constexpr int NGRP = kBwdThreads / OG;      // piece groups (OG threads each)
    static constexpr int ROUND = k16 ? kRoundMax : kRoundMax / 2;  // entries per round
    static constexpr int EPT = ROUND / kBwdThreads;    // staged entries per thread
    static constexpr int PD = 1;                       // blocks of C rows / plan data loaded ahead
    static constexpr int GD = 1;                       // blocks of G rows loaded ahead
};

template <int B> struct Vec;
template <> struct Vec<4> { using type = uint32_t; static constexpr int n = 1; };
template <> struct Vec<8> { using type = uint2; static constexpr int n = 2; };
template <> struct Vec<16> { using type = uint4; static constexpr int n = 4; };

template <int B>
__device__ __forceinline__ void load_words(const void *p, uint32_t *w)
{
    using V = typename Vec<B>::type;
    const V v = *reinterpret_cast<const V *>(p);
    if constexpr (B == 4) {
        w[0] = v;
    } else if constexpr (B == 8) {
        w[0] = v.x; w[1] = v.y;
    } else {
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
}

// OT consecutive elements of one G row as 32-bit words (zero outside the row / matrix).  The
// vector load is used when the whole vector is in range and aligned.
template <int DT, int VB>
__device__ __forceinline__ void load_g(const typename Act<DT>::T *row, int64_t ob, int64_t d_out, bool row_ok,
                                       bool vec_ok, uint32_t (&w)[Vec<VB>::n])
{
    using T = typename Act<DT>::T;
    constexpr int OT = VB / (int)sizeof(T);
    if (row_ok && vec_ok && ob + OT <= d_out) {
        load_words<VB>(row + ob, w);
        return;
    }
#pragma unroll
    for (int k = 0; k < Vec<VB>::n; ++k) w[k] = 0u;
    if (!row_ok) return;
#pragma unroll
    for (int o = 0; o < OT; ++o) {
        if (ob + o >= d_out) break;
        if constexpr (sizeof(T) == 4) {
            w[o] = __float_as_uint(row[ob + o]);
        } else {
            w[o / 2] |= (uint32_t)(uint16_t)row[ob + o] << (16 * (o & 1));
        }
    }
}

template <int IDX64>
__device__ __forceinline__ int64_t flat_at(const void *idx, int64_t k)
{
    return IDX64 ? static_cast<const int64_t *>(idx)[k] : (int64_t) static_cast<const int32_t *>(idx)[k];
}

// off / d for off < 2^25: a float reciprocal, then an exact one-step correction
__device__ __forceinline__ uint32_t div_small(uint32_t off, uint32_t d, float inv_d)
{
    uint32_t q = (uint32_t)((float)off * inv_d);
    if (q * d > off) --q;
    else if ((q + 1) * d <= off) ++q;
    return q;
}

// ------------------------------------------------------------------ the plan
// One round of one (block, part): its bucketed entries, pieces and heavy records all start at
// plan slot `base` (a part's entries of a round occupy a private slot range, and it never has
// more pieces or heavy records than entries).
struct RoundHdr {
    uint32_t base;
    uint32_t n_ent;
    uint32_t n_task;   // column records + pieces
    uint32_t n_heavy;  // features cut into several pieces | matrix-core columns << 16
};

struct BlockHdr {
    RoundHdr r0;           // the block's first round (all zero when the block has no entries)
    uint32_t first_round;  // global index of that round
    uint32_t n_rounds;
    uint32_t pad[2];
};

struct PlanArgs {
    const void *idx;
    const void *data;
    int bits, val_dt, g_dt;
    int64_t nnz, rows, d_in;
    int64_t n_parts, i_span;
    int tb;                  // token rows per block
    uint32_t round_cap;      // entries per round (<= kRoundMax)
    uint32_t groups;         // piece groups of the streaming kernel
    uint32_t slot_cap;       // partial-sum slots of the streaming kernel
    uint32_t cols;           // matrix-core columns per round (0: every feature goes to pieces)
    uint32_t max_rounds;     // rounds the header array holds
    void *ent;               // [nnz] 16-bit G: t_local << 16 | value code (uint32); a matrix-core
                             //       column feature's entry: bit 31 | its Bt tile element << 16 | code;
                             //       fp32 G: {t_local, value bits} (uint2)
    uint2 *task;             // [nnz] column features {feature, 0} first, then pieces
                             //       {feature | slot << 16, entry offset << 8 | entries}
    uint2 *heavy;            // [nnz] {feature | first slot << 16, pieces}
    RoundHdr *rhdr;          // [global round][part]
    BlockHdr *bhdr;          // [block][part]
};

// The product operand of entry e: the integer code (exact in bf16/fp16) for bits 4/8, the stored
// value for bits 0; as G's 16-bit code, or fp32 bits for fp32 G.
// Entry values come in one of four layouts (VK): int8 codes (bits 8), packed int4 codes (bits
// 4), 16-bit or fp32 stored values (bits 0).  The raw load is one branch-free instruction per
// layout, so a thread's loads all stay in flight together; the decode follows.
enum { kValI8 = 0, kValI4 = 1, kVal16 = 2, kVal32 = 3 };
template <int VK>
__device__ __forceinline__ uint32_t entry_raw(const void *data, uint32_t e)
{
    if constexpr (VK == kValI8) return static_cast<const uint8_t *>(data)[e];
    else if constexpr (VK == kValI4) return static_cast<const uint8_t *>(data)[e >> 1];
    else if constexpr (VK == kVal16) return static_cast<const uint16_t *>(data)[e];
    else return static_cast<const uint32_t *>(data)[e];
}
template <int VK>
__device__ __forceinline__ uint32_t entry_value(const PlanArgs &a, uint32_t raw, uint32_t e)
{
    float v;
    if constexpr (VK == kValI8) {
        v = (float)(int8_t)raw;
    } else if constexpr (VK == kValI4) {
        const int n = (int)((e & 1) ? (raw >> 4) : (raw & 0xfu));
        v = (float)(n > 7 ? n - 16 : n);
    } else if constexpr (VK == kVal16) {
        v = a.val_dt == STACR_DTYPE_BF16 ? bf16_bits_to_f(raw) : f16_bits_to_f(raw);
    } else {
        v = __uint_as_float(raw);
    }
    if (a.g_dt == STACR_DTYPE_BF16) return f_to_bf16_bits(v);
    if (a.g_dt == STACR_DTYPE_F16) return f_to_f16_bits(v);
    return __float_as_uint(v);
}

// Exclusive prefix sum over the planner's workgroup with one barrier: the per-wave totals go to
// `buf`, which callers alternate between two arrays, so a wave still reading one scan's totals
// never sees the next scan's (a buffer is reused only after another scan's barrier).
__device__ __forceinline__ uint32_t scan1(uint32_t v, uint32_t *buf, uint32_t *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) buf[wave] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kPlanThreads / 64; ++w) {
        const uint32_t t = buf[w];
        before += w < wave ? t : 0u;
        all += t;
    }
    *total = all;
    return before + x - v;
}

template <int IDX64, int VK>
__global__ __launch_bounds__(kPlanThreads) void k_dw_plan(PlanArgs a)
{
    __shared__ uint32_t cnt[kMaxISlab], ccur[kMaxISlab];
    __shared__ __attribute__((aligned(16))) uint32_t rowbits[16 * kMaxISlab];  // [row / 32][feature]: the round's rows
    static_assert(GradCfg<STACR_DTYPE_BF16, 4>::TB <= 512 && GradCfg<STACR_DTYPE_F32, 4>::TB <= 512 && kMTB <= 512,
                  "blocks of at most 512 rows: 16 bitmap words a feature");
    __shared__ uint32_t s_dup;
    __shared__ uint32_t cstart[kMaxISlab], lstart[kMaxISlab], hstart[kMaxISlab], hidx[kMaxISlab];
    __shared__ uint32_t colh[kMaxISlab];  // 1 + matrix-core column of a feature, 0 for pieces
    __shared__ uint32_t s_tot[2][kPlanThreads / 64];        // scan1 buffers, used alternately
    __shared__ uint32_t s_cnt[2][kPlanThreads / 64];        // range search: per-wave counts
    __shared__ uint32_t s_probe[2][15][kPlanThreads / 64];  // column search: per-wave counts
    const int64_t b = blockIdx.x, p = blockIdx.y;
    const int64_t t0 = b * a.tb, t1 = min(t0 + a.tb, a.rows);
    const int64_t i0 = p * a.i_span;
    const int ni = (int)(min(i0 + a.i_span, a.d_in) - i0);
    const int64_t span = (t1 - t0) * a.d_in;  // flat offsets of the block's rows
    const uint32_t d_in = (uint32_t)a.d_in;
    const float inv_d = 1.f / (float)a.d_in;
    const bool one_part = a.n_parts == 1;
    const uint32_t i_span = (uint32_t)a.i_span;  // features per part (< 65536)
    const float inv_span = 1.f / (float)a.i_span;
    // entry range of a block; the clamps keep indices that are not ascending inside the arrays
    const uint32_t nnz = (uint32_t)a.nnz;
    // The block's entries [e0, e1): the first entries whose flat index is >= t0 * d_in and
    // >= t1 * d_in, found together by a 512-way parallel search of the ascending indices (the
    // result stays in [0, nnz] for indices that are not ascending, and e1 >= e0 is enforced).
    uint32_t e0, e1;
    {
        const int64_t key0 = t0 * a.d_in, key1 = t1 * a.d_in;
        uint32_t lo0 = 0u, hi0 = nnz, lo1 = 0u, hi1 = nnz;
        {   // First step: 2048 consecutive positions centred on the proportional guess nnz * t / rows
            // (where rows of similar density put the boundary).  A boundary inside the window is
            // found exactly; otherwise the search below continues on the side it lies on.
            constexpr int kW = 4 * kPlanThreads;
            const uint32_t g0 = (uint32_t)((uint64_t)nnz * (uint64_t)t0 / (uint64_t)a.rows);
            const uint32_t g1 = (uint32_t)((uint64_t)nnz * (uint64_t)t1 / (uint64_t)a.rows);
            const uint32_t w0 = min(g0 > kW / 2 ? g0 - kW / 2 : 0u, nnz - 1u);
            const uint32_t w1 = min(g1 > kW / 2 ? g1 - kW / 2 : 0u, nnz - 1u);
            const uint32_t nv0 = min((uint32_t)kW, nnz - w0), nv1 = min((uint32_t)kW, nnz - w1);
            int64_t v0[4], v1[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {  // unconditional, clamped positions (nnz > 0 here)
                v0[k] = flat_at<IDX64>(a.idx, min(w0 + threadIdx.x + k * kPlanThreads, nnz - 1u));
                v1[k] = flat_at<IDX64>(a.idx, min(w1 + threadIdx.x + k * kPlanThreads, nnz - 1u));
            }
            uint32_t m = 0u;  // samples below the key, per wave (<= 256 each: 16-bit halves)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t j = threadIdx.x + k * kPlanThreads;
                m += (uint32_t)__popcll(__ballot(j < nv0 && v0[k] < key0));
                m += (uint32_t)__popcll(__ballot(j < nv1 && v1[k] < key1)) << 16;
            }
            if ((threadIdx.x & 63) == 0) s_cnt[1][threadIdx.x >> 6] = m;
            __syncthreads();
            uint32_t c01 = 0u;
#pragma unroll
            for (int w = 0; w < kPlanThreads / 64; ++w) c01 += s_cnt[1][w];
            const uint32_t c0 = c01 & 0xffffu, c1 = c01 >> 16;
            // c == 0: the boundary is at or before the window's first position; c == nv: after its
            // last; otherwise at w + c
            if (c0 == 0u) hi0 = w0;
            else if (c0 < nv0) lo0 = hi0 = w0 + c0;
            else lo0 = w0 + nv0;
            if (c1 == 0u) hi1 = w1;
            else if (c1 < nv1) lo1 = hi1 = w1 + c1;
            else lo1 = w1 + nv1;
        }
        for (int it = 0; lo0 < hi0 || lo1 < hi1; ++it) {
            const uint32_t st0 = max(1u, (hi0 - lo0 + kPlanThreads - 1) / kPlanThreads);
            const uint32_t st1 = max(1u, (hi1 - lo1 + kPlanThreads - 1) / kPlanThreads);
            const uint32_t p0 = lo0 + threadIdx.x * st0, p1 = lo1 + threadIdx.x * st1;
            // both samples loaded unconditionally (clamped positions; nnz > 0 here), one barrier
            const int64_t v0 = flat_at<IDX64>(a.idx, min(p0, nnz - 1u)), v1 = flat_at<IDX64>(a.idx, min(p1, nnz - 1u));
            const bool b0 = p0 < hi0 && v0 < key0;
            const bool b1 = p1 < hi1 && v1 < key1;
            const uint32_t m = (uint32_t)__popcll(__ballot(b0)) | ((uint32_t)__popcll(__ballot(b1)) << 16);
            if ((threadIdx.x & 63) == 0) s_cnt[it & 1][threadIdx.x >> 6] = m;  // <= 512 each: 16-bit halves
            __syncthreads();
            uint32_t c01 = 0u;
#pragma unroll
            for (int w = 0; w < kPlanThreads / 64; ++w) c01 += s_cnt[it & 1][w];
            const uint32_t c0 = c01 & 0xffffu, c1 = c01 >> 16;
            if (c0 == 0u) hi0 = lo0;  // the first sample is not below the key
            else { lo0 += (c0 - 1u) * st0 + 1u; hi0 = min(hi0, lo0 - 1u + st0); }
            if (c1 == 0u) hi1 = lo1;
            else { lo1 += (c1 - 1u) * st1 + 1u; hi1 = min(hi1, lo1 - 1u + st1); }
            if (st0 == 1u) hi0 = lo0;  // unit steps: every position was sampled
            if (st1 == 1u) hi1 = lo1;
        }
        e0 = lo0;
        e1 = max(e0, lo1);
    }
    const uint32_t cap = a.round_cap;
    uint32_t n_rounds = (e1 - e0 + cap - 1) / cap;
    // Round numbering: floor(e0 / cap) + b.  A block with n entries has <= floor(n / cap) + 1
    // rounds, so the ranges of consecutive blocks never overlap and stay below nnz / cap + blocks.
    const uint32_t first = e0 / cap + (uint32_t)b;
    if (first + n_rounds > a.max_rounds) n_rounds = 0;  // only for indices that are not ascending
    if (threadIdx.x == 0 && n_rounds == 0)
        a.bhdr[b * a.n_parts + p] = BlockHdr{RoundHdr{0u, 0u, 0u, 0u}, first, 0u, {0u, 0u}};
    const bool f32 = a.g_dt == STACR_DTYPE_F32;
    for (uint32_t j = 0; j < n_rounds; ++j) {
        const uint32_t c0 = e0 + j * cap, c1 = min(c0 + cap, e1);
        for (int c = threadIdx.x; c < ni; c += kPlanThreads) {
            cnt[c] = 0u;
            ccur[c] = 0u;
        }
        for (int i = threadIdx.x; i < 16 * kMaxISlab / 4; i += kPlanThreads)
            reinterpret_cast<uint4 *>(rowbits)[i] = make_uint4(0u, 0u, 0u, 0u);
        if (threadIdx.x == 0) s_dup = 0u;
        __syncthreads();
        constexpr int EPT = kRoundMax / kPlanThreads;
        uint32_t col[EPT], tl[EPT], val[EPT];
        int64_t fl[EPT];
        // every index and value load is issued before any is used: unconditional, from an entry
        // clamped into the round (c1 > c0), masked below (a load merged from divergent paths
        // would be waited for at once)
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t e = min(c0 + threadIdx.x + k * kPlanThreads, c1 - 1u);
            fl[k] = flat_at<IDX64>(a.idx, e);
            val[k] = entry_raw<VK>(a.data, e);  // decoded where used, at the end
        }
        uint32_t before = 0;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            col[k] = 0xffffffffu;
            tl[k] = 0u;
            const uint32_t e = c0 + threadIdx.x + k * kPlanThreads;
            const int64_t off64 = e < c1 ? fl[k] - t0 * a.d_in : -1;
            if (off64 >= 0 && off64 < span) {
                const uint32_t off = (uint32_t)off64;  // < 2^25: tb <= 512 rows of < 65536 features
                const uint32_t t = div_small(off, d_in, inv_d);
                const uint32_t c = off - t * d_in;
                const uint32_t part = one_part ? 0u : div_small(c, i_span, inv_span);
                before += part < (uint32_t)p;
                if (part == (uint32_t)p) {
                    col[k] = c - (uint32_t)i0;
                    tl[k] = t;
                    atomicAdd(&cnt[col[k]], 1u);
                    // (t < tb <= 512 rows: 16 words a feature)
                    const uint32_t bit = 1u << (t & 31u);
                    if (atomicOr(&rowbits[(t >> 5) * kMaxISlab + col[k]], bit) & bit) s_dup = 1u;
                }
            }
        }
        // The planner's prefix sums take one barrier each (scan1, buffers alternating) and carry
        // several small counts packed into one word; each field's bound is stated where it is packed.
        uint32_t n_before = 0u;
        if (a.n_parts > 1) (void)scan1(before, s_tot[0], &n_before);  // also orders the counts
        else __syncthreads();  // the feature counts are complete
        const uint32_t base = c0 + n_before;
        const int f0 = 2 * threadIdx.x;
        const uint32_t n0 = f0 < ni ? cnt[f0] : 0u, n1 = f0 + 1 < ni ? cnt[f0 + 1] : 0u;
        // Matrix-core columns (cols > 0): the features with the most entries, at most cols of them
        // and at least 2 entries each; ties at the cut go to the lower feature index.  tau is the
        // smallest count with #{count >= tau} <= cols; features with tau - 1 entries fill the rest.
        // Any t > n / (cols + 1) qualifies (cols + 1 features of t entries would exceed the round's
        // n entries), so tau lies in [2, n / (cols + 1) + 1]: at most 125 for rounds of 4096.
        uint32_t tau = 0xffffffffu;
        if (a.cols > 0) {
            // 16-way search: fifteen probes per step, counted by wave ballots, one barrier a step
            uint32_t lo = 2, hi = max(2u, (c1 - c0) / (a.cols + 1) + 1);
            for (int it = 0; lo < hi; ++it) {
                const uint32_t span_ = hi - lo;
#pragma unroll
                for (int i = 0; i < 15; ++i) {
                    const uint32_t pt = lo + (span_ * (uint32_t)(i + 1)) / 16;
                    const uint32_t m = (uint32_t)__popcll(__ballot(n0 >= pt)) + (uint32_t)__popcll(__ballot(n1 >= pt));
                    if ((threadIdx.x & 63) == 0) s_probe[it & 1][i][threadIdx.x >> 6] = m;
                }
                __syncthreads();
                // lane i < 15 totals probe i; the counts fall as the probes rise, so the probes within
                // the cap form a suffix and the first of them is the new upper end
                const int ln = threadIdx.x & 63;
                uint32_t m = 0;
#pragma unroll
                for (int w = 0; w < kPlanThreads / 64; ++w) m += s_probe[it & 1][min(ln, 14)][w];
                const uint64_t ok = __ballot(ln < 15 && m <= a.cols);
                const int i0 = ok ? __ffsll((unsigned long long)ok) - 1 : 15;
                const uint32_t nlo = i0 > 0 ? lo + (span_ * (uint32_t)i0) / 16 + 1 : lo;
                const uint32_t nhi = i0 < 15 ? lo + (span_ * (uint32_t)(i0 + 1)) / 16 : hi;
                lo = nlo;
                hi = max(nhi, nlo);
            }
            tau = lo;
        }
        bool k0 = false, k1 = false;
        uint32_t n_cols, se, tot_e, tot_p;
        {
            // features at or above the cut (total <= cols <= 32: bits 0..5), features one below it
            // (<= 1024 features: bits 6..16), entries (<= 4096: bits 17..31)
            const uint32_t a0 = n0 >= tau, a1 = n1 >= tau;
            const uint32_t t0 = tau > 2 && tau != 0xffffffffu && n0 == tau - 1, t1 = tau > 2 && tau != 0xffffffffu && n1 == tau - 1;
            uint32_t tot;
            const uint32_t x = scan1(a0 + a1 + ((t0 + t1) << 6) + ((n0 + n1) << 17), s_tot[1], &tot);
            const uint32_t room = a.cols - (tot & 63u), rt = (x >> 6) & 2047u;
            se = x >> 17;
            tot_e = tot >> 17;
            k0 = a0 || (t0 && rt < room);
            k1 = a1 || (t1 && rt + t0 < room);
            // column features (<= cols: bits 0..5) and the entries that go to pieces (<= 4096: 6..31)
            const uint32_t m0 = k0 ? 0u : n0, m1 = k1 ? 0u : n1;
            const uint32_t y = scan1(k0 + k1 + ((m0 + m1) << 6), s_tot[0], &tot);
            n_cols = tot & 63u;
            tot_p = tot >> 6;
            const uint32_t sc = y & 63u;
            if (f0 < ni) colh[f0] = k0 ? sc + 1 : 0u;
            if (f0 + 1 < ni) colh[f0 + 1] = k1 ? sc + k0 + 1 : 0u;
        }
        // bucket starts; then, with the piece length fixed by the part's piece-bound entry count,
        // heavy-piece starts (= partial-sum slots), light piece positions and heavy-record
        // positions.  Heavy pieces come first in the piece list (after the column records), so the
        // longest work starts first.
        uint32_t piece;
        float inv_piece;
        {
            const uint32_t m0 = k0 ? 0u : n0, m1 = k1 ? 0u : n1;  // entries that go to pieces
            // pieces of heavy features number < 2 tot_p / piece <= slot_cap, and heavy features
            // < tot_p / piece <= groups
            piece = max((tot_p + a.groups - 1) / a.groups, (2 * tot_p + a.slot_cap - 1) / a.slot_cap);
            piece = min(max(piece, (uint32_t)kMinPiece), 255u);
            if (a.cols > 0) {
                // Shorter pieces when the exact counts allow: a piece of 4 entries is one batch of
                // the streaming kernel, so the waves' piece work evens out.  For P = 4, 8, 16 the
                // partial-sum slots sum(ceil(m / P) over features with m > P) (<= 1843, 967, 496:
                // 11, 10 and 9 bits) and the split features #(m > P) (<= 819, 455, 240: 10, 9 and 8
                // bits) of the round, packed two words.
                auto slots = [](uint32_t m, int sh) { return m > (1u << sh) ? (m + (1u << sh) - 1) >> sh : 0u; };
                const uint32_t w1 = (slots(m0, 2) + slots(m1, 2)) | ((slots(m0, 3) + slots(m1, 3)) << 11) |
                                    ((slots(m0, 4) + slots(m1, 4)) << 21);
                const uint32_t w2 = ((m0 > 4) + (m1 > 4)) | (((m0 > 8) + (m1 > 8)) << 10) | (((m0 > 16) + (m1 > 16)) << 19);
                uint32_t t1, t2;
                (void)scan1(w1, s_tot[1], &t1);
                (void)scan1(w2, s_tot[0], &t2);
                const uint32_t hcap = min(a.groups, (uint32_t)kHeavyCap);
                if ((t1 & 2047u) <= a.slot_cap && (t2 & 1023u) <= hcap) piece = 4;
                else if (((t1 >> 11) & 1023u) <= a.slot_cap && ((t2 >> 10) & 511u) <= hcap) piece = min(piece, 8u);
                else if ((t1 >> 21) <= a.slot_cap && (t2 >> 19) <= hcap) piece = min(piece, 16u);
            }
            inv_piece = 1.f / (float)piece;  // divisions of counts < 2^25: exact with div_small
            const uint32_t p0 = div_small(m0 + piece - 1, piece, inv_piece), p1 = div_small(m1 + piece - 1, piece, inv_piece);
            const uint32_t h0 = p0 > 1 ? p0 : 0u, h1 = p1 > 1 ? p1 : 0u;
            const uint32_t l0 = p0 == 1, l1 = p1 == 1;
            // heavy pieces (<= slot_cap <= 512: bits 0..9), light pieces (<= 1024 features:
            // bits 10..20), heavy features (<= 512: bits 21..31)
            uint32_t tot;
            const uint32_t z = scan1(h0 + h1 + ((l0 + l1) << 10) + (((p0 > 1) + (p1 > 1)) << 21), s_tot[1], &tot);
            const uint32_t sh = z & 1023u, sl = (z >> 10) & 2047u, sx = z >> 21;
            const uint32_t tot_h = tot & 1023u, tot_l = (tot >> 10) & 2047u, tot_x = tot >> 21;
            if (f0 < ni) {
                cstart[f0] = se; hstart[f0] = sh; lstart[f0] = tot_h + sl; hidx[f0] = sx;
                if (a.cols == 0) colh[f0] = 0u;
            }
            if (f0 + 1 < ni) {
                cstart[f0 + 1] = se + n0; hstart[f0 + 1] = sh + h0; lstart[f0 + 1] = tot_h + sl + l0;
                hidx[f0 + 1] = sx + (p0 > 1);
                if (a.cols == 0) colh[f0 + 1] = 0u;
            }
            if (threadIdx.x == 0) {
                const RoundHdr h{base, tot_e, n_cols + tot_h + tot_l, tot_x | (n_cols << 16)};
                a.rhdr[(int64_t)(first + j) * a.n_parts + p] = h;
                if (j == 0) a.bhdr[b * a.n_parts + p] = BlockHdr{h, first, n_rounds, {0u, 0u}};
            }
        }
        __syncthreads();
        const bool dup = s_dup != 0u;  // (set before the count barrier above)
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            if (col[k] != 0xffffffffu) {
                // the feature's entries in earlier rows of the round
                uint32_t rank = 0u;
                if (!dup) {
                    const uint32_t w = tl[k] >> 5;
                    rank = (uint32_t)__popc(rowbits[w * kMaxISlab + col[k]] & ((1u << (tl[k] & 31u)) - 1u));
                    for (uint32_t u = 0; u < w; ++u) rank += (uint32_t)__popc(rowbits[u * kMaxISlab + col[k]]);
                } else {
                    rank = atomicAdd(&ccur[col[k]], 1u);
                }
                const uint32_t pos = base + cstart[col[k]] + rank;
                const uint32_t v = entry_value<VK>(a, val[k], c0 + threadIdx.x + k * kPlanThreads);
                if (f32)
                    static_cast<uint2 *>(a.ent)[pos] = make_uint2(tl[k], v);
                else if (colh[col[k]])  // a column feature's entry: bit 31, then its element of the Bt tile
                    static_cast<uint32_t *>(a.ent)[pos] =
                        0x80000000u | (((colh[col[k]] - 1) * (uint32_t)kMPitch + tl[k]) << 16) | (v & 0xffffu);
                else
                    static_cast<uint32_t *>(a.ent)[pos] = (tl[k] << 16) | (v & 0xffffu);
            }
        }
        for (int c = threadIdx.x; c < ni; c += kPlanThreads) {
            const uint32_t n = cnt[c], hc = colh[c];
            if (hc) {
                a.task[base + hc - 1] = make_uint2((uint32_t)c, 0u);
                continue;
            }
            const uint32_t npc = div_small(n + piece - 1, piece, inv_piece);
            const uint32_t tb = base + n_cols;  // pieces follow the column records
            if (npc == 1) a.task[tb + lstart[c]] = make_uint2((uint32_t)c | (kDirect << 16), (cstart[c] << 8) | n);
            if (npc < 2) continue;
            for (uint32_t pc = 0; pc < npc; ++pc) {
                const uint32_t len = min(piece, n - pc * piece);
                a.task[tb + hstart[c] + pc] =
                    make_uint2((uint32_t)c | ((hstart[c] + pc) << 16), ((cstart[c] + pc * piece) << 8) | len);
            }
            a.heavy[base + hidx[c]] = make_uint2((uint32_t)c | (hstart[c] << 16), npc);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ the streaming pass
struct FusedArgs {
    const void *g, *coeff, *q;
    int64_t rows, d_out, d_in;
    int rank;
    const float *scale;
    int bits;
    int64_t nnz;
    const void *ent;
    const uint2 *task;
    const uint2 *heavy;
    const RoundHdr *rhdr;
    const BlockHdr *bhdr;
    int64_t n_slabs, n_parts, i_span;  // i_span: input features per part (<= kMaxISlab)
    int vec_ok;                        // G rows allow whole-vector loads
    int c_vec;                         // C rows are exactly R wide and aligned for vector loads
    int out_vec_ok;                    // dW rows are 16-byte aligned (Conv1D layout stores)
    int transposed;
    void *dw;
    int dw_dt;
    void *dbias;
    int db_dt;
};

// Shared-memory carve-up of k_dw_fused (byte offsets).
template <int DT, int R>
struct FusedLds {
    using C = GradCfg<DT, R>;
    using T = typename C::T;
    static constexpr size_t ent_bytes = C::k16 ? 4 : 8;
    static constexpr size_t s_acc = 0;                                               // [1024][16] f32
    static constexpr size_t s_gtile = s_acc + (size_t)kMaxISlab * kAccPitch * 4;     // [TB + 1][16] T
    static constexpr size_t s_ent = s_gtile + (size_t)(C::TB + 1) * kOSlab * sizeof(T);  // [ROUND]
    static constexpr size_t s_task = s_ent + (size_t)C::ROUND * ent_bytes;           // [kTaskCap]
    static constexpr size_t s_heavy = s_task + (size_t)kTaskCap * 8;                 // [kHeavyCap]
    static constexpr size_t s_slot = s_heavy + (size_t)kHeavyCap * 8;                // [kSlotCap][16]
    static constexpr size_t s_hdr = s_slot + (size_t)kSlotCap * kOSlab * 4;        // [kHdrRing] BlockHdr
    static constexpr size_t end = s_hdr + (size_t)kHdrRing * sizeof(BlockHdr);
    static constexpr int NPASS = C::NV > 36 ? 4 : 2;  // M reduction passes (LDS holds NV / NPASS per thread)
    static constexpr int HALF = (C::NV + NPASS - 1) / NPASS;
    static constexpr size_t red_end = s_gtile + ((size_t)kBwdThreads * HALF + (size_t)8 * C::OG * HALF +
                                                 (size_t)kOSlab * (R + 1)) * 4;
    static constexpr size_t bytes = end > red_end ? end : red_end;
};

// A round's plan data held in registers between its load and its copy into LDS.
template <typename E, int EPT>
struct Staged {
    E ent[EPT];
    uint2 task[kTaskPT];
    uint2 heavy;
};

// FAST: every G and C row access is a whole aligned vector and the slab lies inside d_out, so
// each load is one unconditional instruction from a clamped row (rows past the matrix are
// zeroed where the values are used).  A load whose result is merged from divergent paths would
// be waited for at once; these are waited for only where they are consumed, a block later.
template <int DT, int R, bool FAST>
__global__ __launch_bounds__(kBwdThreads) void k_dw_fused(FusedArgs a)
{
    using C = GradCfg<DT, R>;
    using T = typename C::T;
    using L = FusedLds<DT, R>;
    constexpr int OT = C::OT, OG = C::OG, TB = C::TB, VB = C::VB, NW = Vec<C::VB>::n, CW = C::CW;
    constexpr int ROUND = C::ROUND, EPT = C::EPT;
    constexpr bool K16 = C::k16;
    using E = typename std::conditional<K16, uint32_t, uint2>::type;  // plan entry
    using Stage = Staged<E, EPT>;
    constexpr int NGRP = C::NGRP;

    extern __shared__ float lds[];
    char *base = reinterpret_cast<char *>(lds);
    float *acc = reinterpret_cast<float *>(base + L::s_acc);
    T *gtile = reinterpret_cast<T *>(base + L::s_gtile);
    E *l_ent = reinterpret_cast<E *>(base + L::s_ent);
    uint2 *l_task = reinterpret_cast<uint2 *>(base + L::s_task);
    uint2 *l_heavy = reinterpret_cast<uint2 *>(base + L::s_heavy);
    float *l_slot = reinterpret_cast<float *>(base + L::s_slot);
    float *mred = reinterpret_cast<float *>(base + L::s_gtile);  // reused after the stream
    BlockHdr *l_hdr = reinterpret_cast<BlockHdr *>(base + L::s_hdr);

    // workgroup -> (o-slab, part); consecutive logical ids land on the same XCD (ids are dealt
    // round-robin over 8 XCDs), so the parts of a slab and neighbouring slabs share an L2
    const int64_t nwg = a.n_slabs * a.n_parts;
    int64_t lid = blockIdx.x;
    if (nwg % 8 == 0) lid = (int64_t)(blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int64_t slab = lid / a.n_parts, part = lid - slab * a.n_parts;
    const int64_t o0 = slab * kOSlab;
    const int64_t i0 = part * a.i_span;
    const int ni = (int)(min(i0 + a.i_span, a.d_in) - i0);

    const int og = threadIdx.x % OG, tp = threadIdx.x / OG;
    const int64_t ob = o0 + og * OT;
    const bool o_ok = FAST || ob < a.d_out;
    const bool vec_ok = a.vec_ok != 0;
    const T *g = static_cast<const T *>(a.g);
    const T *coeff = static_cast<const T *>(a.coeff);
    const bool sparse = a.nnz > 0;
    const float qscale = (sparse && a.bits) ? a.scale[0] : 1.f;

    for (int i = threadIdx.x; i < ni * kAccPitch; i += kBwdThreads) acc[i] = 0.f;
    for (int i = threadIdx.x; i < kOSlab; i += kBwdThreads) gtile[TB * kOSlab + i] = T{};  // zero row

    float m[OT][R + 1];
#pragma unroll
    for (int o = 0; o < OT; ++o)
#pragma unroll
        for (int j = 0; j <= R; ++j) m[o][j] = 0.f;

    auto load_c = [&](int64_t t, uint32_t (&x)[CW]) {
#pragma unroll
        for (int k = 0; k < CW; ++k) x[k] = 0u;
        if (t >= a.rows) return;
        if (a.c_vec) {
            const char *p = reinterpret_cast<const char *>(coeff + t * R);
            if constexpr (CW % 4 == 0) {
#pragma unroll
                for (int k = 0; k < CW / 4; ++k) load_words<16>(p + 16 * k, x + 4 * k);
            } else {
                load_words<8>(p, x);
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < R; ++j) {
            if (j < a.rank) {
                if constexpr (K16) {
                    x[j / 2] |= (uint32_t)coeff[t * a.rank + j] << (16 * (j & 1));
                } else {
                    x[j] = __float_as_uint(coeff[t * a.rank + j]);
                }
            }
        }
    };

    // What a block needs is loaded ahead into register rings (slot d of a ring holds block
    // blk + d at the top of iteration blk): G rows GD blocks ahead, C rows and the block's first
    // plan round PD blocks ahead; the block headers that locate those rounds two further blocks.
    constexpr int PD = C::PD, GD = C::GD;
    uint32_t wq[GD][2][NW], xq[PD][2][CW];
    auto load_grows = [&](int64_t blk, uint32_t (&w)[2][NW]) {
        const int64_t t = blk * TB + 2 * tp;
        if constexpr (FAST) {
            load_words<VB>(g + min(t, a.rows - 1) * a.d_out + ob, w[0]);
            load_words<VB>(g + min(t + 1, a.rows - 1) * a.d_out + ob, w[1]);
        } else {
            load_g<DT, VB>(g + t * a.d_out, ob, a.d_out, o_ok && t < a.rows, vec_ok, w[0]);
            load_g<DT, VB>(g + (t + 1) * a.d_out, ob, a.d_out, o_ok && t + 1 < a.rows, vec_ok, w[1]);
        }
    };
    auto load_crows = [&](int64_t blk, uint32_t (&x)[2][CW]) {
        const int64_t t = blk * TB + 2 * tp;
        if constexpr (FAST) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const char *p = reinterpret_cast<const char *>(coeff + min(t + r, a.rows - 1) * R);
                if constexpr (CW % 4 == 0) {
#pragma unroll
                    for (int k = 0; k < CW / 4; ++k) load_words<16>(p + 16 * k, x[r] + 4 * k);
                } else {
                    load_words<8>(p, x[r]);
                }
            }
        } else {
            load_c(t, x[0]);
            load_c(t + 1, x[1]);
        }
    };

    // plan data of a round: global -> registers -> LDS (round sizes are bounded by the planner;
    // the clamps only keep a malformed plan inside the buffers)
    auto load_stage = [&](Stage &st, const RoundHdr &h) {
        const uint32_t ne = min(h.n_ent, (uint32_t)ROUND), nt = min(h.n_task, (uint32_t)kTaskCap);
        const E *ge = static_cast<const E *>(a.ent) + h.base;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t e = threadIdx.x + k * kBwdThreads;
            st.ent[k] = e < ne ? ge[e] : E{};
        }
#pragma unroll
        for (int k = 0; k < kTaskPT; ++k) {
            const uint32_t e = threadIdx.x + k * kBwdThreads;
            st.task[k] = e < nt ? a.task[h.base + e] : make_uint2(0u, 0u);
        }
        st.heavy = threadIdx.x < min(h.n_heavy & 0xffffu, (uint32_t)kHeavyCap) ? a.heavy[h.base + threadIdx.x]
                                                                     : make_uint2(0u, 0u);
    };
    auto store_stage = [&](const Stage &st) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) l_ent[threadIdx.x + k * kBwdThreads] = st.ent[k];
#pragma unroll
        for (int k = 0; k < kTaskPT; ++k)
            if (threadIdx.x + k * kBwdThreads < kTaskCap) l_task[threadIdx.x + k * kBwdThreads] = st.task[k];
        if (threadIdx.x < kHeavyCap) l_heavy[threadIdx.x] = st.heavy;
    };

    // One piece's entries [e_lo, e_lo + n) accumulated into pa (this thread's OT outputs).  Four
    // entries per batch with no branch inside a batch, so their loads issue together; entries past
    // the piece are redirected to the all-zero G row TB with a zero value, which adds exactly 0.
    auto piece_batch = [&](uint32_t e, uint32_t e_lo, uint32_t n, float (&pa)[OT]) {
        const uint32_t last = e_lo + (n ? n - 1 : 0u);
        E w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const E x = l_ent[min(e + u, last) % ROUND];
            const bool valid = e + u < e_lo + n;
            if constexpr (K16) w[u] = valid ? x : (uint32_t)TB << 16;
            else w[u] = valid ? x : make_uint2((uint32_t)TB, 0u);
        }
        uint32_t gw[4][NW];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t row;
            if constexpr (K16) row = w[u] >> 16;
            else row = w[u].x;
            load_words<VB>(gtile + min(row, (uint32_t)TB) * kOSlab + og * OT, gw[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (K16) {
                const uint32_t vlo = w[u] & 0xffffu, vhi = w[u] << 16;  // (v, 0) and (0, v)
#pragma unroll
                for (int k = 0; k < NW; ++k) {
                    pa[2 * k] = dot2<DT>(gw[u][k], vlo, pa[2 * k]);
                    pa[2 * k + 1] = dot2<DT>(gw[u][k], vhi, pa[2 * k + 1]);
                }
            } else {
                const float v = __uint_as_float(w[u].y);
#pragma unroll
                for (int o = 0; o < OT; ++o) pa[o] = fmaf(__uint_as_float(gw[u][o]), v, pa[o]);
            }
        }
    };
    // A piece's sum: added (scaled) into S, or parked in its slot when the feature has several.
    auto flush = [&](uint2 td, const float (&pa)[OT]) {
        const uint32_t c = td.x & 0xffffu, slot = td.x >> 16;
        if (c >= (uint32_t)ni) return;
        if (slot == kDirect) {
            if constexpr (OT >= 4) {
#pragma unroll
                for (int q4 = 0; q4 < OT / 4; ++q4) {
                    float4 *dst = reinterpret_cast<float4 *>(acc + s_index((int)c, og * OT + 4 * q4));
                    float4 v = *dst;
                    v.x = fmaf(pa[4 * q4], qscale, v.x);
                    v.y = fmaf(pa[4 * q4 + 1], qscale, v.y);
                    v.z = fmaf(pa[4 * q4 + 2], qscale, v.z);
                    v.w = fmaf(pa[4 * q4 + 3], qscale, v.w);
                    *dst = v;
                }
            } else {
#pragma unroll
                for (int o = 0; o < OT; ++o) {
                    float *dst = acc + s_index((int)c, og * OT + o);
                    *dst = fmaf(pa[o], qscale, *dst);
                }
            }
        } else if (slot < (uint32_t)kSlotCap) {
            float *dst = l_slot + slot * kOSlab + og * OT;
#pragma unroll
            for (int o = 0; o < OT; ++o) dst[o] = pa[o];
        }
    };

    // Sum the round's pieces (staged in LDS, the G tile complete) into S.  Group g (OG threads)
    // takes pieces g, g + NGRP, g + 2 NGRP, ...
    auto run_round = [&](const RoundHdr &h) {
        const uint32_t nt = min(h.n_task, (uint32_t)kTaskCap), nh = min(h.n_heavy & 0xffffu, (uint32_t)kHeavyCap);
        if (o_ok) {
            for (uint32_t tk = threadIdx.x / OG; tk < nt; tk += NGRP) {
                const uint2 td = l_task[tk];
                const uint32_t lo = td.y >> 8, n = td.y & 255u;
                float pa[OT];
#pragma unroll
                for (int o = 0; o < OT; ++o) pa[o] = 0.f;
                for (uint32_t k = 0; k < n; k += 4) piece_batch(lo + k, lo, n, pa);
                flush(td, pa);
            }
        }
        __syncthreads();
        // features cut into several pieces: their partial sums added in piece order
        for (uint32_t w = threadIdx.x; w < nh * kOSlab; w += kBwdThreads) {
            const uint2 hd = l_heavy[w / kOSlab];
            const uint32_t o = w % kOSlab, c = hd.x & 0xffffu, s0 = hd.x >> 16;
            if (c < (uint32_t)ni && s0 + hd.y <= (uint32_t)kSlotCap) {
                // eight interleaved partial sums (independent loads), combined in a fixed order
                float s8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                uint32_t k = 0;
                for (; k + 8 <= hd.y; k += 8) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) s8[u] += l_slot[(s0 + k + u) * kOSlab + o];
                }
                for (; k < hd.y; ++k) s8[0] += l_slot[(s0 + k) * kOSlab + o];
                const float sum = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
                acc[s_index((int)c, (int)o)] += sum * qscale;
            }
        }
        __syncthreads();
    };

    const int64_t n_blocks = (a.rows + TB - 1) / TB;
    // Block headers live in an LDS ring of kHdrRing blocks (a uniform value loaded from global
    // memory in the loop would be read into scalar registers, and so waited for, at once).  The
    // ring starts with blocks [0, kHdrRing); every kHdrRing / 2 blocks the half just finished is
    // refilled with the blocks kHdrRing / 2 further on.
    auto hdr_fill = [&](int64_t b0, int64_t count) {
        for (int64_t i = threadIdx.x; i < count; i += kBwdThreads) {
            const int64_t b = b0 + i;
            l_hdr[b % kHdrRing] = (sparse && b < n_blocks) ? a.bhdr[b * a.n_parts + part] : BlockHdr{};
        }
    };
    auto read_hdr = [&](int64_t b) { return b < n_blocks ? l_hdr[b % kHdrRing] : BlockHdr{}; };
    hdr_fill(0, kHdrRing);
    __syncthreads();
    Stage sq[PD];
#pragma unroll
    for (int d = 0; d < GD; ++d) load_grows(d, wq[d]);  // rows past the matrix load as zero
#pragma unroll
    for (int d = 0; d < PD; ++d) load_crows(d, xq[d]);
#pragma unroll
    for (int d = 0; d < PD; ++d) {
        const BlockHdr h = read_hdr(d);
        if (h.n_rounds) load_stage(sq[d], h.r0);
    }
    for (int64_t blk = 0; blk < n_blocks; ++blk) {
        uint32_t ca[NW], cb[NW], ya[CW], yb[CW];
        const bool ra = !FAST || blk * TB + 2 * tp < a.rows, rb = !FAST || blk * TB + 2 * tp + 1 < a.rows;
#pragma unroll
        for (int k = 0; k < NW; ++k) { ca[k] = ra ? wq[0][0][k] : 0u; cb[k] = rb ? wq[0][1][k] : 0u; }
#pragma unroll
        for (int k = 0; k < CW; ++k) { ya[k] = ra ? xq[0][0][k] : 0u; yb[k] = rb ? xq[0][1][k] : 0u; }
        const BlockHdr bh = read_hdr(blk);
        if (sparse) {  // this block's G rows and first round of plan data into LDS
            uint32_t *da = reinterpret_cast<uint32_t *>(gtile + (2 * tp) * kOSlab + og * OT);
            uint32_t *db = reinterpret_cast<uint32_t *>(gtile + (2 * tp + 1) * kOSlab + og * OT);
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                da[k] = ca[k];
                db[k] = cb[k];
            }
            if (bh.n_rounds) store_stage(sq[0]);
        }
        // ---- low rank: m[o][j] += G[t][o] C[t][j] + G[t+1][o] C[t+1][j];  m[o][R] += G[t][o] + G[t+1][o]
        if constexpr (K16) {
            uint32_t pr[OT];  // (G[t][o], G[t+1][o]) pairs
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                pr[2 * k] = __builtin_amdgcn_perm(cb[k], ca[k], 0x05040100u);
                pr[2 * k + 1] = __builtin_amdgcn_perm(cb[k], ca[k], 0x07060302u);
            }
            uint32_t cv[R];  // (C[t][j], C[t+1][j]) pairs
#pragma unroll
            for (int k = 0; k < CW; ++k) {
                cv[2 * k] = __builtin_amdgcn_perm(yb[k], ya[k], 0x05040100u);
                cv[2 * k + 1] = __builtin_amdgcn_perm(yb[k], ya[k], 0x07060302u);
            }
            const uint32_t ones = DT == STACR_DTYPE_BF16 ? 0x3f803f80u : 0x3c003c00u;
#pragma unroll
            for (int o = 0; o < OT; ++o) {
#pragma unroll
                for (int j = 0; j < R; ++j) m[o][j] = dot2<DT>(pr[o], cv[j], m[o][j]);
                m[o][R] = dot2<DT>(pr[o], ones, m[o][R]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const float c0 = __uint_as_float(ya[j]), c1 = __uint_as_float(yb[j]);
#pragma unroll
                for (int o = 0; o < OT; ++o)
                    m[o][j] = fmaf(__uint_as_float(cb[o]), c1, fmaf(__uint_as_float(ca[o]), c0, m[o][j]));
            }
#pragma unroll
            for (int o = 0; o < OT; ++o) m[o][R] += __uint_as_float(ca[o]) + __uint_as_float(cb[o]);
        }
        // advance the rings after this block's low-rank arithmetic, so the registers it consumed are
        // free for the next block's loads, which overlap this block's sparse work
#pragma unroll
        for (int d = 0; d + 1 < GD; ++d)
#pragma unroll
            for (int k = 0; k < NW; ++k) { wq[d][0][k] = wq[d + 1][0][k]; wq[d][1][k] = wq[d + 1][1][k]; }
#pragma unroll
        for (int d = 0; d + 1 < PD; ++d) {
#pragma unroll
            for (int k = 0; k < CW; ++k) { xq[d][0][k] = xq[d + 1][0][k]; xq[d][1][k] = xq[d + 1][1][k]; }
            sq[d] = sq[d + 1];
        }
        // Loads issue in the order they are consumed: the memory counter retires in issue order,
        // so waiting for the next block's C rows and plan data must not also wait for G rows
        // that are only needed GD blocks from now.  (FAST loads past the last block re-read the
        // last rows and are never used.)
        if (FAST || blk + PD < n_blocks) load_crows(blk + PD, xq[PD - 1]);
        {
            const BlockHdr hn = read_hdr(blk + PD);
            if (hn.n_rounds) load_stage(sq[PD - 1], hn.r0);
        }
        if (FAST || blk + GD < n_blocks) load_grows(blk + GD, wq[GD - 1]);
        if (blk % (kHdrRing / 2) == 0 && blk > 0) {  // refill the half of the ring just finished
            __syncthreads();
            hdr_fill(blk + kHdrRing / 2, kHdrRing / 2);
            __syncthreads();
        }
        if (!sparse || bh.n_rounds == 0) continue;
        __syncthreads();  // G tile and first round staged
        run_round(bh.r0);
        for (uint32_t j = 1; j < bh.n_rounds; ++j) {  // blocks with more than ROUND entries
            const RoundHdr h = a.rhdr[(int64_t)(bh.first_round + j) * a.n_parts + part];
            Stage tmp;
            load_stage(tmp, h);
            store_stage(tmp);
            __syncthreads();
            run_round(h);
        }
        // (run_round ends with a barrier, so the next block may overwrite the tile and stage)
    }
    __syncthreads();

    // ---- reduce m over the TP threads that share an output group, in a fixed order.
    // NPASS slices of the per-thread values in turn: every thread parks its half in LDS, 8 threads
    // per output sum TP/8 rows each, one thread per output adds the 8 partial sums.
    constexpr int HALF = L::HALF;
    constexpr int TP = C::TP;
    float *psum = mred + kBwdThreads * HALF;  // [8][OG * HALF]
    float *mfin = psum + 8 * OG * HALF;       // final M: [kOSlab][R + 1]
    for (int h = 0; h < L::NPASS; ++h) {
        const int v0 = h * HALF, v1 = min(C::NV, v0 + HALF);
#pragma unroll
        for (int v = 0; v < C::NV; ++v)
            if (v >= v0 && v < v1) mred[threadIdx.x * HALF + (v - v0)] = m[v / (R + 1)][v % (R + 1)];
        __syncthreads();
        const int nout = OG * (v1 - v0);
        for (int w = threadIdx.x; w < nout * 8; w += kBwdThreads) {
            const int out = w % nout, s = w / nout;
            const int oo = out % OG, vv = out / OG;
            float sum = 0.f;
            for (int p = s * (TP / 8); p < (s + 1) * (TP / 8); ++p) sum += mred[(p * OG + oo) * HALF + vv];
            psum[s * nout + out] = sum;
        }
        __syncthreads();
        for (int out = threadIdx.x; out < nout; out += kBwdThreads) {
            float sum = 0.f;
            for (int s = 0; s < 8; ++s) sum += psum[s * nout + out];
            const int oo = out % OG, v = v0 + out / OG;
            mfin[(oo * OT + v / (R + 1)) * (R + 1) + v % (R + 1)] = sum;
        }
        __syncthreads();
    }

    // ---- epilogue: dW tile = M Q^T + S, one rounding to the weight dtype; dbias from M[:, R].
    // A thread takes one input feature i (its Q row in registers) and all 16 outputs.
    const T *q = static_cast<const T *>(a.q);
    const bool vec_out = a.transposed && a.out_vec_ok && o0 + kOSlab <= a.d_out;
    static_assert(kMaxISlab <= kBwdThreads, "one input feature per thread");
    if (const int ii = threadIdx.x; ii < ni) {
        const int64_t i = i0 + ii;
        float qr[R];
#pragma unroll
        for (int j = 0; j < R; ++j) qr[j] = j < a.rank ? Act<DT>::ld(q[i * a.rank + j]) : 0.f;
        float out[kOSlab];
#pragma unroll
        for (int oo = 0; oo < kOSlab; ++oo) {
            float s = acc[s_index(ii, oo)];
#pragma unroll
            for (int j = 0; j < R; ++j) s = fmaf(mfin[oo * (R + 1) + j], qr[j], s);
            out[oo] = s;
        }
        if (vec_out && a.dw_dt != STACR_DTYPE_F32) {
            // Conv1D layout [d_in, d_out]: the slab's 16 outputs of feature i are 32 contiguous bytes
            const bool bf = a.dw_dt == STACR_DTYPE_BF16;
            uint32_t wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                wv[k] = bf ? (f_to_bf16_bits(out[2 * k]) | (f_to_bf16_bits(out[2 * k + 1]) << 16))
                           : (f_to_f16_bits(out[2 * k]) | (f_to_f16_bits(out[2 * k + 1]) << 16));
            uint4 *dst = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.dw) + i * a.d_out + o0);
            dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
            dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
        } else if (vec_out) {
            float4 *dst = reinterpret_cast<float4 *>(static_cast<float *>(a.dw) + i * a.d_out + o0);
#pragma unroll
            for (int k = 0; k < 4; ++k) dst[k] = make_float4(out[4 * k], out[4 * k + 1], out[4 * k + 2], out[4 * k + 3]);
        } else {
#pragma unroll
            for (int oo = 0; oo < kOSlab; ++oo)
                if (o0 + oo < a.d_out)
                    store_any(a.dw, a.dw_dt, a.transposed ? i * a.d_out + o0 + oo : (o0 + oo) * a.d_in + i, out[oo]);
        }
    }
    if (a.dbias && part == 0)
        for (int oo = threadIdx.x; oo < kOSlab; oo += kBwdThreads)
            if (o0 + oo < a.d_out) store_any(a.dbias, a.db_dt, o0 + oo, mfin[oo * (R + 1) + R]);
}

// ------------------------------------------------------------------ the matrix-core streaming pass
// For 16-bit G, rank 4 or 8 and aligned rows (the FAST conditions): the same plan and the same
// piece path as k_dw_fused for the light features, while the low-rank product, dbias and each
// round's column features (the features with the most entries in the block) go through
// v_mfma_f32_16x16x32 (bf16 / f16 operands, fp32 accumulation):
//     D[o][j] += sum_t G[t][o] B[t][j],  32 token rows per instruction,
// with the operands read row-contiguously from LDS copies of the tiles, G transposed (Gt[o][t]) and
// the B columns (Bt[j][t]):
//   * fixed tile, columns C[:, 0..R) and a column of ones (its D column is dbias): one instruction
//     per wave per block (wave w takes rows 32w..32w+31), partial sums kept in registers across
//     blocks and added over the 16 waves once, in wave order, at the end;
//   * column tiles, up to 32 column features whose integer codes are scattered into a zeroed
//     Bt tile: waves 0 and 1 each run the 16 instructions of one 16-column tile per round, add
//     each column's sums (scaled) into S, and the tile is zeroed again after the round.

template <int R>
struct MfmaLds {
    static constexpr size_t s_acc = 0;                                            // [1024][16] f32
    static constexpr size_t s_gr = s_acc + (size_t)kMaxISlab * kAccPitch * 4;      // [kMGRows][16] row-major
    static constexpr size_t s_bc = s_gr + (size_t)kMGRows * kOSlab * 2;            // [R][kMPitch]
    static constexpr size_t s_bh = s_bc + (size_t)R * kMPitch * 2;                 // [kMCols][kMPitch]
    static constexpr size_t s_ent = s_bh + (size_t)kMCols * kMPitch * 2;           // [kRoundMax] u32
    static constexpr size_t s_task = s_ent + (size_t)kRoundMax * 4;                // [kMTaskCap]
    static constexpr size_t s_heavy = s_task + (size_t)kMTaskCap * 8;              // [kHeavyCap]
    static constexpr size_t s_slot = s_heavy + (size_t)kHeavyCap * 8;              // [kMSlotCap][16] f32
    static constexpr size_t s_hdr = s_slot + (size_t)kMSlotCap * kOSlab * 4;       // [kMHdrRing]
    static constexpr size_t bytes = s_hdr + (size_t)kMHdrRing * sizeof(BlockHdr);
    // after the stream, over the tiles: per-wave partial fixed tiles [16][16][16] f32, then M
    static constexpr size_t s_red = s_gr;
    static constexpr size_t s_mfin = s_red + (size_t)16 * 256 * 4;
    static_assert(s_mfin + (size_t)kOSlab * (R + 1) * 4 <= s_ent, "reduction fits the tile region");
    static_assert(s_gr % 16 == 0 && s_bc % 16 == 0 && s_bh % 16 == 0 && (kMPitch * 2) % 16 == 0,
                  "16-byte operand rows");
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): four 16-bit values, transposed across each 16-lane group (see the
// matrix-core kernel's operand reads); the bits are moved unchanged, so it serves fp16 as well
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p)
{
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
    bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4 *)(p));
    return __builtin_bit_cast(uint2, v);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma_16x16x32(uint4 a, uint4 b, f32x4 c)
{
    if constexpr (DT == STACR_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(8))) __bf16 v8;
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    } else {
        typedef __attribute__((ext_vector_type(8))) _Float16 v8;
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    }
}

template <int DT, int R>
__global__ __launch_bounds__(kBwdThreads) void k_dw_fused_mfma(FusedArgs a)
{
    static_assert(DT != STACR_DTYPE_F32 && (R == 4 || R == 8), "16-bit G, rank 4 or 8");
    using L = MfmaLds<R>;
    constexpr int OT = 4, OG = kOSlab / OT, TP = kBwdThreads / OG, TB = kMTB;
    static_assert(2 * TP == TB, "two token rows per thread");
    constexpr int CQ = R / 4;  // 32-bit words of C a thread loads: columns CQ * 2 * (og >> 1) ..
    constexpr int ROUND = kRoundMax, EPT = ROUND / kBwdThreads;
    constexpr int NGRP = kBwdThreads / OG;
    constexpr uint32_t kOne = DT == STACR_DTYPE_BF16 ? 0x3f80u : 0x3c00u;

    extern __shared__ float lds[];
    char *base = reinterpret_cast<char *>(lds);
    float *acc = reinterpret_cast<float *>(base + L::s_acc);
    uint16_t *gr = reinterpret_cast<uint16_t *>(base + L::s_gr);
    uint16_t *bc = reinterpret_cast<uint16_t *>(base + L::s_bc);
    uint16_t *bh = reinterpret_cast<uint16_t *>(base + L::s_bh);
    uint32_t *l_ent = reinterpret_cast<uint32_t *>(base + L::s_ent);
    uint2 *l_task = reinterpret_cast<uint2 *>(base + L::s_task);
    uint2 *l_heavy = reinterpret_cast<uint2 *>(base + L::s_heavy);
    float *l_slot = reinterpret_cast<float *>(base + L::s_slot);
    BlockHdr *l_hdr = reinterpret_cast<BlockHdr *>(base + L::s_hdr);

    // workgroup -> (o-slab, part), consecutive logical ids on one XCD (as in k_dw_fused)
    const int64_t nwg = a.n_slabs * a.n_parts;
    int64_t lid = blockIdx.x;
    if (nwg % 8 == 0) lid = (int64_t)(blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int64_t slab = lid / a.n_parts, part = lid - slab * a.n_parts;
    const int64_t o0 = slab * kOSlab;
    const int64_t i0 = part * a.i_span;
    const int ni = (int)(min(i0 + a.i_span, a.d_in) - i0);
    const int og = threadIdx.x % OG, tp = threadIdx.x / OG;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint16_t *g = static_cast<const uint16_t *>(a.g);
    const uint16_t *coeff = static_cast<const uint16_t *>(a.coeff);
    const bool sparse = a.nnz > 0;
    const float qscale = (sparse && a.bits) ? a.scale[0] : 1.f;

    for (int i = threadIdx.x; i < ni * kAccPitch; i += kBwdThreads) acc[i] = 0.f;
    if (threadIdx.x < kOSlab) gr[TB * kOSlab + threadIdx.x] = 0;  // the zero row
    for (int i = threadIdx.x; i < kMCols * kMPitch / 8; i += kBwdThreads)
        reinterpret_cast<uint4 *>(bh)[i] = make_uint4(0u, 0u, 0u, 0u);

    const int64_t n_blocks = (a.rows + TB - 1) / TB;
    auto hdr_fill = [&](int64_t b0, int64_t count) {
        for (int64_t i = threadIdx.x; i < count; i += kBwdThreads) {
            const int64_t b = b0 + i;
            l_hdr[b % kMHdrRing] = (sparse && b < n_blocks) ? a.bhdr[b * a.n_parts + part] : BlockHdr{};
        }
    };
    auto read_hdr = [&](int64_t b) { return b < n_blocks ? l_hdr[b % kMHdrRing] : BlockHdr{}; };

    // unconditional loads from clamped rows (the rows past the matrix are zeroed where used): a
    // uniform base row rb = min(block start, rows - 1) and a 32-bit row offset clamped to the
    // last row, so the address arithmetic per thread is 32-bit
    const uint32_t dout32 = (uint32_t)a.d_out;
    auto block_base = [&](int64_t blk, int64_t &rb, uint32_t &lim) {
        rb = min(blk * TB, a.rows - 1);
        lim = (uint32_t)min(a.rows - 1 - rb, (int64_t)TB);
    };
    auto load_grows = [&](int64_t blk, uint32_t (&w)[2][2]) {
        int64_t rb;
        uint32_t lim;
        block_base(blk, rb, lim);
        const uint16_t *gb = g + rb * a.d_out + o0;
        load_words<8>(gb + min((uint32_t)(2 * tp), lim) * dout32 + og * OT, w[0]);
        load_words<8>(gb + min((uint32_t)(2 * tp + 1), lim) * dout32 + og * OT, w[1]);
    };
    // thread (tp, og) loads C row 2 tp + (og & 1), columns [R / 2 (og >> 1), R / 2 (og >> 1) + R / 2)
    auto load_crow = [&](int64_t blk, uint32_t (&x)[CQ]) {
        int64_t rb;
        uint32_t lim;
        block_base(blk, rb, lim);
        load_words<4 * CQ>(coeff + rb * R + min((uint32_t)(2 * tp + (og & 1)), lim) * R + (R / 2) * (og >> 1), x);
    };
    struct StageM {
        uint32_t ent[EPT];
        uint2 task[kMTaskPT];
        uint2 heavy;
    };
    auto load_stage = [&](StageM &st, const RoundHdr &h) {
        const uint32_t ne = min(h.n_ent, (uint32_t)ROUND), nt = min(h.n_task, (uint32_t)kMTaskCap);
        const uint32_t *ge = static_cast<const uint32_t *>(a.ent) + h.base;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t e = threadIdx.x + k * kBwdThreads;
            st.ent[k] = e < ne ? ge[e] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kMTaskPT; ++k) {
            const uint32_t e = threadIdx.x + k * kBwdThreads;
            st.task[k] = e < nt ? a.task[h.base + e] : make_uint2(0u, 0u);
        }
        st.heavy = threadIdx.x < min(h.n_heavy & 0xffffu, (uint32_t)kHeavyCap) ? a.heavy[h.base + threadIdx.x]
                                                                               : make_uint2(0u, 0u);
    };
    // plan data into LDS, and each column feature's codes into its (zeroed) Bt row
    auto store_stage = [&](const StageM &st) {
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t w = st.ent[k];
            l_ent[threadIdx.x + k * kBwdThreads] = w;
            if (w >> 31) bh[min((w >> 16) & 0x7fffu, (uint32_t)(kMCols * kMPitch - 1))] = (uint16_t)w;
        }
#pragma unroll
        for (int k = 0; k < kMTaskPT; ++k)
            if (threadIdx.x + k * kBwdThreads < kMTaskCap) l_task[threadIdx.x + k * kBwdThreads] = st.task[k];
        if (threadIdx.x < kHeavyCap) l_heavy[threadIdx.x] = st.heavy;
    };

    // Matrix-core operand Gᵀ[o][t0 + 8 (lane / 16) .. + 7], o = lane % 16, from the row-major tile by
    // two transposing reads (ds_read_b64_tr_b16): in a 16-lane group, lane n receives value j from
    // position n % 4 of the 8 bytes lane 4 j + n / 4 addresses (checked on the GPU), so lane m
    // addresses row r0 + m / 4, outputs 4 (m % 4) .. + 3, and lane n gets G[r0 + j][n], j = 0..3.
    auto g_operand = [&](int t0) -> uint4 {
        const uint16_t *p = gr + (t0 + 8 * (lane >> 4) + ((lane & 15) >> 2)) * kOSlab + (lane & 3) * 4;
        const uint2 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * kOSlab);
        return make_uint4(lo.x, lo.y, hi.x, hi.y);
    };

    // One piece's entries [e_lo, e_lo + n) into pa (this thread's 4 outputs), G from the tile: four
    // entries per batch; entries past the piece read the zero column TB with value 0.
    auto piece_batch = [&](uint32_t e, uint32_t e_lo, uint32_t n, float (&pa)[OT]) {
        const uint32_t last = e_lo + (n ? n - 1 : 0u);
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t x = l_ent[min(e + u, last) % ROUND];
            w[u] = e + u < e_lo + n ? x : (uint32_t)TB << 16;
        }
        uint32_t gw[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // G[t][og * 4 .. + 3]: (o0, o0 + 1) and (o0 + 2, o0 + 3) as the dot products' pairs
            const uint2 g2 = *reinterpret_cast<const uint2 *>(gr + min((w[u] >> 16) & 0x3ffu, (uint32_t)TB) * kOSlab + og * OT);
            gw[u][0] = g2.x;
            gw[u][1] = g2.y;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t vlo = w[u] & 0xffffu, vhi = w[u] << 16;  // (v, 0) and (0, v)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                pa[2 * k] = dot2<DT>(gw[u][k], vlo, pa[2 * k]);
                pa[2 * k + 1] = dot2<DT>(gw[u][k], vhi, pa[2 * k + 1]);
            }
        }
    };
    auto flush = [&](uint2 td, const float (&pa)[OT]) {
        const uint32_t c = td.x & 0xffffu, slot = td.x >> 16;
        if (c >= (uint32_t)ni) return;
        if (slot == kDirect) {
            float4 *dst = reinterpret_cast<float4 *>(acc + s_index((int)c, og * OT));
            float4 v = *dst;
            v.x = fmaf(pa[0], qscale, v.x);
            v.y = fmaf(pa[1], qscale, v.y);
            v.z = fmaf(pa[2], qscale, v.z);
            v.w = fmaf(pa[3], qscale, v.w);
            *dst = v;
        } else if (slot < (uint32_t)kMSlotCap) {
            float *dst = l_slot + slot * kOSlab + og * OT;
#pragma unroll
            for (int o = 0; o < OT; ++o) dst[o] = pa[o];
        }
    };

    // A round's features split into several pieces have their partial sums in the slots.  Thread
    // t (t < 16 x the round's split features) adds feature t / 16's output t % 16 into S; it runs
    // after the round's last barrier and before the next round's pieces write the slots again
    // (the planner keeps split features <= kMSlotCap / 2, so one item a thread suffices).
    uint2 pend_hd = make_uint2(0xffffu, 0u);  // feature 0xffff: nothing pending
    auto combine_pending = [&]() {
        const uint32_t o = threadIdx.x % kOSlab, c = pend_hd.x & 0xffffu, s0 = pend_hd.x >> 16;
        if (c < (uint32_t)ni && s0 + pend_hd.y <= (uint32_t)kMSlotCap) {
            float s8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            uint32_t k = 0;
            for (; k + 8 <= pend_hd.y; k += 8) {
#pragma unroll
                for (int u = 0; u < 8; ++u) s8[u] += l_slot[(s0 + k + u) * kOSlab + o];
            }
            for (; k < pend_hd.y; ++k) s8[0] += l_slot[(s0 + k) * kOSlab + o];
            const float sum = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
            acc[s_index((int)c, (int)o)] += sum * qscale;
        }
        pend_hd = make_uint2(0xffffu, 0u);
    };

    // One round: the column tile (wave 0) and the pieces, then the split features' partial sums.
    auto run_round = [&](const RoundHdr &h) {
        const uint32_t ncol = min(h.n_heavy >> 16, (uint32_t)kMCols);
        const uint32_t nt = min(h.n_task, (uint32_t)kMTaskCap), nh = min(h.n_heavy & 0xffffu, (uint32_t)kHeavyCap);
        if (wave < kMCols / 16 && ncol > (uint32_t)(16 * wave)) {  // wave w: columns 16 w .. 16 w + 15
            const int jj = lane & 15, k8 = 8 * (lane >> 4), cj = 16 * wave + jj;
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < TB / 32; ++s) {
                const uint4 av = g_operand(32 * s);
                const uint4 bv = *reinterpret_cast<const uint4 *>(bh + cj * kMPitch + 32 * s + k8);
                d = mfma_16x16x32<DT>(av, bv, d);
            }
            // lane: column cj, outputs 4 (lane / 16) .. + 3
            if ((uint32_t)cj < ncol) {
                const uint32_t c = l_task[cj].x & 0xffffu;
                if (c < (uint32_t)ni) {
                    float4 *dst = reinterpret_cast<float4 *>(acc + s_index((int)c, 4 * (lane >> 4)));
                    float4 v = *dst;
                    v.x = fmaf(d[0], qscale, v.x);
                    v.y = fmaf(d[1], qscale, v.y);
                    v.z = fmaf(d[2], qscale, v.z);
                    v.w = fmaf(d[3], qscale, v.w);
                    *dst = v;
                }
            }
        }
        // pieces, group g taking pieces g, g + NGRP, ...; waves 0 and 1 (busy with the column
        // tiles) have the groups that come last
        const uint32_t grp = (uint32_t)(threadIdx.x / OG + NGRP - (kMCols / 16) * 64 / OG) % NGRP;
        for (uint32_t tk = ncol + grp; tk < nt; tk += NGRP) {
            const uint2 td = l_task[tk];
            const uint32_t lo = td.y >> 8, n = td.y & 255u;
            float pa[OT] = {0.f, 0.f, 0.f, 0.f};
            for (uint32_t k = 0; k < n; k += 4) piece_batch(lo + k, lo, n, pa);
            flush(td, pa);
        }
        __syncthreads();
        // the split features' partial sums are added after the next barrier (combine_pending),
        // by waves that wait there anyway; this keeps only the heavy record
        pend_hd = threadIdx.x < nh * kOSlab ? l_heavy[threadIdx.x / kOSlab] : make_uint2(0xffffu, 0u);
        for (uint32_t i = threadIdx.x; i < ncol * (kMPitch / 8); i += kBwdThreads)
            reinterpret_cast<uint4 *>(bh)[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
    };

    hdr_fill(0, kMHdrRing);
    __syncthreads();
    uint32_t wq[2][2], xq[CQ];
    StageM sq;
    load_grows(0, wq);
    load_crow(0, xq);
    {
        const BlockHdr h = read_hdr(0);
        if (h.n_rounds) load_stage(sq, h.r0);
    }
    f32x4 accf = {0.f, 0.f, 0.f, 0.f};
    for (int64_t blk = 0; blk < n_blocks; ++blk) {
        const int rem = (int)min(a.rows - blk * TB, (int64_t)TB);  // rows of this block (uniform, >= 1)
        const bool ra = 2 * tp < rem, rb = 2 * tp + 1 < rem;
        const bool rc = (og & 1) ? rb : ra;
        uint32_t ca[2], cb[2], yc[CQ];
#pragma unroll
        for (int k = 0; k < 2; ++k) { ca[k] = ra ? wq[0][k] : 0u; cb[k] = rb ? wq[1][k] : 0u; }
#pragma unroll
        for (int k = 0; k < CQ; ++k) yc[k] = rc ? xq[k] : 0u;
        const BlockHdr bh_ = read_hdr(blk), hn = read_hdr(blk + 1);
        // G rows 2 tp and 2 tp + 1, outputs og * 4 .. + 3, into the row-major tile
        *reinterpret_cast<uint2 *>(gr + (2 * tp) * kOSlab + og * OT) = make_uint2(ca[0], ca[1]);
        *reinterpret_cast<uint2 *>(gr + (2 * tp + 1) * kOSlab + og * OT) = make_uint2(cb[0], cb[1]);
        {   // Bt[j][t] = C[t][j] for this thread's row and R / 2 columns
            const int t = 2 * tp + (og & 1), j0 = (R / 2) * (og >> 1);
#pragma unroll
            for (int k = 0; k < CQ; ++k) {
                bc[(j0 + 2 * k) * kMPitch + t] = (uint16_t)yc[k];
                bc[(j0 + 2 * k + 1) * kMPitch + t] = (uint16_t)(yc[k] >> 16);
            }
        }
        if (sparse && bh_.n_rounds) store_stage(sq);
        // next block's loads, in the order they are consumed (past the last block they re-read
        // the last rows and are never used)
        load_crow(blk + 1, xq);
        if (hn.n_rounds) load_stage(sq, hn.r0);
        load_grows(blk + 1, wq);
        if (blk % (kMHdrRing / 2) == 0 && blk > 0) {
            __syncthreads();
            hdr_fill(blk + kMHdrRing / 2, kMHdrRing / 2);
        }
        combine_pending();  // the previous round's split features
        __syncthreads();  // tiles and the first round staged
        {   // fixed tile: rows 32 wave .. 32 wave + 31 of the block
            const int jj = lane & 15, kk = 32 * wave + 8 * (lane >> 4);
            const uint4 av = g_operand(32 * wave);
            uint4 bv = make_uint4(0u, 0u, 0u, 0u);
            if (jj < R) bv = *reinterpret_cast<const uint4 *>(bc + jj * kMPitch + kk);
            else if (jj == R) bv = make_uint4(kOne | kOne << 16, kOne | kOne << 16, kOne | kOne << 16, kOne | kOne << 16);
            accf = mfma_16x16x32<DT>(av, bv, accf);
        }
        if (!sparse || bh_.n_rounds == 0) {
            __syncthreads();  // the next block rewrites the tiles
            continue;
        }
        run_round(bh_.r0);
        for (uint32_t j = 1; j < bh_.n_rounds; ++j) {  // blocks with more than ROUND entries
            const RoundHdr h = a.rhdr[(int64_t)(bh_.first_round + j) * a.n_parts + part];
            StageM tmp;
            load_stage(tmp, h);
            store_stage(tmp);
            combine_pending();
            __syncthreads();
            run_round(h);
        }
    }
    combine_pending();
    __syncthreads();

    // ---- the fixed tile over the 16 waves, in wave order: M[o][j] (j < R), dbias (j = R)
    float *red = reinterpret_cast<float *>(base + L::s_red);
    float *mfin = reinterpret_cast<float *>(base + L::s_mfin);
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * 16 + 4 * (lane >> 4) + r) * 16 + (lane & 15)] = accf[r];
    __syncthreads();
    for (int t = threadIdx.x; t < kOSlab * (R + 1); t += kBwdThreads) {
        const int o = t / (R + 1), j = t % (R + 1);
        float sum = 0.f;
        for (int w = 0; w < 16; ++w) sum += red[(w * 16 + o) * 16 + j];
        mfin[o * (R + 1) + j] = sum;
    }
    __syncthreads();

    // ---- epilogue: dW tile = M Q^T + S, one rounding to the weight dtype; dbias from M[:, R]
    const uint16_t *q = static_cast<const uint16_t *>(a.q);
    const bool vec_out = a.transposed && a.out_vec_ok && o0 + kOSlab <= a.d_out;
    if (const int ii = threadIdx.x; ii < ni) {
        const int64_t i = i0 + ii;
        float qr[R];
#pragma unroll
        for (int j = 0; j < R; ++j) qr[j] = Act<DT>::ld(q[i * R + j]);
        float out[kOSlab];
#pragma unroll
        for (int oo = 0; oo < kOSlab; ++oo) {
            float s = acc[s_index(ii, oo)];
#pragma unroll
            for (int j = 0; j < R; ++j) s = fmaf(mfin[oo * (R + 1) + j], qr[j], s);
            out[oo] = s;
        }
        if (vec_out && a.dw_dt != STACR_DTYPE_F32) {
            const bool bf = a.dw_dt == STACR_DTYPE_BF16;
            uint32_t wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                wv[k] = bf ? (f_to_bf16_bits(out[2 * k]) | (f_to_bf16_bits(out[2 * k + 1]) << 16))
                           : (f_to_f16_bits(out[2 * k]) | (f_to_f16_bits(out[2 * k + 1]) << 16));
            uint4 *dst = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.dw) + i * a.d_out + o0);
            dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
            dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
        } else if (vec_out) {
            float4 *dst = reinterpret_cast<float4 *>(static_cast<float *>(a.dw) + i * a.d_out + o0);
#pragma unroll
            for (int k = 0; k < 4; ++k) dst[k] = make_float4(out[4 * k], out[4 * k + 1], out[4 * k + 2], out[4 * k + 3]);
        } else {
#pragma unroll
            for (int oo = 0; oo < kOSlab; ++oo)
                if (o0 + oo < a.d_out)
                    store_any(a.dw, a.dw_dt, a.transposed ? i * a.d_out + o0 + oo : (o0 + oo) * a.d_in + i, out[oo]);
        }
    }
    if (a.dbias && part == 0)
        for (int oo = threadIdx.x; oo < kOSlab; oo += kBwdThreads)
            if (o0 + oo < a.d_out) store_any(a.dbias, a.db_dt, o0 + oo, mfin[oo * (R + 1) + R]);
}

int pad_rank(int rank) { return rank <= 4 ? 4 : rank <= 8 ? 8 : rank <= 16 ? 16 : 32; }

struct CfgInfo {
    int tb, round;
};
template <int DT, int R> constexpr CfgInfo cfg_info()
{
    return CfgInfo{GradCfg<DT, R>::TB, GradCfg<DT, R>::ROUND};
}
CfgInfo block_geometry(int dt, int R)
{
    if (dt == STACR_DTYPE_F32)
        return R <= 4 ? cfg_info<0, 4>() : R <= 8 ? cfg_info<0, 8>() : R <= 16 ? cfg_info<0, 16>() : cfg_info<0, 32>();
    return R <= 4 ? cfg_info<1, 4>() : R <= 8 ? cfg_info<1, 8>() : R <= 16 ? cfg_info<1, 16>() : cfg_info<1, 32>();
}

enum { GW_ENT, GW_TASK, GW_HEAVY, GW_RHDR, GW_BHDR, GW_N };

struct GPlan {
    int R, tb, round_cap;
    int64_t n_slabs, n_parts, i_span, n_blocks, max_rounds;
};

GPlan make_gplan(const StacrGradArgs &a)
{
    GPlan p{};
    p.R = pad_rank(a.rank);
    p.n_slabs = (a.d_out + kOSlab - 1) / kOSlab;
    p.n_parts = hmax<int64_t>(1, (a.d_in + kMaxISlab - 1) / kMaxISlab);
    p.i_span = (a.d_in + p.n_parts - 1) / p.n_parts;
    const CfgInfo ci = block_geometry(a.dtype, p.R);
    p.tb = ci.tb;
    p.round_cap = ci.round;
    p.n_blocks = (a.rows + p.tb - 1) / p.tb;
    p.max_rounds = a.nnz / p.round_cap + p.n_blocks + 1;  // sum over blocks of ceil(entries / cap)
    return p;
}

size_t glayout(const StacrGradArgs &a, const GPlan &p, size_t *off)
{
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    const bool sp = a.nnz > 0;
    const size_t n = sp ? (size_t)a.nnz : 0;
    take(GW_ENT, n * 8);
    take(GW_TASK, n * 8);
    take(GW_HEAVY, n * 8);
    take(GW_RHDR, sp ? (size_t)p.max_rounds * p.n_parts * sizeof(RoundHdr) : 0);
    take(GW_BHDR, sp ? (size_t)p.n_blocks * p.n_parts * sizeof(BlockHdr) : 0);
    return cur;
}

template <typename K>
void raise_lds_limit(K kernel, size_t bytes)
{
    static bool done = false;  // once per kernel instantiation
    if (!done) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)bytes);
        done = true;
    }
}

template <int DT, int R>
int launch_grad(const StacrGradArgs &a, const GPlan &p, char *ws, const size_t *off)
{
    using Cfg = GradCfg<DT, R>;
    using L = FusedLds<DT, R>;
    hipStream_t s = a.stream;
    FusedArgs f{};
    f.g = a.g;
    f.coeff = a.coeff;
    f.q = a.q;
    f.rows = a.rows;
    f.d_out = a.d_out;
    f.d_in = a.d_in;
    f.rank = a.rank;
    f.scale = a.scale;
    f.bits = a.bits;
    f.nnz = a.rows > 0 ? a.nnz : 0;
    f.n_slabs = p.n_slabs;
    f.n_parts = p.n_parts;
    f.i_span = p.i_span;
    f.vec_ok = (a.d_out * (int64_t)sizeof(typename Cfg::T)) % Cfg::VB == 0 && (uintptr_t)a.g % Cfg::VB == 0;
    const int c_align = Cfg::CW * 4 >= 16 ? 16 : Cfg::CW * 4;
    f.c_vec = a.rank == R && (uintptr_t)a.coeff % c_align == 0;
    const int wb = a.dw_dtype == STACR_DTYPE_F32 ? 4 : 2;
    f.out_vec_ok = (a.d_out * wb) % 16 == 0 && (uintptr_t)a.dw % 16 == 0;
    f.transposed = a.transposed;
    f.dw = a.dw;
    f.dw_dt = a.dw_dtype;
    f.dbias = a.dbias;
    f.db_dt = a.dbias_dtype;
    const bool fast = a.rows > 0 && f.vec_ok && f.c_vec && a.d_out % kOSlab == 0;
    constexpr bool kMfmaCfg = DT != STACR_DTYPE_F32 && R <= 8;
    const bool mfma = kMfmaCfg && fast;  // the matrix-core kernel (its plan has column features)
    if (f.nnz > 0) {
        PlanArgs pa{};
        pa.idx = a.idx;
        pa.data = a.data;
        pa.bits = a.bits;
        pa.val_dt = a.val_dtype;
        pa.g_dt = a.dtype;
        pa.nnz = a.nnz;
        pa.rows = a.rows;
        pa.d_in = a.d_in;
        pa.n_parts = p.n_parts;
        pa.i_span = p.i_span;
        pa.tb = p.tb;
        pa.round_cap = (uint32_t)p.round_cap;
        pa.max_rounds = (uint32_t)p.max_rounds;
        pa.groups = (uint32_t)Cfg::NGRP;
        pa.slot_cap = (uint32_t)(mfma ? kMSlotCap : kSlotCap);
        pa.cols = mfma ? (uint32_t)kMCols : 0u;
        pa.ent = ws + off[GW_ENT];
        pa.task = reinterpret_cast<uint2 *>(ws + off[GW_TASK]);
        pa.heavy = reinterpret_cast<uint2 *>(ws + off[GW_HEAVY]);
        pa.rhdr = reinterpret_cast<RoundHdr *>(ws + off[GW_RHDR]);
        pa.bhdr = reinterpret_cast<BlockHdr *>(ws + off[GW_BHDR]);
        const dim3 pg((unsigned)p.n_blocks, (unsigned)p.n_parts);
        auto plan = [&](auto idx64, auto vk) {
            stacr_launch("k_dw_plan", s, [&] { k_dw_plan<decltype(idx64)::value, decltype(vk)::value><<<pg, kPlanThreads, 0, s>>>(pa); });
        };
        auto plan_vk = [&](auto idx64) {
            if (a.bits == 8) plan(idx64, std::integral_constant<int, kValI8>{});
            else if (a.bits == 4) plan(idx64, std::integral_constant<int, kValI4>{});
            else if (a.val_dtype == STACR_DTYPE_F32) plan(idx64, std::integral_constant<int, kVal32>{});
            else plan(idx64, std::integral_constant<int, kVal16>{});
        };
        if (a.index_bytes == 8) plan_vk(std::integral_constant<int, 1>{});
        else plan_vk(std::integral_constant<int, 0>{});
        f.ent = pa.ent;
        f.task = pa.task;
        f.heavy = pa.heavy;
        f.rhdr = pa.rhdr;
        f.bhdr = pa.bhdr;
    }
    constexpr size_t lds = L::bytes;
    static_assert(lds <= 160 * 1024, "LDS budget");
    const unsigned nwg = (unsigned)(p.n_slabs * p.n_parts);
    if constexpr (kMfmaCfg) {
        if (mfma) {
            constexpr size_t ml = MfmaLds<R>::bytes;
            static_assert(ml <= 160 * 1024, "LDS budget");
            static_assert(GradCfg<DT, R>::TB == kMTB && GradCfg<DT, R>::ROUND == kRoundMax, "plan geometry");
            raise_lds_limit(k_dw_fused_mfma<DT, R>, ml);
            stacr_launch("k_dw_fused_mfma", s, [&] { k_dw_fused_mfma<DT, R><<<nwg, kBwdThreads, ml, s>>>(f); });
            return stacr_hip_check(hipGetLastError(), "weight_grad kernels");
        }
    }
    if (fast) {
        raise_lds_limit(k_dw_fused<DT, R, true>, lds);
        stacr_launch("k_dw_fused", s, [&] { k_dw_fused<DT, R, true><<<nwg, kBwdThreads, lds, s>>>(f); });
    } else {
        raise_lds_limit(k_dw_fused<DT, R, false>, lds);
        stacr_launch("k_dw_fused", s, [&] { k_dw_fused<DT, R, false><<<nwg, kBwdThreads, lds, s>>>(f); });
    }
    return stacr_hip_check(hipGetLastError(), "weight_grad kernels");
}

template <int DT>
int grad_dispatch(const StacrGradArgs &a, const GPlan &p, char *ws, const size_t *off)
{
    switch (p.R) {
    case 4: return launch_grad<DT, 4>(a, p, ws, off);
    case 8: return launch_grad<DT, 8>(a, p, ws, off);
    case 16: return launch_grad<DT, 16>(a, p, ws, off);
    default: return launch_grad<DT, 32>(a, p, ws, off);
    }
}

}  // namespace

size_t stacr_grad_ws_layout(const StacrGradArgs &a, size_t *offsets)
{
    if (stacr_tiles_eligible(a)) return stacr_tiles_ws(a);
    const GPlan p = make_gplan(a);
    size_t tmp[GW_N];
    return glayout(a, p, offsets ? offsets : tmp);
}

int stacr_grad_launch(const StacrGradArgs &a)
{
    if (stacr_tiles_eligible(a)) return stacr_tiles_launch(a);
    const GPlan p = make_gplan(a);
    size_t off[GW_N];
    const size_t need = glayout(a, p, off);
    if (a.workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_weight_grad: workspace has %zu bytes, needs %zu",
                          a.workspace_bytes, need);
    if (a.d_in >= 65536)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_weight_grad: d_in must be below 65536");
    char *ws = static_cast<char *>(a.workspace);
    switch (a.dtype) {
    case STACR_DTYPE_F32: return grad_dispatch<STACR_DTYPE_F32>(a, p, ws, off);
    case STACR_DTYPE_BF16: return grad_dispatch<STACR_DTYPE_BF16>(a, p, ws, off);
    default: return grad_dispatch<STACR_DTYPE_F16>(a, p, ws, off);
    }
}
