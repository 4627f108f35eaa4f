// Weight gradient from the saved factors on the matrix cores: dW = (G^T C) Q^T + G^T R_s and
// dbias = sum_t G (stacr/layers.py:172-198), with G streamed once from memory.
//
// For 16-bit G and C, or fp32 G and C with 4 / 8-bit residual codes, rank (+ the bias column) <= 16,
// d_out a multiple of 16, d_in <= 8192.  Other problems use the kernels of weight_grad.hip.
// Accumulation is fp32 and dW is rounded once.
//
// Three launches.
//   k_tile_count  (sparse only) 16 workgroups over contiguous chunks of the residual entries: the
//     chunk's count of entries per input feature, and the first entry of every block of 512 token
//     rows (entries are ascending, so block b starts where the block of the entries changes).
//   k_tile_plan   one workgroup per (block of 512 rows, input part of <= 1024 features):
//     * (for k_tile_grad) the part's column features: the 48 with most entries over the whole
//       problem, ties to the lowest feature; every workgroup selects the same set;
//     * the block's column entries as dense matrix-core operands, in the order in which the lanes
//       of the streaming kernel load them, zero where no entry was selected: int8 codes for 4 / 8-bit
//       residuals (converted to G's dtype, exactly, as the streaming kernel loads them), else the
//       values in G's dtype (rounded as the reference rounds them);
//     * the block's other ("light") entries of the part as records t | (f mod 16) << 9 | value << 16,
//       grouped by feature and within a feature by ascending t (each entry's place is its feature's offset
//       plus the number of that feature's entries in earlier rows, counted from a per-feature row
//       bitmap), so the order, and so every sum, is the same on every run;
//     * part 0 also packs the block's coefficients [C | 1] as matrix-core operands.
//   k_tile_grad   one workgroup per (16 output features, input part), over the blocks in order:
//     * the G tile [512 rows][16 outputs], the light records and their offsets of block b + 2 are
//       copied straight into one of three LDS buffers (global_load_lds) while block b runs, and the
//       operands of block b + 1 are loaded into registers;
//     * wave w takes rows 32w .. 32w + 31: one v_mfma_f32_16x16x32 for M = G^T [C | 1] and one per
//       16-column tile of the column entries, all on the same G^T operand, accumulated in
//       registers over the blocks;
//     * thread f owns input feature f of the part and adds value * G[t][0..15] of each of its light
//       entries to 16 fp32 registers;
//     and at the end reduces the per-wave tiles over the waves (in wave order) and writes
//     dW[o][f] = sum_j M[o][j] Q[f][j] + scale * (light sum + column sum).
//   k_tile_wide   in place of k_tile_grad for problems with at least 256 workgroups of 32 outputs
//     (the plan then selects no column features: every entry is a light record): one workgroup per
//     (32 output features, part), the same three-buffer stream of G tiles and records, every entry
//     summed on the matrix cores in chunks of 32 records (see the kernel).
#include <type_traits>

#include "internal.h"

using namespace stacr;

namespace {

constexpr int kTB = 512;             // token rows per block
constexpr int kOS = 16;              // output features per workgroup
constexpr int kPartMax = 1024;       // input features per part (one owner thread each)
constexpr int kThreads = 1024;       // 16 waves
constexpr int kWaves = kThreads / 64;
constexpr int kOffWords = kPartMax + 1 + 255;  // a region's offsets, padded to whole 1 KiB (5 of them)
constexpr int kLightCap = kThreads / 64 * 256;   // light records staged per block (1 KiB per wave); more are read from memory
constexpr int kChunks = 16;          // entry chunks of the feature count
constexpr int kMaxFeat = 8192;       // input features the count kernel's LDS histogram holds
constexpr int kMaxBlocks = 256;      // blocks per problem (rows <= 131072): headers held in LDS
constexpr int kBatch = 8;            // entries per thread whose loads the count and the plan issue together
constexpr int kRounds = 3;           // rounds of kBatch entries a thread the plan keeps in registers between its passes
constexpr int kMaxRowSplit = 8;     // (no entries) workgroups over the rows of one o-slab, at most
constexpr int kSplitTargetWgs = 1024;  // rows are split until this many workgroups: two rounds of two a CU

static_assert(kThreads == 2 * kTB, "two G tile rows per lane pair: one 16-byte copy per lane");
static_assert(kTB == kCensusRows, "a save's entry census gives the first entry of every block");
static_assert(kOffWords % 256 == 0, "offsets are staged in whole 1 KiB copies");

constexpr int kNT = 3;               // 16-column matrix-core tiles of column entries per part (48 columns:
                                     // fewer light entries than 32, fewer operand bytes than 64; measured)
constexpr int kNC = 16 * kNT;        // column features per part
// LDS stride of one column of a block's column entries in the plan (elements): 8 past the block's
// rows, so that the 16 columns a 16-lane group reads when the tile is written out in lane order
// start in different banks
constexpr int kBtStride = kTB + 8;

struct TileHdr {  // per (block, part)
    uint32_t light_base;   // the region's first word in the record array (its offsets, then its records)
    uint32_t light_count;  // records
    uint32_t pad[2];
};

struct TileArgs {
    // problem
    const void *g, *coeff, *q, *idx, *data;
    const float *scale;
    int64_t rows, d_out, d_in, nnz;
    int rank, idx64, bits, val_dt, g_dt;
    int transposed;
    void *dw, *dbias;
    int dw_dt, db_dt;
    // geometry
    int n_blocks, n_parts, part_w, ncol, bias_col;
    // workspace
    uint32_t *hist;     // [n_hist][d_in] partial entry counts per feature (chunks, or census copies)
    int n_hist;
    uint32_t *bstart;   // [n_blocks + 1] first entry of each block
    void *cp;           // [n_blocks][16 waves][4 row groups][ncol][8] coefficient operands (G's dtype)
    void *bt;           // [n_blocks][n_parts][nt][16 waves][64 lanes][8] column operands
    uint32_t *light;    // regions of kOffWords offsets then light records (see the plan)
    TileHdr *hdr;       // [n_blocks][n_parts]
    int32_t *colmap;    // [n_parts][kNC] feature in the part, or -1
    int sparse;         // nnz > 0: the plan builds the entry structures
    int row_split;      // (no entries) workgroups over the rows of one o-slab; above 1 their M tiles go to mpart
    float *mpart;       // [o-slabs][row_split][256] the row ranges' M tiles (k_tile_lr_finish sums them)
    int columns;        // the plan picks kNC column features per part (0: every entry is a light record)
    // division by d_in as a multiply-high and shifts (Granlund and Montgomery, "Division by invariant
    // integers using multiplication", 1994, figure 4.1): exact for every 32-bit dividend
    uint32_t div_m;
    int div_s1, div_s2;
};

// The magic number and shifts of division by d (1 <= d < 2^32) for TileArgs::div_m / div_s1 / div_s2.
inline void div_magic(uint32_t d, uint32_t *m, int *s1, int *s2)
{
    int l = 0;
    while ((1ull << l) < d) ++l;  // ceil(log2 d)
    *m = (uint32_t)((((1ull << 32) * ((1ull << l) - d)) / d) + 1u);
    *s1 = l > 0 ? 1 : 0;
    *s2 = l > 0 ? l - 1 : 0;
}

// Words of the record array: every region's offsets and records (at most nnz records in all), the
// alignment slack, and the staging copy's overrun past the last region.
__host__ __device__ inline uint64_t record_words(int64_t nnz, uint64_t regions)
{
    return (uint64_t)nnz + regions * (uint64_t)(kOffWords + 3) + 3 + kLightCap;
}

// (token row, feature) of a flat index; rows * d_in < 2^32 (the host checks), so 32-bit division,
// by the argument block's multiply-high.  An index outside the problem (invalid input) still yields
// a feature < d_in.
__device__ __forceinline__ void split_flat(int64_t flat, const TileArgs &a, uint32_t &t, uint32_t &f)
{
    const uint32_t x = (uint32_t)flat;
    const uint32_t h = __umulhi(a.div_m, x);
    t = (h + ((x - h) >> a.div_s1)) >> a.div_s2;
    f = x - t * (uint32_t)a.d_in;
}

// Batched loads of kBatch entries e[k] (each an existing entry): the flat indices, and the product
// operands (the integer code for bits 4 / 8, or the stored value for bits 0).  The index width and
// the value encoding are uniform branches outside the unrolled loads, so a thread's loads are all
// issued before the first result is used (one memory round trip for the batch, not one per load).
__device__ __forceinline__ void load_flats(const TileArgs &a, const int64_t (&e)[kBatch], int64_t (&out)[kBatch])
{
    if (a.idx64) {
        const int64_t *p = static_cast<const int64_t *>(a.idx);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) out[k] = p[e[k]];
    } else {
        const int32_t *p = static_cast<const int32_t *>(a.idx);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) out[k] = (int64_t)p[e[k]];
    }
}

__device__ __forceinline__ void load_values(const TileArgs &a, const int64_t (&e)[kBatch], float (&out)[kBatch])
{
    if (a.bits == 8) {
        const int8_t *p = static_cast<const int8_t *>(a.data);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) out[k] = (float)(int)p[e[k]];
    } else if (a.bits == 4) {
        const uint8_t *p = static_cast<const uint8_t *>(a.data);
        uint32_t byte[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) byte[k] = p[e[k] >> 1];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int n = (int)((e[k] & 1) ? (byte[k] >> 4) : (byte[k] & 0xfu));
            out[k] = (float)(n > 7 ? n - 16 : n);
        }
    } else if (a.val_dt == STACR_DTYPE_F32) {
        const float *p = static_cast<const float *>(a.data);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) out[k] = p[e[k]];
    } else {
        const uint16_t *p = static_cast<const uint16_t *>(a.data);
        uint32_t h[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) h[k] = p[e[k]];
        const bool bf = a.val_dt == STACR_DTYPE_BF16;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) out[k] = bf ? bf16_bits_to_f(h[k]) : f16_bits_to_f(h[k]);
    }
}

// A light record's 16-bit value: an operand in G's dtype, exact for the integer codes; a stored value
// is rounded to G's dtype, as the reference casts the values to G's dtype before its sparse product.
// fp32 G takes codes only, kept as bf16 (exact for |code| <= 127).
__device__ __forceinline__ uint32_t to_g16(float v, int g_dt)
{
    return g_dt == STACR_DTYPE_F16 ? f_to_f16_bits(v) : f_to_bf16_bits(v);
}

template <int DT>
__device__ __forceinline__ float g16_to_f(uint32_t v)
{
    if constexpr (DT == STACR_DTYPE_BF16) return bf16_bits_to_f(v);
    else return f16_bits_to_f(v);
}

// ------------------------------------------------------------------ the entry count
__global__ __launch_bounds__(kThreads) void k_tile_count(TileArgs a)
{
    __shared__ uint32_t s_h[kMaxFeat];
    const int c = blockIdx.x, tid = threadIdx.x;
    const int64_t per = (a.nnz + kChunks - 1) / kChunks;
    const int64_t e0 = (int64_t)c * per < a.nnz ? (int64_t)c * per : a.nnz;
    const int64_t e1 = e0 + per < a.nnz ? e0 + per : a.nnz;
    const uint32_t d_in = (uint32_t)a.d_in;
    const int64_t last_blk = a.n_blocks - 1;
    for (int f = tid; f < (int)d_in; f += kThreads) s_h[f] = 0u;
    __syncthreads();
    auto block_of = [&](uint32_t t) {
        const int64_t b = (int64_t)(t / kTB);
        return b < last_blk ? b : last_blk;
    };
    // kBatch entries per thread per round, their loads issued together
    for (int64_t r0 = e0; r0 < e1; r0 += kBatch * kThreads) {
        // lanes past e1 load entry e1 - 1 (r0 < e1, so it exists) and skip it below; prev is used
        // only for e > 0
        int64_t cur[kBatch], prev[kBatch], ec[kBatch], ep[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int64_t e = r0 + k * kThreads + tid;
            ec[k] = e < e1 ? e : e1 - 1;
            ep[k] = ec[k] > 0 ? ec[k] - 1 : 0;
        }
        load_flats(a, ec, cur);
        load_flats(a, ep, prev);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int64_t e = r0 + k * kThreads + tid;
            if (e >= e1) continue;
            uint32_t t, f;
            split_flat(cur[k], a, t, f);
            atomicAdd(&s_h[f], 1u);
            // every block b with block(e - 1) < b <= block(e) starts at e; past the last entry, nnz
            const int64_t bcur = block_of(t);
            int64_t bprev = -1;
            if (e > 0) {
                uint32_t tp, fp;
                split_flat(prev[k], a, tp, fp);
                bprev = block_of(tp);
            }
            for (int64_t b = bprev + 1; b <= bcur; ++b) a.bstart[b] = (uint32_t)e;
            if (e == a.nnz - 1)
                for (int64_t b = bcur + 1; b <= a.n_blocks; ++b) a.bstart[b] = (uint32_t)a.nnz;
        }
    }
    __syncthreads();
    for (int f = tid; f < (int)d_in; f += kThreads) a.hist[(int64_t)c * d_in + f] = s_h[f];
}

// ------------------------------------------------------------------ the plan
// Exclusive prefix sums of two values over the workgroup's threads in one exchange (two barriers);
// the totals in *t0 and *t1.  s_tot2 holds 2 kWaves words.  Every thread must call it.
__device__ __forceinline__ uint32_t block_exclusive_scan2(uint32_t v0, uint32_t v1, uint32_t *s_tot2, uint32_t *t0,
                                                          uint32_t *t1)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t x0 = wave_inclusive_scan(v0), x1 = wave_inclusive_scan(v1);
    if (lane == 63) {
        s_tot2[wave] = x0;
        s_tot2[kWaves + wave] = x1;
    }
    __syncthreads();
    uint32_t before = 0, all0 = 0, all1 = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const uint32_t t = s_tot2[w];
        before += w < wave ? t : 0u;
        all0 += t;
        all1 += s_tot2[kWaves + w];
    }
    __syncthreads();
    *t0 = all0;
    *t1 = all1;
    return before + x0 - v0;
}

// One level of the column selection: wave 0 finds, from the 256-bin histogram h (counted from the
// top), the bin holding the need-th largest value and the need left inside it, and returns
// {bin, need} to every thread through *res (bin -1 when the histogram holds fewer than need
// values).  Every thread calls it (it contains a barrier).
__device__ __forceinline__ int2 select_bin256(const uint32_t *__restrict__ h, uint32_t need, int2 *res)
{
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        // lane l holds bins 255 - 4 l .. 252 - 4 l (from the top); inclusive sums across the lanes
        uint32_t c[4], t = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = h[255 - 4 * lane - i];
            t += c[i];
        }
        const uint32_t incl = wave_inclusive_scan(t);
        const uint32_t before = incl - t;
        const uint64_t hit = __ballot(incl >= need);
        const int first = hit ? __ffsll((unsigned long long)hit) - 1 : -1;
        if (lane == 0 && first < 0) *res = make_int2(-1, 0);
        if (lane == first) {
            uint32_t run = before;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (run + c[i] >= need) {
                    *res = make_int2(255 - 4 * lane - i, (int)(need - run));
                    break;
                }
                run += c[i];
            }
        }
    }
    __syncthreads();
    return *res;
}

template <bool BT8>
__global__ __launch_bounds__(kThreads) void k_tile_plan(TileArgs a)
{
    using BE = typename std::conditional<BT8, uint8_t, uint16_t>::type;  // one column-operand element
    __shared__ uint32_t s_key[kPartMax];         // colmap staging, then light offsets
    __shared__ int32_t s_slot[kPartMax];         // column slot of each feature of the part, or -1
    __shared__ uint32_t s_mask[16 * kPartMax];   // light rows of each feature, word w of feature f at w * kPartMax + f
    __shared__ uint16_t s_pre[8 * kPartMax];     // light rows of feature f in words below 2 v, at v * kPartMax + f
    __shared__ uint32_t s_h[256];
    __shared__ int2 s_sel;
    __shared__ __attribute__((aligned(16))) BE s_bt[kNC * kBtStride];  // the block's column entries [slot][t]
    __shared__ uint32_t s_tot[2 * kWaves];

    const int b = blockIdx.x, part = blockIdx.y, tid = threadIdx.x;
    // with entries, the workgroups past the last part pack the coefficient operands, in parallel
    // with the parts' entry work; without, part 0 packs them
    const bool pack_c = a.sparse ? part == a.n_parts : part == 0;
    const int64_t plo = (int64_t)part * a.part_w;
    const int pw = (int)(a.d_in - plo < a.part_w ? a.d_in - plo : a.part_w);

    if (a.sparse && !pack_c) {
        // the feature's partial counts (n_hist <= kChunks), issued first and unconditionally (addresses
        // clamped, values masked where used): they arrive with the block's starts, and the column
        // selection below does not wait for the block's entries, which are issued after them
        uint32_t hv[kChunks];
        {
            const int64_t fo = plo + (tid < pw ? tid : pw - 1);
#pragma unroll
            for (int c = 0; c < kChunks; ++c) hv[c] = a.hist[(int64_t)(c < a.n_hist ? c : a.n_hist - 1) * a.d_in + fo];
        }
        // ---- entry range of the block (clamped, whatever the starts hold)
        int64_t e_b0 = a.bstart[b], e_b1 = a.bstart[b + 1];
        e_b0 = e_b0 < a.nnz ? e_b0 : a.nnz;
        e_b1 = e_b1 < a.nnz ? e_b1 : a.nnz;
        e_b1 = e_b1 > e_b0 ? e_b1 : e_b0;

        // kBatch entries per thread per round, loaded together: flat index and value.  A block whose
        // entries fit one round loads them here, so their latency overlaps the column selection,
        // and keeps them in registers for both passes below.
        int64_t fl[kBatch];
        float val[kBatch];
        // (lanes past the block's entries load an existing entry, e_b1 - 1 or 0 as nnz >= 1 here,
        // and mark it flat -1, value 0)
        auto load_batch = [&](int64_t r0) {
            int64_t ec[kBatch];
            const int64_t e_safe = e_b1 > 0 ? e_b1 - 1 : 0;
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int64_t e = r0 + k * kThreads + tid;
                ec[k] = e < e_b1 ? e : e_safe;
            }
            load_flats(a, ec, fl);
            load_values(a, ec, val);
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                if (r0 + k * kThreads + tid >= e_b1) {
                    fl[k] = -1;
                    val[k] = 0.f;
                }
            }
        };
        // the first round is loaded here, so that its latency overlaps the column selection; blocks of
        // at most kRounds rounds keep their part's light entries in registers for the second pass
        const bool cached = e_b1 - e_b0 <= (int64_t)kRounds * kBatch * kThreads;
        load_batch(e_b0);

        // ---- column features: the kNC largest of the unique keys count << 16 | (65535 - f) over the
        // features with entries (count clamped to 65535): every feature with a clamped count above the
        // kNC-th largest one's, c64, and the lowest features with count c64 as far as needed.  c64 by
        // two radix levels of 8 bits (LDS histograms of the counts, the bin found by wave 0); then one
        // scan over the features gives, packed, the features above c64 and those equal to it below f,
        // which places every column at its slot in feature order.  (Every workgroup selects the same set.)
        uint32_t cnt = 0;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) cnt += c < a.n_hist ? hv[c] : 0u;
        cnt = tid < pw && a.columns ? (cnt < 0xffffu ? cnt : 0xffffu) : 0u;
        s_slot[tid] = -1;
        if (a.columns) {  // (uniform; without column features every entry is a light record)
            if (tid < 256) s_h[tid] = 0u;
            __syncthreads();
            {   // most features have fewer than 256 entries: bin 0 is added once per wave (a ballot
                // count), not once per lane, which would serialize about a thousand same-address atomics
                const bool low = cnt != 0u && (cnt >> 8) == 0u;
                const uint64_t lowm = __ballot(low);
                if (cnt != 0u && !low) atomicAdd(&s_h[cnt >> 8], 1u);
                if ((tid & 63) == 0 && lowm) atomicAdd(&s_h[0], (uint32_t)__popcll(lowm));
            }
            __syncthreads();
            const int2 l1 = select_bin256(s_h, (uint32_t)kNC, &s_sel);
            uint32_t c64 = 0u, take_eq = 0u;  // (fewer than kNC features with entries: all of them, c64 = 0)
            if (l1.x >= 0) {
                if (tid < 256) s_h[tid] = 0u;
                __syncthreads();
                if (cnt && (int)(cnt >> 8) == l1.x) atomicAdd(&s_h[cnt & 0xffu], 1u);
                __syncthreads();
                const int2 l2 = select_bin256(s_h, (uint32_t)l1.y, &s_sel);
                c64 = ((uint32_t)l1.x << 8) | (uint32_t)l2.x;
                take_eq = (uint32_t)l2.y;
            }
            const bool above = l1.x >= 0 ? cnt > c64 : cnt > 0u;
            const bool tie = l1.x >= 0 && cnt == c64;
            uint32_t packed_all;
            const uint32_t packed = block_exclusive_scan<kThreads>((above ? 1u : 0u) | (tie ? 1u << 16 : 0u), s_tot,
                                                                   &packed_all);
            const uint32_t n_above = packed & 0xffffu, ties_below = packed >> 16;
            const bool is_col = above || (tie && ties_below < take_eq);
            const uint32_t slot = n_above + (ties_below < take_eq ? ties_below : take_eq);
            if (is_col) s_slot[tid] = (int32_t)slot;
            if (b == 0 && tid < kNC) s_key[tid] = 0xffffffffu;
            __syncthreads();
            if (b == 0) {
                if (is_col) s_key[slot] = (uint32_t)tid;
                __syncthreads();
                if (tid < kNC) a.colmap[part * kNC + tid] = (int32_t)s_key[tid];
            }
        }

        // ---- this block's entries: the column tile and the light bitmaps
        static_assert((kNC * kBtStride * sizeof(BE)) % 16 == 0, "the column tile clears in 16-byte words");
        for (int i = tid; a.columns && i < (int)(kNC * kBtStride * sizeof(BE) / 16); i += kThreads)
            reinterpret_cast<uint4 *>(s_bt)[i] = make_uint4(0u, 0u, 0u, 0u);
        for (int i = tid; i < 16 * kPartMax / 4; i += kThreads)
            reinterpret_cast<uint4 *>(s_mask)[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
        const int64_t t_base = (int64_t)b * kTB;
        // (row in the block, feature in the part) of a loaded entry; false when it lies outside
        // the block (valid input has no such entry) or, with `in_part`, outside the part
        auto place = [&](int64_t flat, int &tl, int64_t &f) {
            uint32_t t, fg;
            split_flat(flat, a, t, fg);
            const int64_t tl64 = (int64_t)t - t_base;
            f = (int64_t)fg - plo;
            tl = (int)tl64;
            return flat >= 0 && tl64 >= 0 && tl64 < kTB;
        };
        uint32_t before_part = 0;  // entries of this block in lower parts: where the part's records start
        // entry k of the loaded round: its column operand, or its light-row bit; a light entry of the
        // part is returned as row | feature << 9 with its record value, else ~0
        static_assert(kTB == 1 << 9, "a block row in 9 bits");
        auto first_entry = [&](int k, uint32_t &pko, uint32_t &v16) {
            pko = ~0u;
            v16 = 0u;
            int tl;
            int64_t f;
            if (!place(fl[k], tl, f)) return;
            before_part += f < 0;
            if (f < 0 || f >= pw) return;
            const int s = s_slot[f];
            if (s >= 0) {
                if constexpr (BT8) s_bt[s * kBtStride + tl] = (BE)(uint8_t)(int8_t)(int)val[k];
                else s_bt[s * kBtStride + tl] = (BE)to_g16(val[k], a.g_dt);
            } else {
                atomicOr(&s_mask[(tl >> 5) * kPartMax + f], 1u << (tl & 31));
                pko = (uint32_t)tl | ((uint32_t)f << 9);
                v16 = to_g16(val[k], a.g_dt);
            }
        };
        uint32_t pk[kRounds][kBatch];      // (cached) light entries as row | feature << 9, else ~0
        uint32_t pv[kRounds][kBatch / 2];  // (cached) their record values, two a word
        if (cached) {
#pragma unroll
            for (int rr = 0; rr < kRounds; ++rr) {
                const int64_t r0 = e_b0 + (int64_t)rr * kBatch * kThreads;
                if (rr > 0 && r0 < e_b1) load_batch(r0);  // (uniform)
#pragma unroll
                for (int k = 0; k < kBatch; k += 2) {
                    uint32_t v0 = 0u, v1 = 0u;
                    pk[rr][k] = pk[rr][k + 1] = ~0u;
                    if (r0 < e_b1) {
                        first_entry(k, pk[rr][k], v0);
                        first_entry(k + 1, pk[rr][k + 1], v1);
                    }
                    pv[rr][k / 2] = v0 | (v1 << 16);
                }
            }
        } else {
            for (int64_t r0 = e_b0; r0 < e_b1; r0 += kBatch * kThreads) {
                if (r0 != e_b0) load_batch(r0);
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    uint32_t unused0, unused1;
                    first_entry(k, unused0, unused1);
                }
            }
        }
        __syncthreads();
        // light count of each feature; then, in one exchange, their offsets and the block's entries
        // in lower parts
        uint32_t lcnt = 0;
        if (tid < pw) {
#pragma unroll
            for (int w = 0; w < 16; ++w) {
                if (!(w & 1)) s_pre[(w >> 1) * kPartMax + tid] = (uint16_t)lcnt;
                lcnt += __popc(s_mask[w * kPartMax + tid]);
            }
        }
        uint32_t n_light, all_before;
        const uint32_t off = block_exclusive_scan2(lcnt, before_part, s_tot, &n_light, &all_before);
        // the region of (block, part): kOffWords words of offsets (feature f's records start at
        // word kOffWords + offset[f]; offset[pw] ends them), then the records.  Regions are ordered
        // by (block, part); region r starts at or after the entries of the earlier regions plus
        // r (kOffWords + 3) words, rounded up to 4 words: disjoint (a region holds at most its
        // entries' records) and 16-byte aligned for the staging copies.
        const uint32_t region = (uint32_t)(b * a.n_parts + part);
        const uint32_t base = ((uint32_t)e_b0 + all_before + region * (uint32_t)(kOffWords + 3) + 3u) & ~3u;
        uint32_t *reg = a.light + base;
        if (tid < pw) reg[tid] = off;
        if (tid == 0) reg[pw] = n_light;  // the part's end (pw may be 1024, past the last thread)
        if (tid == 0) a.hdr[b * a.n_parts + part] = TileHdr{base, n_light, {0u, 0u}};
        s_key[tid] = tid < pw ? off : 0u;
        __syncthreads();
        // each light entry at its feature's offset + the feature's light entries in earlier rows
        // (blocks of at most kRounds rounds have them in registers already)
        auto write_record = [&](int tl, int64_t f, uint32_t v16) {
            const int w = tl >> 5;
            uint32_t r = s_pre[(w >> 1) * kPartMax + f] + __popc(s_mask[w * kPartMax + f] & ((1u << (tl & 31)) - 1u));
            if (w & 1) r += __popc(s_mask[(w - 1) * kPartMax + f]);
            reg[kOffWords + s_key[f] + r] = (uint32_t)tl | ((uint32_t)(f & 15) << 9) | (v16 << 16);
        };
        if (cached) {
#pragma unroll
            for (int rr = 0; rr < kRounds; ++rr) {
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    if (pk[rr][k] == ~0u) continue;
                    write_record((int)(pk[rr][k] & (kTB - 1)), (int64_t)(pk[rr][k] >> 9),
                                 (pv[rr][k / 2] >> (16 * (k & 1))) & 0xffffu);
                }
            }
        } else {
            for (int64_t r0 = e_b0; r0 < e_b1; r0 += kBatch * kThreads) {
                load_batch(r0);
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    int tl;
                    int64_t f;
                    if (!place(fl[k], tl, f) || f < 0 || f >= pw || s_slot[f] >= 0) continue;
                    write_record(tl, f, to_g16(val[k], a.g_dt));
                }
            }
        }
        // the column operands in lane order: (tile i, wave w, lane l) holds rows 32 w + 8 (l / 16)
        // .. + 7 of column 16 i + l % 16, 8 elements
        using BV = typename std::conditional<BT8, uint2, uint4>::type;  // 8 elements
        BV *bt = static_cast<BV *>(a.bt) + ((int64_t)b * a.n_parts + part) * kNT * kWaves * 64;
        for (int u = tid; a.columns && u < kNT * kWaves * 64; u += kThreads) {
            const int l = u & 63, w = (u >> 6) & 15, i = u >> 10;
            bt[u] = *reinterpret_cast<const BV *>(s_bt + (16 * i + (l & 15)) * kBtStride + 32 * w + 8 * (l >> 4));
        }
    }

    // ---- the block's coefficient operands [C | 1]: (wave w, row group g, column n) holds rows
    // 32 w + 8 g .. + 7 of column n.  ncol <= 16 (the host checks), so a thread packs at most
    // kTB * 16 / kThreads elements: all their loads are issued before the first store, one memory
    // round trip in place of one per element.
    if (pack_c) {
        auto pack = [&](auto *cp, const auto *c, auto one) {
            constexpr int kPer = kTB * 16 / kThreads;
            cp += (int64_t)b * kTB * a.ncol;
            const int n_el = kTB * a.ncol;
            uint32_t v[kPer];  // (a register each: 16-bit values merged into shared registers would wait)
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int i = tid + u * kThreads;
                const int k = i & 7, n = (i >> 3) % a.ncol, wg = (i >> 3) / a.ncol;  // wg = 4 w + g
                const int64_t t = (int64_t)b * kTB + 8 * wg + k;
                v[u] = 0u;
                if (i < n_el && t < a.rows) {
                    if (n < a.rank) v[u] = c[t * a.rank + n];
                    else if (n == a.bias_col) v[u] = one;
                }
            }
            // every load has landed before the predicated stores, or each store would wait for the
            // stores before it (on this ISA the vector memory counter counts stores too)
            __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
            for (int u = 0; u < kPer; ++u)
                if (tid + u * kThreads < n_el) cp[tid + u * kThreads] = (decltype(one))v[u];
        };
        if (a.g_dt == STACR_DTYPE_F32)
            pack(static_cast<uint32_t *>(a.cp), static_cast<const uint32_t *>(a.coeff), 0x3f800000u);
        else
            pack(static_cast<uint16_t *>(a.cp), static_cast<const uint16_t *>(a.coeff),
                 (uint16_t)(a.g_dt == STACR_DTYPE_BF16 ? 0x3f80u : 0x3c00u));
    }
}

// ------------------------------------------------------------------ the streaming kernel
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c)
{
    if constexpr (DT == STACR_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(8))) __bf16 v8;
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    } else {
        typedef __attribute__((ext_vector_type(8))) _Float16 v8;
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
    }
}

// ds_read_b64_tr_b16: four 16-bit values transposed across each 16-lane group
__device__ __forceinline__ uint2 lds_tr16(const uint16_t *p)
{
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
    bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4 *)(p));
    return __builtin_bit_cast(uint2, v);
}

// c + a.lo b.lo + a.hi b.hi for two pairs of 16-bit values in G's dtype (v_dot2c_f32_bf16 / f16)
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
{
    if constexpr (DT == STACR_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 v2;
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 v2;
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
    }
}

// A raw buffer resource over `bytes` bytes at p (clamped to 4 GiB - 1); dword 3 is the gfx9-family
// raw-buffer format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint64_t bytes)
{
    const int n = bytes < 0xffffffffull ? (int)(uint32_t)bytes : (int)0xffffffffu;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}

// 16 bytes per lane at byte voffset + soffset of the resource into LDS at `wave_dst` + 16 * lane
// (wave_dst and soffset wave-uniform)
__device__ __forceinline__ void copy16(__amdgpu_buffer_rsrc_t r, void *wave_dst, uint32_t voffset, uint32_t soffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)wave_dst, 16, (int)voffset,
                                             (int)soffset, 0, 0);
}

__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset)
{
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, (int)soffset, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 load8(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset)
{
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voffset, (int)soffset, 0);
    return make_uint2(v.x, v.y);
}

// two integer-valued floats (|x| <= 128, exact in either dtype) packed in G's dtype: one packed
// conversion (v_cvt_pk_bf16_f32 / v_cvt_pkrtz_f16_f32)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    if constexpr (DT == STACR_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(2))) float f2;
        typedef __attribute__((ext_vector_type(2))) __bf16 b2;
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
}

// eight int8 codes -> eight 16-bit operands in G's dtype
template <int DT>
__device__ __forceinline__ uint4 codes_to_operand(uint2 w)
{
    auto f = [&](int k) {
        const uint32_t word = k < 4 ? w.x : w.y;
        return (float)(int)(int8_t)(word >> (8 * (k & 3)));
    };
    return make_uint4(pack2<DT>(f(0), f(1)), pack2<DT>(f(2), f(3)), pack2<DT>(f(4), f(5)), pack2<DT>(f(6), f(7)));
}

// LDS layout of one stream buffer (byte offsets).  The kernel holds three buffers as three
// distinct __shared__ arrays: the compiler then knows that reads of one never alias the
// direct-to-LDS copies into the others, and waits for those copies only where the code says so.
template <bool SP, int GB>
struct TileLds {
    // light records staged per block: fp32 G tiles are twice as large, so half as many records
    static constexpr int light_cap = GB == 4 ? kLightCap / 2 : kLightCap;
    static constexpr size_t g = 0;                                           // [kTB][16] G elements
    static constexpr size_t off = g + (size_t)kTB * kOS * GB;                // [kOffWords] u32
    static constexpr size_t light = off + (size_t)kOffWords * 4;             // [light_cap] u32
    static constexpr size_t size = SP ? light + (size_t)light_cap * 4 : off;  // with entries 37 KiB (45 fp32)
    static_assert(size % 1024 == 0, "buffers start on 1 KiB boundaries");
    static_assert(3 * size + kMaxBlocks * sizeof(TileHdr) <= 160 * 1024, "fits the CU's LDS");
    static_assert(size >= (size_t)kWaves * 256 * 4, "one tile of every wave fits a buffer (the reduction)");
};

// dW row i's outputs o0 .. o0 + 15, rounded once to dW's dtype: Conv1D (transposed, dW d_in x d_out)
// as two 16-byte words, nn.Linear (dW d_out x d_in) one value per output row.
__device__ __forceinline__ void store_dw_row(const TileArgs &a, int64_t i, int64_t o0, const float (&out)[kOS])
{
    if (a.transposed) {  // Conv1D: dW is d_in x d_out, 16 consecutive outputs per thread
        if (a.dw_dt == STACR_DTYPE_F32) {
            float4 *dst = reinterpret_cast<float4 *>(static_cast<float *>(a.dw) + i * a.d_out + o0);
#pragma unroll
            for (int k = 0; k < 4; ++k) dst[k] = make_float4(out[4 * k], out[4 * k + 1], out[4 * k + 2], out[4 * k + 3]);
        } else {
            const bool bf = a.dw_dt == STACR_DTYPE_BF16;
            uint32_t wv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                wv[k] = bf ? (f_to_bf16_bits(out[2 * k]) | (f_to_bf16_bits(out[2 * k + 1]) << 16))
                           : (f_to_f16_bits(out[2 * k]) | (f_to_f16_bits(out[2 * k + 1]) << 16));
            uint4 *dst = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.dw) + i * a.d_out + o0);
            dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
            dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
        }
    } else {  // nn.Linear: dW is d_out x d_in; consecutive threads write consecutive features
#pragma unroll
        for (int o = 0; o < kOS; ++o) store_any(a.dw, a.dw_dt, (o0 + o) * a.d_in + i, out[o]);
    }
}

// Without entries the buffers are small and two workgroups share a CU: 8 waves per SIMD, so
// <= 64 VGPRs.  fp32 G (entries with 4 / 8-bit codes only) runs v_mfma_f32_16x16x4_f32: eight
// products a tile over the same 32 rows a wave takes, row 32 w + 8 (lane / 16) + s in step s, so the
// operands keep the 16-bit layout's (row, column) assignment per lane.
template <int DT, bool SP, bool BT8>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(SP ? 4 : 8, SP ? 4 : 8))) void k_tile_grad(TileArgs a)
{
    constexpr int GB = DT == STACR_DTYPE_F32 ? 4 : 2;  // bytes of a G / C / Q element
    static_assert(GB == 2 || (SP && BT8), "fp32 G with residual codes only");
    using L = TileLds<SP, GB>;
    using QT = typename std::conditional<GB == 4, uint32_t, uint16_t>::type;
    constexpr int NT = SP ? kNT : 0;
    using BW = typename std::conditional<BT8, uint2, uint4>::type;  // one lane's column operand
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[L::size];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[L::size];
    __shared__ __attribute__((aligned(1024))) unsigned char lds2[L::size];
    __shared__ TileHdr s_hdr[SP ? kMaxBlocks : 1];
    // with entries, the part's Q rows (<= 1024 features x <= 16 values), loaded while the first two
    // blocks are copied and read by the epilogue
    constexpr bool kQLds = SP && GB == 2;  // (fp32 Q rows would not fit beside the fp32 buffers)
    __shared__ uint16_t s_q[kQLds ? kPartMax * 16 : 1];
    static_assert(!kQLds || 3 * L::size + kMaxBlocks * sizeof(TileHdr) + kPartMax * 16 * 2 <= 160 * 1024,
                  "the stream buffers, headers and Q rows fit the CU's LDS");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // workgroup -> (o-slab, part): consecutive logical ids share an XCD (ids are dealt to the 8 XCDs
    // round-robin), so the o-slabs and parts that read the same G lines meet in one L2
    const int nwg = gridDim.x;
    int logical = blockIdx.x;
    if (nwg % 8 == 0) logical = (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    // without entries the rows may be split over row_split workgroups per o-slab (slab-major, so
    // that neighbouring slabs, which read the same G lines, still meet in one L2): this one takes
    // blocks bb .. bb + nb - 1 and leaves its M tile for k_tile_lr_finish
    const int split = SP ? 0 : logical / (nwg / a.row_split);
    if constexpr (!SP) logical -= split * (nwg / a.row_split);
    const int part = logical % a.n_parts;
    const int64_t o0 = (int64_t)(logical / a.n_parts) * kOS;
    const int64_t plo = (int64_t)part * a.part_w;
    const int pw = (int)(a.d_in - plo < a.part_w ? a.d_in - plo : a.part_w);
    const int bb = SP ? 0 : (int)((int64_t)split * a.n_blocks / a.row_split);
    const int nb = SP ? a.n_blocks : (int)((int64_t)(split + 1) * a.n_blocks / a.row_split) - bb;

    const int n = lane & 15, grp = lane >> 4;

    if constexpr (SP) {
        for (int b = tid; b < nb; b += kThreads) s_hdr[b] = a.hdr[b * a.n_parts + part];
        __syncthreads();
    }

    // Every load goes through a buffer resource (base and size in scalar registers) with a 32-bit
    // per-lane offset that is the same for every block and a uniform per-block offset.  Kept apart
    // like this, no 64-bit per-lane address has to live across the stream.
    const uint32_t row_bytes = (uint32_t)a.d_out * GB;
    // G tile row and bytes into the row of this lane's 16-byte copy (fp32: one of two, 256 rows apart)
    const uint32_t g_lane_row = GB == 2 ? 32u * wave + (lane >> 1) : 16u * wave + (lane >> 2);
    const uint32_t g_lane_col = (uint32_t)o0 * GB + (GB == 2 ? 16u * (lane & 1) : 16u * (lane & 3));
    const uint32_t rec_lane = (256u * wave + 4u * lane) * 4;                  // light / offset copies
    const uint32_t cp_lane = ((wave * 4u + grp) * a.ncol + n) * 8 * GB;       // coefficient operand
    const uint32_t bt_lane = (wave * 64u + lane) * sizeof(BW);                // column operand
    const bool has_c = n < a.ncol;
    const uint32_t regions = (uint32_t)a.n_blocks * (uint32_t)a.n_parts;
    const __amdgpu_buffer_rsrc_t r_cp = make_rsrc(a.cp, (uint64_t)a.n_blocks * kTB * a.ncol * GB);  // (every block's)
    // (without entries these three are empty resources that nothing reads)
    const __amdgpu_buffer_rsrc_t r_light = make_rsrc(a.light, SP ? record_words(a.nnz, regions) * 4 : 0);
    const __amdgpu_buffer_rsrc_t r_bt = make_rsrc(a.bt, SP ? (uint64_t)regions * NT * kWaves * 64 * sizeof(BW) : 0);

    // ---- block `blk`'s copies into buffer B: light records (only the 1 KiB chunks the block has)
    // and offsets, then (issue_g) the G tile (this lane: row 32 wave + lane / 2, outputs 8 (lane & 1) ..)
    auto issue_records = [&](int blk, unsigned char *B) {
        if constexpr (SP) {
            // the region's offsets (1 KiB copies by waves 0..4, as far as the part needs) and the
            // 1 KiB chunks of records the block has
            const uint32_t lbase = __builtin_amdgcn_readfirstlane(s_hdr[blk].light_base);
            const uint32_t lcount = __builtin_amdgcn_readfirstlane(s_hdr[blk].light_count);
            if (wave < kOffWords / 256 && 256 * wave <= pw) copy16(r_light, B + L::off + (size_t)wave * 1024, rec_lane, lbase * 4);
            if (wave < L::light_cap / 256 && 256u * (uint32_t)wave < lcount)
                copy16(r_light, B + L::light + (size_t)wave * 1024, rec_lane, (lbase + kOffWords) * 4);
        }
    };
    auto issue_g = [&](int blk, unsigned char *B) {
        // rows past the end repeat the last (their operands are zero)
        const int64_t gb = (int64_t)(blk + bb);  // the block's index in the problem
        const uint32_t rows_here = (uint32_t)(a.rows - gb * kTB) < (uint32_t)kTB
                                       ? (uint32_t)(a.rows - gb * kTB) : (uint32_t)kTB;
        const __amdgpu_buffer_rsrc_t r_g =
            make_rsrc(static_cast<const char *>(a.g) + (size_t)gb * kTB * row_bytes, (uint64_t)rows_here * row_bytes);
#pragma unroll
        for (int h = 0; h < GB / 2; ++h) {
            const uint32_t row = g_lane_row + 256u * h;
            const uint32_t r = row < rows_here - 1 ? row : rows_here - 1;
            copy16(r_g, B + L::g + (size_t)h * 16384 + (size_t)wave * 1024, r * row_bytes + g_lane_col, 0u);
        }
    };

    // ---- block `blk`'s operands for this lane: rows 32 wave + 8 grp .. + 7 of column n
    struct Ops {
        uint4 c[GB / 2];
        BW t[NT > 0 ? NT : 1];
    };
    auto load_ops = [&](int blk, Ops &r) {
#pragma unroll
        for (int h = 0; h < GB / 2; ++h) {
            r.c[h] = make_uint4(0u, 0u, 0u, 0u);
            if (has_c) r.c[h] = load16(r_cp, cp_lane + 16u * h, (uint32_t)(blk + bb) * kTB * a.ncol * GB);
        }
        if constexpr (SP) {
            const uint32_t base = ((uint32_t)blk * a.n_parts + part) * (uint32_t)(NT * kWaves * 64 * sizeof(BW));
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const uint32_t so = base + (uint32_t)(i * kWaves * 64 * sizeof(BW));
                if constexpr (BT8) r.t[i] = load8(r_bt, bt_lane, so);
                else r.t[i] = load16(r_bt, bt_lane, so);
            }
        }
    };

    f32x4 acc_m = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc_t[NT > 0 ? NT : 1];
#pragma unroll
    for (int i = 0; i < (NT > 0 ? NT : 1); ++i) acc_t[i] = acc_m;
    float s[kOS];
#pragma unroll
    for (int o = 0; o < kOS; ++o) s[o] = 0.f;

    // ---- the block in buffer B with operands r: the matrix-core products
    auto products = [&](const unsigned char *B, const Ops &r) {
        if constexpr (GB == 4) {
            // step s: lane (g, n) gives G[32 w + 8 g + s][n] and the operands of that row, column n
            const float *gt = reinterpret_cast<const float *>(B + L::g);
            const int r0 = 32 * wave + 8 * grp;
            float av[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) av[k] = gt[(r0 + k) * kOS + n];
            const uint32_t cw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[GB / 2 - 1].x, r.c[GB / 2 - 1].y,
                                    r.c[GB / 2 - 1].z, r.c[GB / 2 - 1].w};
#pragma unroll
            for (int k = 0; k < 8; ++k) acc_m = __builtin_amdgcn_mfma_f32_16x16x4f32(av[k], __uint_as_float(cw[k]), acc_m, 0, 0, 0);
            if constexpr (SP) {
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const uint32_t w2[2] = {r.t[i].x, r.t[i].y};  // eight int8 codes, row order
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float code = (float)(int)(int8_t)(w2[k >> 2] >> (8 * (k & 3)));  // signed
                        acc_t[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[k], code, acc_t[i], 0, 0, 0);
                    }
                }
            }
        } else {
            const uint16_t *gt = reinterpret_cast<const uint16_t *>(B + L::g);
            // G^T[o][t0 .. t0 + 7], o = lane % 16, t0 = 32 wave + 8 (lane / 16): two transposing reads
            // (in a 16-lane group lane m addresses row r0 + m / 4, outputs 4 (m % 4) .. + 3, and lane n
            // receives G[r0 + j][n], j = 0..3)
            const int kk = 32 * wave + 8 * grp;
            const uint16_t *pa = gt + (kk + ((lane & 15) >> 2)) * kOS + (lane & 3) * 4;
            const uint2 lo = lds_tr16(pa), hi = lds_tr16(pa + 4 * kOS);
            const uint4 av = make_uint4(lo.x, lo.y, hi.x, hi.y);
            acc_m = mfma16<DT>(av, r.c[0], acc_m);
            if constexpr (SP) {
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    if constexpr (BT8) acc_t[i] = mfma16<DT>(av, codes_to_operand<DT>(r.t[i]), acc_t[i]);
                    else acc_t[i] = mfma16<DT>(av, r.t[i], acc_t[i]);
                }
            }
        }
    };

    // ---- this thread's feature: its light entries of the block in buffer B
    auto light_entries = [&](int blk, const unsigned char *B) {
        if constexpr (SP) {
            if (tid < pw) {
                const TileHdr h = s_hdr[blk];
                const uint32_t *off = reinterpret_cast<const uint32_t *>(B + L::off);
                const uint32_t *lrec = reinterpret_cast<const uint32_t *>(B + L::light);
                // the owner's range, clamped to the block's records whatever the offsets hold
                const uint32_t k1 = off[tid + 1] < h.light_count ? off[tid + 1] : h.light_count;
                const uint32_t k0 = off[tid] < k1 ? off[tid] : k1;
                // the record's G row (GB 16-byte words) from the tile
                struct GRow {
                    uint4 w[GB];
                };
                auto read_row = [&](uint32_t rec) {
                    const uint4 *p = reinterpret_cast<const uint4 *>(B + L::g + (size_t)(rec & 511u) * kOS * GB);
                    GRow r;
#pragma unroll
                    for (int i = 0; i < GB; ++i) r.w[i] = p[i];
                    return r;
                };
                auto add_row = [&](uint32_t rec, const GRow &g) {
                    if constexpr (GB == 4) {
                        // s[o] += G[t][o] v, the code v kept as bf16 in the record's high half
                        const float v = __uint_as_float(rec & 0xffff0000u);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            s[4 * i] = fmaf(__uint_as_float(g.w[i].x), v, s[4 * i]);
                            s[4 * i + 1] = fmaf(__uint_as_float(g.w[i].y), v, s[4 * i + 1]);
                            s[4 * i + 2] = fmaf(__uint_as_float(g.w[i].z), v, s[4 * i + 2]);
                            s[4 * i + 3] = fmaf(__uint_as_float(g.w[i].w), v, s[4 * i + 3]);
                        }
                    } else {
                        // s[2 k] += lo(w_k) v and s[2 k + 1] += hi(w_k) v for the row's eight 32-bit
                        // words w_k: dot products with the pairs (v, 0) and (0, v), no conversions
                        const uint32_t v_lo = rec >> 16, v_hi = rec & 0xffff0000u;
                        const uint32_t w[8] = {g.w[0].x, g.w[0].y, g.w[0].z, g.w[0].w,
                                               g.w[GB - 1].x, g.w[GB - 1].y, g.w[GB - 1].z, g.w[GB - 1].w};
#pragma unroll
                        for (int o = 0; o < 8; ++o) {
                            s[2 * o] = dot2<DT>(w[o], v_lo, s[2 * o]);
                            s[2 * o + 1] = dot2<DT>(w[o], v_hi, s[2 * o + 1]);
                        }
                    }
                };
                auto add_entry = [&](uint32_t rec) { add_row(rec, read_row(rec)); };
                // records staged in LDS, two at a time (both rows read before either is summed, in
                // record order), then (blocks with more than the staged records) the rest from memory
                const uint32_t kl = k1 < (uint32_t)L::light_cap ? k1 : (uint32_t)L::light_cap;
                uint32_t k = k0;
                for (; k + 1 < kl; k += 2) {
                    const uint32_t ra = lrec[k], rb = lrec[k + 1];
                    const GRow ga = read_row(ra), gb = read_row(rb);
                    add_row(ra, ga);
                    add_row(rb, gb);
                }
                if (k < kl) add_entry(lrec[k]);
                for (uint32_t k = k0 > kl ? k0 : kl; k < k1; ++k) add_entry(a.light[h.light_base + kOffWords + k]);
            }
        }
    };

    // ---- the stream: block blk runs in buffer blk % 3 while block blk + 2 is copied into
    // buffer (blk + 2) % 3.  A step: the products of block blk (its operands then die), the operand
    // loads of block blk + 1, the copies of block blk + 2, the light entries of block blk, then
    // (issue_g) the G copy of block blk + 2; then a wait that lets only that last memory
    // instruction stay in flight across the barrier.
    Ops ops;
    load_ops(0, ops);
    issue_records(0, lds0);
    issue_g(0, lds0);
    if (nb > 1) {
        issue_records(1, lds1);
        issue_g(1, lds1);
    }
    const QT *q = static_cast<const QT *>(a.q);
    if constexpr (kQLds) {
        // the part's Q rows (pw * rank <= 16384 values, contiguous): all loads issued, then stored
        const int n_q = pw * a.rank;
        const uint16_t *qs = q + plo * a.rank;
        uint32_t qv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) qv[k] = tid + k * kThreads < n_q ? qs[tid + k * kThreads] : 0u;
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (tid + k * kThreads < n_q) s_q[tid + k * kThreads] = (uint16_t)qv[k];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    auto step = [&](int blk, const unsigned char *__restrict__ B, unsigned char *__restrict__ B2) {
        products(B, ops);
        load_ops(blk + 1, ops);
        if (blk + 2 < nb) issue_records(blk + 2, B2);
        light_entries(blk, B);
        // every step ends its memory instructions with the G copy (fp32: two), so that the wait
        // below always covers the operand loads; in the step before last it copies the last block
        // again into the buffer of block blk - 1, which nothing reads any more
        issue_g(blk + 2 < nb ? blk + 2 : nb - 1, B2);
        // vmcnt(1) (fp32: 2) lgkmcnt(0) (expcnt unconstrained), as a builtin so that the compiler
        // knows the operand loads have landed; then the barrier, not __syncthreads(), whose fence
        // would wait for every copy in flight
        if constexpr (GB == 4) __builtin_amdgcn_s_waitcnt(0x0072);
        else __builtin_amdgcn_s_waitcnt(0x0071);
        asm volatile("s_barrier" ::: "memory");
    };
    // every block but the last through `step` (the last loads nothing more)
    int cb = 0;
    for (int blk = 0; blk + 1 < nb; ++blk, cb = cb == 2 ? 0 : cb + 1) {
        unsigned char *B = cb == 0 ? lds0 : cb == 1 ? lds1 : lds2;
        unsigned char *B2 = cb == 0 ? lds2 : cb == 1 ? lds0 : lds1;
        step(blk, B, B2);
    }
    {
        const unsigned char *B = cb == 0 ? lds0 : cb == 1 ? lds1 : lds2;
        products(B, ops);
        light_entries(nb - 1, B);
    }

    // ---- what the epilogue reads from memory, loaded before the reduction hides the latency: the
    // scale (it exists only with residual entries; without them the sparse sums are zero) and the
    // part's column map
    const float scale = SP && a.bits ? *a.scale : 1.f;
    const int colf = SP && tid < kNC ? a.colmap[part * kNC + tid] : -1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // ---- reduce the per-wave tiles over the waves, in wave order.  Every wave's tiles are staged
    // at once (16 KiB a tile: tiles 0, 1 in lds0, 2, 3 in lds1, 4 in lds2, as many as there are); the sums and the part's
    // column slots follow the last tile (in lds1 without entries, whose one tile is in lds0)
    constexpr int NTILE = 1 + NT;
    constexpr size_t kTileBytes = (size_t)kWaves * 256 * 4;
    static_assert(L::size >= (SP ? 2 : 1) * kTileBytes, "two tiles (one without entries) fit a buffer");
    static_assert(!SP || NTILE <= 5, "at most five tiles with entries");
    static_assert(!SP || kTileBytes + NTILE * 256 * 4 + kPartMax * 4 <= L::size, "the last tile, sums and slots fit a buffer");
    auto stage_of = [&](int tile) {
        unsigned char *b = tile < 2 ? lds0 : tile < 4 ? lds1 : lds2;
        return reinterpret_cast<float *>(b + (size_t)(tile & 1) * kTileBytes);
    };
    unsigned char *fin_base = SP ? lds2 + kTileBytes : lds1;
    float *fin = reinterpret_cast<float *>(fin_base);                         // [NTILE][o][j]
    int32_t *slots = reinterpret_cast<int32_t *>(fin_base + NTILE * 256 * 4);  // [pw]
#pragma unroll
    for (int tile = 0; tile < NTILE; ++tile) {
        const f32x4 acc = tile == 0 ? acc_m : acc_t[tile > 0 ? tile - 1 : 0];
        float *stage = stage_of(tile);
#pragma unroll
        for (int r = 0; r < 4; ++r)  // D layout: rows 4 (lane / 16) .. + 3 of column lane % 16
            stage[wave * 256 + (4 * grp + r) * 16 + n] = acc[r];
    }
    if constexpr (SP) {
        if (tid < pw) slots[tid] = -1;
    }
    __syncthreads();
    for (int e = tid; e < NTILE * 256; e += kThreads) {
        const float *stage = stage_of(e >> 8);
        float sum = 0.f;
        for (int w = 0; w < kWaves; ++w) sum += stage[w * 256 + (e & 255)];
        fin[e] = sum;
    }
    if constexpr (SP) {
        if (colf >= 0 && colf < pw) slots[colf] = tid;
    }
    __syncthreads();

    if constexpr (!SP) {
        if (a.row_split > 1) {  // (uniform) this row range's M tile, summed over the splits later
            if (tid < 256) a.mpart[((int64_t)(o0 / kOS) * a.row_split + split) * 256 + tid] = fin[tid];
            return;
        }
    }

    // ---- dW tile: M Q^T + scale (light + column sums), one rounding; dbias from M[:, bias_col].
    // With entries a part has <= 1024 features, one per thread (thread f finishes feature f); 16-bit
    // Q rows are in s_q already.  Otherwise the Q rows of a chunk of features are first copied to
    // LDS (fp32 with entries: lds0, free after the reduction; without entries: lds2), and without
    // entries the threads loop over the chunk's features.
    const int qfit = (int)(L::size / ((size_t)a.rank * GB));
    const int qchunk = kQLds || qfit > kThreads ? kThreads : qfit;
    QT *sq = kQLds ? reinterpret_cast<QT *>(s_q) : reinterpret_cast<QT *>(SP ? lds0 : lds2);
    auto qval = [&](QT v) {
        if constexpr (GB == 4) return __uint_as_float(v);
        else return g16_to_f<DT>(v);
    };
    for (int c0 = 0; c0 < pw; c0 += qchunk) {
        const int nf = pw - c0 < qchunk ? pw - c0 : qchunk;
        if constexpr (!kQLds) {
            __syncthreads();  // the previous chunk's Q rows are no longer read
            for (int e = tid; e < nf * a.rank; e += kThreads) sq[e] = q[(plo + c0) * a.rank + e];
            __syncthreads();
        }
        for (int fl = SP ? tid : c0 + tid; fl < c0 + nf; fl += kThreads) {
        if (SP && fl < c0) continue;  // (with entries: this thread's feature is in a later chunk)
        const int64_t i = plo + fl;
        const int slot = SP ? slots[fl] : -1;
        float out[kOS];
#pragma unroll
        for (int o = 0; o < kOS; ++o) {
            const float col = slot >= 0 ? fin[(1 + (slot >> 4)) * 256 + o * 16 + (slot & 15)] : 0.f;
            out[o] = SP ? scale * (s[o] + col) : 0.f;
        }
        // + sum_j M[o][j] Q[i][j] (the M reads are LDS broadcasts)
        for (int j = 0; j < a.rank; ++j) {
            const float qj = qval(sq[(fl - c0) * a.rank + j]);
#pragma unroll
            for (int o = 0; o < kOS; ++o) out[o] = fmaf(fin[o * 16 + j], qj, out[o]);
        }
        store_dw_row(a, i, o0, out);
        }
    }
    if (a.dbias && part == 0 && tid < kOS) store_any(a.dbias, a.db_dt, o0 + tid, fin[tid * 16 + a.bias_col]);
}

// ------------------------------------------------------------------ row-split finish (no entries)
// Without entries, the rows of an o-slab may be split over row_split workgroups of k_tile_grad,
// each leaving its M tile (Gᵀ[C | 1] over its rows) in mpart.  One workgroup per (o-slab, 256 input
// features): M = the tiles summed in row-range order, then dW = M Qᵀ rounded once, as k_tile_grad's
// epilogue computes it, and dbias from M's bias column.
template <int DT>
__global__ __launch_bounds__(256) void k_tile_lr_finish(TileArgs a)
{
    __shared__ float s_m[256];
    const int tid = threadIdx.x;
    // workgroup -> (o-slab, chunk of 256 features), slabs fastest; consecutive logical ids share an
    // XCD (ids are dealt to the 8 XCDs round-robin), so the 32-byte pieces neighbouring slabs write
    // into one Conv1D dW row meet in one L2
    const int nwg = gridDim.x, n_slabs = (int)(a.d_out / kOS);
    const int logical = nwg % 8 == 0 ? (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8 : blockIdx.x;
    const int64_t slab = logical % n_slabs, o0 = slab * kOS, chunk = logical / n_slabs;
    const int64_t i = chunk * 256 + tid;
    const bool live = i < a.d_in && a.rank > 0;
    // this thread's Q row (rank < 16 values), loaded first so that its latency overlaps the M
    // tiles': unconditional loads of the row's own values, index clamped (a branch per load would
    // make each wait for the one before)
    const uint16_t *q = static_cast<const uint16_t *>(a.q) + (live ? i : 0) * a.rank;
    uint32_t qv[16];
    if (a.rank > 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) qv[j] = q[j < a.rank ? j : a.rank - 1];
    }
    // M: the slab's row-range tiles summed in range order
    const float *mp = a.mpart + slab * a.row_split * 256;
    float v[kMaxRowSplit];
#pragma unroll
    for (int r = 0; r < kMaxRowSplit; ++r) v[r] = r < a.row_split ? mp[r * 256 + tid] : 0.f;
    float m = v[0];
#pragma unroll
    for (int r = 1; r < kMaxRowSplit; ++r)
        if (r < a.row_split) m += v[r];
    s_m[tid] = m;
    __syncthreads();
    if (chunk == 0 && a.dbias && tid < kOS) store_any(a.dbias, a.db_dt, o0 + tid, s_m[tid * 16 + a.bias_col]);
    if (i >= a.d_in) return;
    // dW[i][o0 .. o0 + 15] = sum_j M[o][j] Q[i][j] in j order, rounded once
    float out[kOS];
#pragma unroll
    for (int o = 0; o < kOS; ++o) out[o] = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        if (j < a.rank) {
            const float qj = g16_to_f<DT>(qv[j]);
#pragma unroll
            for (int o = 0; o < kOS; ++o) out[o] = fmaf(s_m[o * 16 + j], qj, out[o]);
        }
    }
    store_dw_row(a, i, o0, out);
}

// ------------------------------------------------------------------ the wide streaming kernel
// For problems large enough to fill the chip with 32-output slabs: one workgroup per (32 outputs,
// part), every entry of the part a light record (the plan selects no column features).  Wave w
// owns features 64 w .. 64 w + 63 of the part as four 16-feature tiles, whose records of a block
// are contiguous (grouped by feature, then by row).  The wave takes each tile's records 32 at a
// time as one chunk: the G rows of the 32 records, gathered by two transposing reads per 16
// outputs, are the A operand; the records scatter their values into a zeroed [16 features][32
// slots] LDS scratch at (feature in the tile, slot), the scratch read in operand order is the B
// operand (cleared again after the read), and one v_mfma_f32_16x16x32 per 16 outputs adds
// G[t_k][o] v_k to (o, feature).  So each wave's work is about its entry count / 32 + 4 matrix
// instructions a block, whatever the spread of the entries over the features, and the sums have a
// fixed order (chunks in record order, blocks in order).
constexpr int kWOS = 32;         // outputs per workgroup
constexpr int kWRecBuf = 3584;   // record words of a stream buffer
constexpr int kWRecCap = kWRecBuf - 32;  // blocks with at most this many records read them from LDS
                                         // (a chunk reads up to 31 words past its first record)

struct WideLds {
    static constexpr size_t g = 0;                                  // [kTB][kWOS] G elements
    static constexpr size_t rec = g + (size_t)kTB * kWOS * 2;       // [kWRecBuf] records
    static constexpr size_t size = rec + (size_t)kWRecBuf * 4;      // 46 KiB
    static_assert(size % 1024 == 0, "buffers start on 1 KiB boundaries");
    static_assert(kWRecBuf % 256 == 0, "records are staged in 1 KiB copies");
    static_assert(3 * size + kWaves * (1024 + 64) + kMaxBlocks * sizeof(TileHdr) <= 160 * 1024, "fits the CU's LDS");
    static_assert(size >= (size_t)kWaves * 2 * 256 * 4, "every wave's two coefficient tiles fit a buffer");
    static_assert(size >= (size_t)kPartMax * 16 * 2, "the part's Q rows fit a buffer");
};

template <int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void k_tile_wide(TileArgs a)
{
    using L = WideLds;
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[L::size];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[L::size];
    __shared__ __attribute__((aligned(1024))) unsigned char lds2[L::size];
    __shared__ __attribute__((aligned(16))) uint16_t s_bs[kWaves * 512];  // per wave [16 features][32 slots]
    __shared__ uint16_t s_spare[kWaves * 32];  // per wave, a word each for the lanes whose stores go nowhere
    __shared__ TileHdr s_hdr[kMaxBlocks];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, grp = lane >> 4;

    // workgroup -> (o-slab, part), consecutive logical ids on one XCD (as k_tile_grad)
    const int nwg = gridDim.x;
    int logical = blockIdx.x;
    if (nwg % 8 == 0) logical = (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int part = logical % a.n_parts;
    const int64_t o0 = (int64_t)(logical / a.n_parts) * kWOS;
    const int64_t plo = (int64_t)part * a.part_w;
    const int pw = (int)(a.d_in - plo < a.part_w ? a.d_in - plo : a.part_w);
    const int nb = a.n_blocks;

    for (int b = tid; b < nb; b += kThreads) s_hdr[b] = a.hdr[b * a.n_parts + part];
    uint16_t *bs = s_bs + wave * 512;
    reinterpret_cast<uint4 *>(bs)[lane] = make_uint4(0u, 0u, 0u, 0u);  // 1 KiB: the scratch starts zero
    __syncthreads();

    const uint32_t row_bytes = (uint32_t)a.d_out * 2;
    const uint32_t g_lane_row = (uint32_t)tid >> 2;                        // + 256 for the second copy
    const uint32_t g_lane_col = (uint32_t)o0 * 2 + 16u * (uint32_t)(tid & 3);
    const uint32_t rec_lane = (256u * wave + 4u * lane) * 4;
    const uint32_t cp_lane = ((wave * 4u + grp) * a.ncol + n) * 16;
    const bool has_c = n < a.ncol;
    const uint32_t regions = (uint32_t)nb * (uint32_t)a.n_parts;
    const __amdgpu_buffer_rsrc_t r_cp = make_rsrc(a.cp, (uint64_t)nb * kTB * a.ncol * 2);
    const __amdgpu_buffer_rsrc_t r_light = make_rsrc(a.light, record_words(a.nnz, regions) * 4);

    // A block with more records than a buffer stages runs as several windows of kWRecCap records
    // over the same G tile ("steps"): step = (block, window), in order.  A step's state in scalar
    // registers: its block, window, record region and count.
    struct Step {
        int blk;
        uint32_t w, base, count;
    };
    auto windows = [&](uint32_t count) { return count <= (uint32_t)kWRecCap ? 1u : (count + kWRecCap - 1) / kWRecCap; };
    auto step_at = [&](int blk, uint32_t w) {
        const int b = blk < nb ? blk : nb - 1;
        return Step{blk, w, (uint32_t)__builtin_amdgcn_readfirstlane(s_hdr[b].light_base),
                    (uint32_t)__builtin_amdgcn_readfirstlane(s_hdr[b].light_count)};
    };
    auto next_step = [&](const Step &st) {
        return st.w + 1 < windows(st.count) ? Step{st.blk, st.w + 1, st.base, st.count} : step_at(st.blk + 1, 0u);
    };
    // the step's records (window w: records [w kWRecCap, ..), the 1 KiB chunks it has) into buffer B
    auto issue_records = [&](const Step &st, unsigned char *B) {
        const uint32_t first = st.w * (uint32_t)kWRecCap;
        const uint32_t left = st.count - first;
#pragma unroll
        for (int h = 0; h < kWRecBuf / 256; h += kWaves) {
            const int c = h + wave;
            if (c < kWRecBuf / 256 && 256u * (uint32_t)c < left)
                copy16(r_light, B + L::rec + (size_t)c * 1024, rec_lane + (uint32_t)h * 1024,
                       (st.base + kOffWords + first) * 4);
        }
    };
    // block `blk`'s G tile [512 rows][32 outputs] into buffer B: two 16-byte copies a lane
    auto issue_g = [&](int blk, unsigned char *B) {
        const uint32_t rows_here = (uint32_t)(a.rows - (int64_t)blk * kTB) < (uint32_t)kTB
                                       ? (uint32_t)(a.rows - (int64_t)blk * kTB) : (uint32_t)kTB;
        const __amdgpu_buffer_rsrc_t r_g =
            make_rsrc(static_cast<const char *>(a.g) + (size_t)blk * kTB * row_bytes, (uint64_t)rows_here * row_bytes);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t row = g_lane_row + 256u * h;
            const uint32_t r = row < rows_here - 1 ? row : rows_here - 1;
            copy16(r_g, B + L::g + (size_t)h * 16384 + (size_t)wave * 1024, r * row_bytes + g_lane_col, 0u);
        }
    };
    // this wave's tile bounds of the step's block: lane i <= 4 loads the offset of feature
    // 64 w + 16 i (the part's end past pw), clamped to the block's records
    auto load_bounds = [&](const Step &st) {
        const int f = 64 * wave + 16 * (lane < 5 ? lane : 4);
        const uint32_t fo = (uint32_t)(f < pw ? f : pw);
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r_light, (int)(fo * 4), (int)(st.base * 4), 0);
        return v < st.count ? v : st.count;
    };
    auto load_c = [&](int blk) {
        uint4 c = make_uint4(0u, 0u, 0u, 0u);
        if (has_c) c = load16(r_cp, cp_lane, (uint32_t)(blk < nb ? blk : nb - 1) * kTB * a.ncol * 2);
        return c;
    };

    f32x4 acc_m[2], acc[4][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        acc_m[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = acc_m[j];
    }

    // Each chunk is up to 32 consecutive records of one of the wave's four tiles (a tile's records
    // are grouped by feature, the tiles' ranges follow each other).  Lane 16 g + 4 q + h (h = 0, 1) holds the record
    // of slot 8 g + 4 h + q (lanes with h = 2, 3 repeat h = 0, 1): so the quad's first two lanes
    // hold slots k1 = 8 g + q and k1 + 4, the rows this lane's transposing reads need, and
    // every slot < 32 is held once by a lane with h < 2, which scatters its value.
    const uint32_t my = 8u * grp + 4u * (lane & 1) + ((lane >> 2) & 3);  // the slot this lane holds
    const bool scatters = (lane & 2) == 0;
    uint16_t *spare = s_spare + wave * 32 + 2 * (lane >> 2) + (lane & 1);
    // the scratch row of feature f keeps its four 16-byte slot groups rotated by rot(f): a 16-byte
    // read is served eight lanes a cycle over 32 banks, and (f & 1, rot(f)) differ across each eight
    // consecutive features (a rotation by f's bits 2..3 alone gave every read two cycles of conflicts)
    // rot(f) = f2 | (f1 ^ f2 ^ f3) << 1, two bits a feature of the constant
    auto rot = [](uint32_t f) { return (0xf50a5fa0u >> (2u * f)) & 3u; };
    const uint16_t *bsrd_lane = s_bs + wave * 512 + n * 32 + 8 * (grp ^ rot((uint32_t)n));
    const uint32_t ga_lane = (n & 3) * 4;

    // the step in buffer B: (window 0) M = G^T [C | 1] over the wave's 32 rows, then the wave's
    // records of the window as chunks
    auto run_step = [&](const Step &st, const unsigned char *B, uint4 cop, uint32_t bnd) {
        const uint16_t *gt = reinterpret_cast<const uint16_t *>(B + L::g);
        if (st.w == 0) {
            const int kk = 32 * wave + 8 * grp;
            const uint16_t *pa = gt + (kk + (n >> 2)) * kWOS + (n & 3) * 4;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint2 lo = lds_tr16(pa + 16 * j), hi = lds_tr16(pa + 16 * j + 4 * kWOS);
                acc_m[j] = mfma16<DT>(make_uint4(lo.x, lo.y, hi.x, hi.y), cop, acc_m[j]);
            }
        }
        const uint32_t *recs = reinterpret_cast<const uint32_t *>(B + L::rec);
        // tile i spans records [b_i, b_i+1) of the block (every value here is wave-uniform)
        const uint32_t b0 = __builtin_amdgcn_readlane(bnd, 0);
        uint32_t b1 = __builtin_amdgcn_readlane(bnd, 1), b2 = __builtin_amdgcn_readlane(bnd, 2);
        uint32_t b3 = __builtin_amdgcn_readlane(bnd, 3), b4 = __builtin_amdgcn_readlane(bnd, 4);
        b1 = b1 > b0 ? b1 : b0;
        b2 = b2 > b1 ? b2 : b1;
        b3 = b3 > b2 ? b3 : b2;
        b4 = b4 > b3 ? b4 : b3;
        const uint32_t bb[5] = {b0, b1, b2, b3, b4};
        // the window's records [w0, w1) staged from recs[0]; this wave's part of them [lo, hi)
        const uint32_t w0 = st.w * (uint32_t)kWRecCap;
        const uint32_t w1 = st.count - w0 < (uint32_t)kWRecCap ? st.count : w0 + kWRecCap;
        uint16_t *bs = s_bs + wave * 512;
        const uint16_t *ga = gt + ga_lane;
        // this wave's records in the window
        const uint32_t lo = b0 > w0 ? b0 : w0, hi0 = b4 < w1 ? b4 : w1, hi = hi0 > lo ? hi0 : lo;
        // one chunk of tile i at records [e0, e0 + 32) (slots at or past t_hi hold whatever follows:
        // the next tile's records or a stale word of the buffer; their lanes store zero, and the G
        // row they address is in the tile, t & 511): A = the G rows of slots k1 (.. + 3 over the
        // group) and k1 + 4, per 16 outputs; B = the tile's values at (feature in the tile, slot) of
        // the zeroed scratch (rows of 32 slots, the four 16-byte groups of a row rotated by rot(f)),
        // cleared again after the read; one product per 16 outputs.  Every lane stores unconditionally: a lane past
        // t_hi stores zero at its own slot, which no other lane of the chunk writes and which is
        // zero already, and the lanes that repeat another's record store into their spare word.
        auto chunk = [&](f32x4 (&ac)[2], uint32_t rec, uint32_t e0, uint32_t t_hi) {
            const uint32_t r1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)rec, 0x00, 0xf, 0xf, false);
            const uint32_t r2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)rec, 0x55, 0xf, 0xf, false);
            const uint16_t *p1 = ga + (r1 & 511u) * kWOS;
            const uint16_t *p2 = ga + (r2 & 511u) * kWOS;
            const uint2 lo0 = lds_tr16(p1), hi0 = lds_tr16(p2);
            const uint2 lo1 = lds_tr16(p1 + 16), hi1 = lds_tr16(p2 + 16);
            const uint4 a0 = make_uint4(lo0.x, lo0.y, hi0.x, hi0.y), a1 = make_uint4(lo1.x, lo1.y, hi1.x, hi1.y);
            const uint32_t fo = (rec >> 9) & 15u;
            uint16_t *slot = scatters ? bs + fo * 32 + 8 * ((my >> 3) ^ rot(fo)) + (my & 7) : spare;
            const uint16_t v = e0 + my < t_hi ? (uint16_t)(rec >> 16) : (uint16_t)0;
            // The lanes exchange values through the scratch: wavefront-scope fences keep the
            // compiler from moving one lane's store across another lane's load (a wave's LDS
            // operations are performed in order, so they cost no wait).
            *slot = v;
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            const uint4 bop = *reinterpret_cast<const uint4 *>(bsrd_lane);
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            *slot = 0;
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            ac[0] = mfma16<DT>(a0, bop, ac[0]);
            ac[1] = mfma16<DT>(a1, bop, ac[1]);
        };
        // tile by tile, the tile's records of the window [max(b_i, lo), min(b_i+1, hi)) in chunks,
        // each chunk's record read before the previous one runs.  The chunks follow each other in
        // record order (a tile's first record is where the previous tile's ended), so the next
        // start is always e0 + 32 or the tile's end; its index, at most hi - w0 + 31 <= kWRecCap +
        // 31, is inside the buffer.
        if (lo < hi) {
            uint32_t nx = recs[lo - w0 + my];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t_lo = bb[i] > lo ? bb[i] : lo;
                const uint32_t t_hi = bb[i + 1] < hi ? bb[i + 1] : hi;
                for (uint32_t e0 = t_lo; e0 < t_hi; e0 += 32) {
                    const uint32_t cur = nx;
                    nx = recs[(e0 + 32 < t_hi ? e0 + 32 : t_hi) - w0 + my];
                    chunk(acc[i], cur, e0, t_hi);
                }
            }
        }
    };

    // ---- the stream: step v runs in buffer v % 3 while step v + 2 is copied into buffer
    // (v + 2) % 3; the operands (C, tile bounds) of step v + 1 are loaded into registers.  (The
    // states of steps v, v + 1 and v + 2 are carried in scalar registers; a step past the last
    // repeats the last block's copies into a buffer nothing reads any more.)
    int n_steps = 0;
    for (int b = 0; b < nb; ++b) n_steps += (int)windows((uint32_t)__builtin_amdgcn_readfirstlane(s_hdr[b].light_count));
    Step s0 = step_at(0, 0u);
    Step s1 = next_step(s0);
    Step s2 = next_step(s1);
    uint4 cop = load_c(0);
    uint32_t bnd = load_bounds(s0);
    issue_records(s0, lds0);
    issue_g(0, lds0);
    if (n_steps > 1) {
        issue_records(s1, lds1);
        issue_g(s1.blk < nb ? s1.blk : nb - 1, lds1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    auto step = [&](int v, const unsigned char *__restrict__ B, unsigned char *__restrict__ B2) {
        const uint4 c_here = cop;
        const uint32_t b_here = bnd;
        cop = load_c(s1.blk);
        bnd = load_bounds(s1);
        if (v + 2 < n_steps) issue_records(s2, B2);
        run_step(s0, B, c_here, b_here);
        issue_g(s2.blk < nb ? s2.blk : nb - 1, B2);
        const Step s3 = next_step(s2);
        __builtin_amdgcn_s_waitcnt(0x0072);  // vmcnt(2) lgkmcnt(0): only the two G copies stay in flight
        asm volatile("s_barrier" ::: "memory");
        s0 = s1;
        s1 = s2;
        s2 = s3;
    };
    int cb = 0;
    for (int v = 0; v + 1 < n_steps; ++v, cb = cb == 2 ? 0 : cb + 1) {
        unsigned char *B = cb == 0 ? lds0 : cb == 1 ? lds1 : lds2;
        unsigned char *B2 = cb == 0 ? lds2 : cb == 1 ? lds0 : lds1;
        step(v, B, B2);
    }
    run_step(s0, cb == 0 ? lds0 : cb == 1 ? lds1 : lds2, cop, bnd);

    const float scale = a.bits ? *a.scale : 1.f;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // ---- M over the waves, in wave order: every wave's two tiles staged in lds0, sums in lds2;
    // the part's Q rows (16-bit) in lds1
    float *stage = reinterpret_cast<float *>(lds0);
    float *fin = reinterpret_cast<float *>(lds2);  // [2][16 o][16 j]
    uint16_t *sq = reinterpret_cast<uint16_t *>(lds1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[(wave * 2 + j) * 256 + (4 * grp + r) * 16 + n] = acc_m[j][r];
    const uint16_t *q = static_cast<const uint16_t *>(a.q);
    for (int e = tid; e < pw * a.rank; e += kThreads) sq[e] = q[plo * a.rank + e];
    __syncthreads();
    if (tid < 512) {
        float sum = 0.f;
        for (int w = 0; w < kWaves; ++w) sum += stage[(w * 2 + (tid >> 8)) * 256 + (tid & 255)];
        fin[tid] = sum;
    }
    __syncthreads();

    // ---- dW: lane (n, grp) of wave w holds, per tile i and o-tile j, outputs 16 j + 4 grp .. + 3 of
    // feature 64 w + 16 i + n
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int fl = 64 * wave + 16 * i + n;
        if (fl >= pw) continue;
        const int64_t f = plo + fl;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float out[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) out[r] = scale * acc[i][j][r];
            for (int c = 0; c < a.rank; ++c) {
                const float qc = g16_to_f<DT>(sq[fl * a.rank + c]);
#pragma unroll
                for (int r = 0; r < 4; ++r) out[r] = fmaf(fin[j * 256 + (4 * grp + r) * 16 + c], qc, out[r]);
            }
            const int64_t o = o0 + 16 * j + 4 * grp;
            if (a.transposed) {  // Conv1D: dW is d_in x d_out, four consecutive outputs
                if (a.dw_dt == STACR_DTYPE_F32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(a.dw) + f * a.d_out + o) =
                        make_float4(out[0], out[1], out[2], out[3]);
                } else {
                    const bool bf = a.dw_dt == STACR_DTYPE_BF16;
                    uint32_t wv[2];
#pragma unroll
                    for (int k = 0; k < 2; ++k)
                        wv[k] = bf ? (f_to_bf16_bits(out[2 * k]) | (f_to_bf16_bits(out[2 * k + 1]) << 16))
                                   : (f_to_f16_bits(out[2 * k]) | (f_to_f16_bits(out[2 * k + 1]) << 16));
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(a.dw) + f * a.d_out + o) = make_uint2(wv[0], wv[1]);
                }
            } else {  // nn.Linear: dW is d_out x d_in
#pragma unroll
                for (int r = 0; r < 4; ++r) store_any(a.dw, a.dw_dt, (o + r) * a.d_in + f, out[r]);
            }
        }
    }
    if (a.dbias && part == 0 && tid < kWOS) store_any(a.dbias, a.db_dt, o0 + tid, fin[(tid >> 4) * 256 + (tid & 15) * 16 + a.bias_col]);
}

}  // namespace

// ------------------------------------------------------------------ host side
namespace {

struct TileGeom {
    int n_blocks, n_parts, part_w, ncol, bias_col;
    int gb;  // bytes of a G / C element
    bool sparse, bt8;
    bool wide;  // k_tile_wide (every entry a light record, no column operands) in place of k_tile_grad
    int row_split;  // (no entries) k_tile_grad workgroups over the rows of one o-slab
};

// Workgroups of the wide kernel that make it the better choice: at least one per CU (256) with
// 32-output slabs.  Below that the 16-output kernel's twice as many workgroups fill the chip better.
constexpr int kWideMinWgs = 256;

bool tile_geom(const StacrGradArgs &a, TileGeom *g)
{
    // 16-bit G; or fp32 G with residual codes (bits 4 / 8: integer operands, kept as bf16 exactly)
    const bool f32 = a.dtype == STACR_DTYPE_F32;
    if (a.dtype != STACR_DTYPE_BF16 && a.dtype != STACR_DTYPE_F16 && !(f32 && a.nnz > 0 && a.bits != 0)) return false;
    if (a.rows < 1 || a.d_in < 1 || a.d_out < kOS || a.d_out % kOS) return false;
    const int cols = a.rank + (a.dbias ? 1 : 0);
    if (cols > 16) return false;
    if ((uintptr_t)a.g % 16) return false;
    if (a.rows > (int64_t)kMaxBlocks * kTB || a.d_in > kMaxFeat) return false;
    if ((uint64_t)a.rows * (uint64_t)a.d_in >= (1ull << 32)) return false;  // 32-bit flat indices
    if ((uint64_t)kTB * (uint64_t)a.d_out * (f32 ? 4 : 2) >= (1ull << 31)) return false;  // 32-bit lane offsets
    if (a.nnz > 0 && a.index_bytes != 4 && a.index_bytes != 8) return false;
    if (a.nnz >= (1ll << 31)) return false;
    g->n_blocks = (int)((a.rows + kTB - 1) / kTB);
    // with entries, parts of <= 1024 features (one owner thread each); without, one part
    g->n_parts = a.nnz > 0 ? (int)((a.d_in + kPartMax - 1) / kPartMax) : 1;
    g->part_w = (int)((a.d_in + g->n_parts - 1) / g->n_parts);
    g->ncol = cols;
    g->bias_col = a.dbias ? a.rank : -1;
    g->gb = f32 ? 4 : 2;
    g->sparse = a.nnz > 0;
    g->bt8 = a.bits != 0;
    g->wide = g->sparse && !f32 && a.d_out % kWOS == 0 && (a.d_out / kWOS) * g->n_parts >= kWideMinWgs;
    // without entries a workgroup's results are its M tile alone, so the rows of each o-slab are
    // split (at least two blocks a workgroup) until the launch fills the chip evenly; the tiles are
    // summed in a fixed order by k_tile_lr_finish
    g->row_split = 1;
    while (!g->sparse && g->row_split < kMaxRowSplit && (a.d_out / kOS) * g->row_split < kSplitTargetWgs &&
           g->n_blocks >= 4 * g->row_split)
        g->row_split *= 2;
    return true;
}

enum { TW_HIST, TW_BSTART, TW_CP, TW_BT, TW_LIGHT, TW_HDR, TW_COLMAP, TW_MPART, TW_N };

size_t tile_layout(int64_t nnz, int64_t d_in, int64_t d_out, const TileGeom &g, size_t *off)
{
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    const size_t regions = (size_t)g.n_blocks * g.n_parts;
    // column operands: kNT tiles of int8 codes (32 KiB per region) or 16-bit values (64 KiB)
    const size_t bt_bytes = regions * (size_t)kNT * kWaves * 64 * (g.bt8 ? 8 : 16);
    take(TW_HIST, g.sparse ? (size_t)kChunks * d_in * 4 : 0);
    take(TW_BSTART, g.sparse ? ((size_t)g.n_blocks + 1) * 4 : 0);
    take(TW_CP, (size_t)g.n_blocks * kTB * g.ncol * g.gb);
    take(TW_BT, g.sparse && !g.wide ? bt_bytes : 0);
    take(TW_LIGHT, g.sparse ? (size_t)record_words(nnz, regions) * 4 : 0);
    take(TW_HDR, g.sparse ? regions * sizeof(TileHdr) : 0);
    take(TW_COLMAP, g.sparse ? (size_t)g.n_parts * kNC * 4 : 0);
    take(TW_MPART, g.row_split > 1 ? (size_t)(d_out / kOS) * g.row_split * 256 * 4 : 0);
    return cur;
}

template <int DT, bool SP, bool BT8>
int launch_tile_grad(const TileArgs &t, int nwg, hipStream_t s)
{
    stacr_launch("k_tile_grad", s, [&] { k_tile_grad<DT, SP, BT8><<<nwg, kThreads, 0, s>>>(t); });
    return stacr_hip_check(hipGetLastError(), "weight_grad matrix-core kernel");
}

template <int DT>
int launch_tile_grad_dt(const TileArgs &t, const TileGeom &g, int nwg, hipStream_t s)
{
    if (!g.sparse) return launch_tile_grad<DT, false, true>(t, nwg, s);
    return g.bt8 ? launch_tile_grad<DT, true, true>(t, nwg, s) : launch_tile_grad<DT, true, false>(t, nwg, s);
}

}  // namespace

bool stacr_tiles_eligible(const StacrGradArgs &a)
{
    TileGeom g;
    return tile_geom(a, &g);
}

size_t stacr_tiles_ws(const StacrGradArgs &a)
{
    TileGeom g;
    size_t off[TW_N];
    return tile_geom(a, &g) ? tile_layout(a.nnz, a.d_in, a.d_out, g, off) : 0;
}

size_t stacr_tiles_ws_bound(int64_t rows, int64_t d_out, int64_t d_in, int64_t nnz)
{
    if (rows < 1 || d_in < 1 || d_out < kOS) return 0;
    TileGeom g;
    g.n_blocks = (int)((rows + kTB - 1) / kTB);
    g.n_parts = nnz > 0 ? (int)((d_in + kPartMax - 1) / kPartMax) : 1;
    g.part_w = (int)((d_in + g.n_parts - 1) / g.n_parts);
    g.ncol = 16;  // the widest coefficient operand (rank + bias column up to 16)
    g.bias_col = -1;
    g.gb = 4;       // fp32 coefficient operands
    g.sparse = nnz > 0;
    g.bt8 = false;  // the wider column-operand form
    g.wide = false;  // (with column operands: the larger layout)
    g.row_split = nnz > 0 ? 1 : kMaxRowSplit;  // (the most M tiles)
    size_t off[TW_N];
    return tile_layout(nnz, d_in, d_out, g, off);
}

int stacr_tiles_launch(const StacrGradArgs &a)
{
    TileGeom g;
    if (!tile_geom(a, &g)) return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_weight_grad: matrix-core path not applicable");
    size_t off[TW_N];
    const size_t need = tile_layout(a.nnz, a.d_in, a.d_out, g, off);
    if (a.workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_weight_grad: workspace has %zu bytes, needs %zu", a.workspace_bytes,
                          need);
    char *ws = static_cast<char *>(a.workspace);
    TileArgs t{};
    t.g = a.g;
    t.coeff = a.coeff;
    t.q = a.q;
    t.idx = a.idx;
    t.data = a.data;
    t.scale = a.scale;
    t.rows = a.rows;
    t.d_out = a.d_out;
    t.d_in = a.d_in;
    t.nnz = a.nnz;
    t.rank = a.rank;
    t.idx64 = a.index_bytes == 8;
    t.bits = a.bits;
    t.val_dt = a.val_dtype;
    t.g_dt = a.dtype;
    t.transposed = a.transposed;
    t.dw = a.dw;
    t.dbias = a.dbias;
    t.dw_dt = a.dw_dtype;
    t.db_dt = a.dbias_dtype;
    t.n_blocks = g.n_blocks;
    t.n_parts = g.n_parts;
    t.part_w = g.part_w;
    t.ncol = g.ncol;
    t.bias_col = g.bias_col;
    t.cp = ws + off[TW_CP];
    // with a census from the save, its per-feature counts and block starts replace the count pass
    const bool census = g.sparse && a.census;
    if (g.sparse) {
        t.hist = census ? const_cast<uint32_t *>(a.census) : reinterpret_cast<uint32_t *>(ws + off[TW_HIST]);
        t.n_hist = census ? kCensusCopies : kChunks;
        t.bstart = census ? const_cast<uint32_t *>(a.census) + (size_t)kCensusCopies * a.d_in
                          : reinterpret_cast<uint32_t *>(ws + off[TW_BSTART]);
        t.bt = ws + off[TW_BT];
        t.light = reinterpret_cast<uint32_t *>(ws + off[TW_LIGHT]);
        t.hdr = reinterpret_cast<TileHdr *>(ws + off[TW_HDR]);
        t.colmap = reinterpret_cast<int32_t *>(ws + off[TW_COLMAP]);
    }
    t.sparse = g.sparse ? 1 : 0;
    t.row_split = g.row_split;
    t.mpart = reinterpret_cast<float *>(ws + off[TW_MPART]);
    t.columns = g.wide ? 0 : 1;
    div_magic((uint32_t)a.d_in, &t.div_m, &t.div_s1, &t.div_s2);
    hipStream_t s = a.stream;
    int rc;
    if (g.sparse && !census) {
        stacr_launch("k_tile_count", s, [&] { k_tile_count<<<kChunks, kThreads, 0, s>>>(t); });
        rc = stacr_hip_check(hipGetLastError(), "weight_grad entry count");
        if (rc) return rc;
    }
    const dim3 pgrid((unsigned)g.n_blocks, g.sparse ? (unsigned)g.n_parts + 1u : 1u);
    if (g.bt8) stacr_launch("k_tile_plan", s, [&] { k_tile_plan<true><<<pgrid, kThreads, 0, s>>>(t); });
    else stacr_launch("k_tile_plan", s, [&] { k_tile_plan<false><<<pgrid, kThreads, 0, s>>>(t); });
    rc = stacr_hip_check(hipGetLastError(), "weight_grad plan");
    if (rc) return rc;
    if (g.wide) {
        const int nw = (int)(a.d_out / kWOS) * g.n_parts;
        if (a.dtype == STACR_DTYPE_BF16)
            stacr_launch("k_tile_wide", s, [&] { k_tile_wide<STACR_DTYPE_BF16><<<nw, kThreads, 0, s>>>(t); });
        else
            stacr_launch("k_tile_wide", s, [&] { k_tile_wide<STACR_DTYPE_F16><<<nw, kThreads, 0, s>>>(t); });
        return stacr_hip_check(hipGetLastError(), "weight_grad wide matrix-core kernel");
    }
    const int nwg = (int)(a.d_out / kOS) * g.n_parts * g.row_split;
    if (a.dtype == STACR_DTYPE_F32) return launch_tile_grad<STACR_DTYPE_F32, true, true>(t, nwg, s);
    rc = a.dtype == STACR_DTYPE_BF16 ? launch_tile_grad_dt<STACR_DTYPE_BF16>(t, g, nwg, s)
                                     : launch_tile_grad_dt<STACR_DTYPE_F16>(t, g, nwg, s);
    if (rc || g.row_split == 1) return rc;
    const unsigned fgrid = (unsigned)((a.d_out / kOS) * ((a.d_in + 255) / 256));
    if (a.dtype == STACR_DTYPE_BF16)
        stacr_launch("k_tile_lr_finish", s, [&] { k_tile_lr_finish<STACR_DTYPE_BF16><<<fgrid, 256, 0, s>>>(t); });
    else
        stacr_launch("k_tile_lr_finish", s, [&] { k_tile_lr_finish<STACR_DTYPE_F16><<<fgrid, 256, 0, s>>>(t); });
    return stacr_hip_check(hipGetLastError(), "weight_grad row-split finish");
}
