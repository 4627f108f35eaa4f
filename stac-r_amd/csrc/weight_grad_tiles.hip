// Weight gradient from the saved factors on the matrix cores, with the G stream double-buffered
// straight into LDS: dW = (G^T C) Q^T + G^T R_s, dbias = sum_t G (stacr/layers.py:172-198).
//
// For 16-bit G and C, rank (+ the bias column) <= 16, d_out a multiple of 16.  Other problems use
// the kernels of weight_grad.hip.  Accumulation is fp32 and dW is rounded once to its dtype.
//
// Two launches.
//   k_tile_plan  one workgroup per (block of 512 token rows, input part of <= 1024 features):
//     * the part's column features: those with at least kMinColCount entries in block 0 (the
//       sample), the 32 with most entries, ties to the lowest feature, slots in feature order;
//     * the block's column entries as a dense tile Bt[slot][t] (values in G's dtype, zero where
//       no entry was selected);
//     * the block's other ("light") entries of the part as records t | value << 16, grouped by
//       feature and within a feature by ascending t: each entry's place is its feature's offset
//       plus the number of that feature's entries in earlier rows of the block, counted from a
//       per-feature row bitmap, so the order (and so every sum) is the same on every run;
//     * block 0's workgroups also pack the block's coefficients transposed, Cp[col][t], with a
//       column of ones (its matrix-core column is dbias) and zeros past the rank and the rows.
//   k_tile_grad  one workgroup per (16 output features, input part); per block of 512 rows:
//     * the next block's G tile [t][16], Cp tile, Bt tile, light records and their offsets are
//       loaded straight into the other LDS buffer (global_load_lds_dwordx4) while this block runs;
//     * wave w takes rows 32w..32w+31: one v_mfma_f32_16x16x32 for M = G^T [C | 1] and one per
//       16-column tile of Bt, all on the same G^T operand, accumulated in registers across blocks;
//     * thread f owns input feature f of the part and adds value * G[t][0..15] of each of its
//       light entries to 16 fp32 registers;
//     and at the end reduces the per-wave tiles over the waves (in wave order) and writes
//     dW[o][f] = sum_j M[o][j] Q[f][j] + scale * (light sum + column sum).
#include <mutex>

#include "internal.h"

using namespace stacr;

namespace {

constexpr int kTB = 512;             // token rows per block
constexpr int kOS = 16;              // output features per workgroup
constexpr int kPartMax = 1024;       // input features per part (one owner thread each)
constexpr int kNC = 32;              // column features per part (two 16-column tiles)
constexpr int kThreads = 1024;       // 16 waves
constexpr int kLightCap = 2048;      // light records staged per block (8 KiB); more are read from memory
constexpr int kMinColCount = 16;     // entries in the sample block a column feature needs
constexpr int kOffWords = kPartMax + 1 + 255;  // offsets staged as whole 1 KiB wave loads (5 of them)

static_assert(kThreads == 2 * kTB, "two G tile rows per lane pair: one 16-byte load per lane");

struct TileHdr {  // per (block, part)
    uint32_t light_base;   // first light record (index into the record array)
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
    uint16_t *cp;       // [n_blocks][ncol][kTB]
    uint16_t *bt;       // [n_blocks][n_parts][kNC][kTB]
    uint32_t *light;    // [nnz + kLightCap]
    uint32_t *loff;     // [n_blocks][n_parts][kOffWords]
    TileHdr *hdr;       // [n_blocks][n_parts]
    int32_t *colmap;    // [n_parts][kNC] feature in the part, or -1
    int sparse;         // nnz > 0: the plan builds the entry structures
};

__device__ __forceinline__ int64_t flat_at(const void *idx, int idx64, int64_t k)
{
    return idx64 ? static_cast<const int64_t *>(idx)[k] : (int64_t) static_cast<const int32_t *>(idx)[k];
}

// First entry position p in [0, n) with idx[p] >= key (idx ascending), found by the whole
// workgroup: each round probes 1024 evenly spaced positions of the remaining range.
__device__ int64_t block_lower_bound(const void *idx, int idx64, int64_t n, int64_t key)
{
    int64_t lo = 0, hi = n;  // the answer lies in [lo, hi]
    for (int round = 0; round < 8 && lo < hi; ++round) {
        const int64_t step = (hi - lo + kThreads - 1) / kThreads;
        const int64_t p = lo + (int64_t)threadIdx.x * step;
        const bool less = p < hi && flat_at(idx, idx64, p) < key;
        const int64_t c = __syncthreads_count(less);
        if (step == 1) return lo + c;
        if (c == 0) return lo;
        const int64_t nlo = lo + (c - 1) * step + 1;
        hi = hi < lo + c * step ? hi : lo + c * step;
        lo = nlo;
    }
    return lo;
}

// The 16-bit G-dtype encoding of entry e's product operand: the integer code for bits 4 / 8
// (exact), or the stored value rounded to G's dtype for bits 0 (the reference casts the values to
// G's dtype before its sparse product).
__device__ __forceinline__ uint32_t entry_operand(const TileArgs &a, int64_t e)
{
    float v;
    if (a.bits == 8) {
        v = (float)static_cast<const int8_t *>(a.data)[e];
    } else if (a.bits == 4) {
        const uint32_t b = static_cast<const uint8_t *>(a.data)[e >> 1];
        const int n = (int)((e & 1) ? (b >> 4) : (b & 0xfu));
        v = (float)(n > 7 ? n - 16 : n);
    } else {
        v = load_any(a.data, a.val_dt, e);
    }
    return a.g_dt == STACR_DTYPE_BF16 ? f_to_bf16_bits(v) : f_to_f16_bits(v);
}

__device__ __forceinline__ float g16_to_f(uint32_t v, int g_dt)
{
    return g_dt == STACR_DTYPE_BF16 ? bf16_bits_to_f(v) : f16_bits_to_f(v);
}

// ------------------------------------------------------------------ the plan
__global__ __launch_bounds__(kThreads) void k_tile_plan(TileArgs a)
{
    __shared__ uint32_t s_cnt[kPartMax];        // sample counts, then light counts of the block
    __shared__ int32_t s_slot[kPartMax];         // column slot of each feature of the part, or -1
    __shared__ uint32_t s_mask[kPartMax * 16];   // light rows of each feature (512-bit bitmaps)
    __shared__ uint16_t s_bt[kNC * kTB];         // the block's column tile
    __shared__ uint32_t s_tot[kThreads / 64];
    __shared__ uint32_t s_hist[kTB + 2];          // counts of the sample counts (0..512)
    __shared__ uint32_t s_pick[2];
    __shared__ int32_t s_colfeat[kNC];

    const int b = blockIdx.x, part = blockIdx.y, tid = threadIdx.x;
    const int64_t plo = (int64_t)part * a.part_w;
    const int pw = (int)(a.d_in - plo < a.part_w ? a.d_in - plo : a.part_w);
    const int64_t block_elems = (int64_t)kTB * a.d_in;

    if (!a.sparse) goto pack_coefficients;
    {
    // ---- entry ranges: the sample (block 0) and this block
    const int64_t e_s1 = block_lower_bound(a.idx, a.idx64, a.nnz, block_elems);
    const int64_t e_b0 = b == 0 ? 0 : block_lower_bound(a.idx, a.idx64, a.nnz, (int64_t)b * block_elems);
    const int64_t e_b1 = b == 0 ? e_s1 : block_lower_bound(a.idx, a.idx64, a.nnz, (int64_t)(b + 1) * block_elems);

    // ---- column features of the part, from the sample's counts
    for (int f = tid; f < kPartMax; f += kThreads) s_cnt[f] = 0u;
    for (int h = tid; h < kTB + 2; h += kThreads) s_hist[h] = 0u;
    __syncthreads();
    for (int64_t e = tid; e < e_s1; e += kThreads) {
        const int64_t f = flat_at(a.idx, a.idx64, e) % a.d_in - plo;
        if (f >= 0 && f < pw) atomicAdd(&s_cnt[f], 1u);
    }
    __syncthreads();
    // the count c32 of the 32nd feature (counts at least kMinColCount), then the features above
    // it and the first `need` (by feature) at it
    if (tid < pw && s_cnt[tid] >= (uint32_t)kMinColCount) atomicAdd(&s_hist[s_cnt[tid] > kTB ? kTB : s_cnt[tid]], 1u);
    __syncthreads();
    if (tid == 0) {
        uint32_t above = 0, c32 = 0xffffffffu, need = 0;
        for (int c = kTB; c >= kMinColCount; --c) {
            const uint32_t h = s_hist[c];
            if (above + h >= (uint32_t)kNC) {
                c32 = (uint32_t)c;
                need = kNC - above;
                break;
            }
            above += h;
        }
        if (c32 == 0xffffffffu) {  // fewer than 32 candidates: take every one
            c32 = kMinColCount;
            need = 0xffffffffu;
        }
        s_pick[0] = c32;
        s_pick[1] = need;
    }
    __syncthreads();
    const uint32_t c32 = s_pick[0], need = s_pick[1];
    const uint32_t mycnt = tid < pw ? s_cnt[tid] : 0u;
    const bool at_cut = mycnt == c32 && mycnt >= (uint32_t)kMinColCount;
    uint32_t n_at;
    const uint32_t rank_at = block_exclusive_scan<kThreads>(at_cut ? 1u : 0u, s_tot, &n_at);
    const bool is_col = tid < pw && ((mycnt > c32 && mycnt >= (uint32_t)kMinColCount) || (at_cut && rank_at < need));
    uint32_t n_col;
    const uint32_t slot = block_exclusive_scan<kThreads>(is_col ? 1u : 0u, s_tot, &n_col);
    if (tid < kPartMax) s_slot[tid] = is_col ? (int32_t)slot : -1;
    if (tid < kNC) s_colfeat[tid] = -1;
    __syncthreads();
    if (is_col) s_colfeat[slot] = tid;
    __syncthreads();
    if (b == 0 && tid < kNC) a.colmap[part * kNC + tid] = s_colfeat[tid];

    // ---- this block's entries: the column tile and the light bitmaps
    for (int i = tid; i < kNC * kTB; i += kThreads) s_bt[i] = 0;
    for (int i = tid; i < kPartMax * 16; i += kThreads) s_mask[i] = 0u;
    __syncthreads();
    const int64_t t_base = (int64_t)b * kTB;
    uint32_t before_part = 0;  // entries of this block in lower parts: where the part's records start
    for (int64_t e = e_b0 + tid; e < e_b1; e += kThreads) {
        const int64_t flat = flat_at(a.idx, a.idx64, e);
        const int64_t t = flat / a.d_in, f = flat - t * a.d_in - plo;
        const int64_t tl64 = t - t_base;
        if (tl64 < 0 || tl64 >= kTB) continue;  // only indices inside the block (valid input has no other)
        before_part += f < 0;
        if (f < 0 || f >= pw) continue;
        const int tl = (int)tl64;
        const int s = s_slot[f];
        if (s >= 0) s_bt[s * kTB + tl] = (uint16_t)entry_operand(a, e);
        else atomicOr(&s_mask[f * 16 + (tl >> 5)], 1u << (tl & 31));
    }
    __syncthreads();
    uint32_t all_before;
    (void)block_exclusive_scan<kThreads>(before_part, s_tot, &all_before);
    // light count of each feature, their offsets
    uint32_t cnt = 0;
    if (tid < pw) {
#pragma unroll
        for (int w = 0; w < 16; ++w) cnt += __popc(s_mask[tid * 16 + w]);
    }
    uint32_t n_light;
    const uint32_t off = block_exclusive_scan<kThreads>(cnt, s_tot, &n_light);
    uint32_t *loff = a.loff + ((int64_t)b * a.n_parts + part) * kOffWords;
    if (tid < pw) loff[tid] = off;
    if (tid == 0) loff[pw] = n_light;  // the part's end (pw may be 1024, past the last thread)
    // regions are disjoint and ordered by (block, part); shifting region r by 3 r and rounding up
    // to 4 keeps them disjoint and makes every start 16-byte aligned for the staging loads
    const uint32_t region = (uint32_t)(b * a.n_parts + part);
    const uint32_t base = ((uint32_t)e_b0 + all_before + 3u * region + 3u) & ~3u;
    if (tid == 0) a.hdr[b * a.n_parts + part] = TileHdr{base, n_light, {0u, 0u}};
    if (tid < kPartMax) s_cnt[tid] = tid < pw ? off : 0u;
    __syncthreads();
    // each light entry at its feature's offset + the feature's light entries in earlier rows
    for (int64_t e = e_b0 + tid; e < e_b1; e += kThreads) {
        const int64_t flat = flat_at(a.idx, a.idx64, e);
        const int64_t t = flat / a.d_in, f = flat - t * a.d_in - plo;
        const int64_t tl64 = t - t_base;
        if (tl64 < 0 || tl64 >= kTB || f < 0 || f >= pw || s_slot[f] >= 0) continue;
        const int tl = (int)tl64;
        uint32_t r = __popc(s_mask[f * 16 + (tl >> 5)] & ((1u << (tl & 31)) - 1u));
        for (int w = 0; w < (tl >> 5); ++w) r += __popc(s_mask[f * 16 + w]);
        a.light[base + s_cnt[f] + r] = (uint32_t)tl | (entry_operand(a, e) << 16);
    }
    // the column tile, coalesced
    uint4 *bt = reinterpret_cast<uint4 *>(a.bt + ((int64_t)b * a.n_parts + part) * kNC * kTB);
    const uint4 *sb = reinterpret_cast<const uint4 *>(s_bt);
    for (int i = tid; i < kNC * kTB / 8; i += kThreads) bt[i] = sb[i];

    }
pack_coefficients:
    // ---- the block's coefficients, transposed, with the ones column (part 0 only)
    if (part == 0) {
        const uint16_t *c = static_cast<const uint16_t *>(a.coeff);
        const uint32_t one = a.g_dt == STACR_DTYPE_BF16 ? 0x3f80u : 0x3c00u;
        uint16_t *cp = a.cp + (int64_t)b * a.ncol * kTB;
        for (int i = tid; i < a.ncol * kTB; i += kThreads) {
            const int col = i / kTB, tl = i - col * kTB;
            const int64_t t = (int64_t)b * kTB + tl;
            uint16_t v = 0;
            if (t < a.rows) {
                if (col < a.rank) v = c[t * a.rank + col];
                else if (col == a.bias_col) v = (uint16_t)one;
            }
            cp[i] = v;
        }
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

// 16 bytes per lane from `src` into LDS at `wave_dst` + 16 * lane (wave_dst wave-uniform)
__device__ __forceinline__ void async_copy16(const void *src, void *wave_dst)
{
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)wave_dst, 16, 0, 0);
}

// LDS layout of one buffer (byte offsets)
template <int NCOL, bool SP>
struct TileLds {
    static constexpr size_t g = 0;                                   // [kTB][16] u16
    static constexpr size_t c = g + (size_t)kTB * kOS * 2;           // [NCOL][kTB] u16
    static constexpr size_t bt = c + (size_t)NCOL * kTB * 2;         // [kNC][kTB] u16
    static constexpr size_t light = bt + (SP ? (size_t)kNC * kTB * 2 : 0);  // [kLightCap] u32
    static constexpr size_t off = light + (SP ? (size_t)kLightCap * 4 : 0); // [kOffWords] u32
    static constexpr size_t size = off + (SP ? (size_t)kOffWords * 4 : 0);
    // after the stream: the per-wave tiles [16 waves][16][16] f32 for M and the two column tiles
    static constexpr size_t red = 0;
    static constexpr size_t mfin = red + (size_t)3 * 16 * 256 * 4;
    static constexpr size_t cfin = mfin + (size_t)256 * 4;
    static constexpr size_t slots = cfin + (size_t)2 * 256 * 4;
    static constexpr size_t reduce_end = slots + (size_t)kPartMax * 4;
    static constexpr size_t total = 2 * size > reduce_end ? 2 * size : reduce_end;
    static_assert(size % 1024 == 0, "buffers start on 1 KiB boundaries");
    static_assert(total <= 160 * 1024, "fits the CU's LDS");
};

template <int DT, int NCOL, bool SP>
__global__ __launch_bounds__(kThreads) void k_tile_grad(TileArgs a)
{
    using L = TileLds<NCOL, SP>;
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // workgroup -> (o-slab, part): consecutive logical ids share an XCD (ids are dealt to the 8 XCDs
    // round-robin), so the o-slabs and parts that read the same G lines meet in one L2
    const int nwg = gridDim.x;
    int logical = blockIdx.x;
    if (nwg % 8 == 0) logical = (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int part = logical % a.n_parts;
    const int64_t o0 = (int64_t)(logical / a.n_parts) * kOS;
    const int64_t plo = (int64_t)part * a.part_w;
    const int pw = (int)(a.d_in - plo < a.part_w ? a.d_in - plo : a.part_w);
    const int nb = a.n_blocks;
    const int g_dt = a.g_dt;

    const uint16_t *g = static_cast<const uint16_t *>(a.g);
    const int64_t last_row = a.rows - 1;

    // this lane's source row of the G tile: row 32 wave + lane / 2, 8 outputs at half lane & 1.
    // `h` is the block's header, loaded one iteration earlier so its latency never delays the copies.
    auto issue = [&](int blk, int buf, const TileHdr &h) {
        unsigned char *B = lds + (size_t)buf * L::size;
        int64_t t = (int64_t)blk * kTB + 32 * wave + (lane >> 1);
        t = t < last_row ? t : last_row;  // rows past the end repeat the last (their C is zero)
        async_copy16(g + t * a.d_out + o0 + 8 * (lane & 1), B + L::g + (size_t)wave * 1024);
        if (wave < NCOL) async_copy16(a.cp + ((int64_t)blk * NCOL + wave) * kTB + 8 * lane, B + L::c + (size_t)wave * 1024);
        if constexpr (SP) {
            const uint16_t *bt = a.bt + ((int64_t)blk * a.n_parts + part) * kNC * kTB;
            async_copy16(bt + (size_t)wave * 512 + 8 * lane, B + L::bt + (size_t)wave * 1024);
            async_copy16(bt + (size_t)(wave + 16) * 512 + 8 * lane, B + L::bt + (size_t)(wave + 16) * 1024);
            if (wave < 8) async_copy16(a.light + h.light_base + 256 * wave + 4 * lane, B + L::light + (size_t)wave * 1024);
            else if (wave < 13)
                async_copy16(a.loff + ((int64_t)blk * a.n_parts + part) * kOffWords + 256 * (wave - 8) + 4 * lane,
                             B + L::off + (size_t)(wave - 8) * 1024);
        }
    };

    f32x4 acc_m = {0.f, 0.f, 0.f, 0.f}, acc_c0 = acc_m, acc_c1 = acc_m;
    float s[kOS];
#pragma unroll
    for (int o = 0; o < kOS; ++o) s[o] = 0.f;

    const TileHdr zero_hdr{0u, 0u, {0u, 0u}};
    auto header = [&](int blk) { return SP && blk < nb ? a.hdr[blk * a.n_parts + part] : zero_hdr; };
    TileHdr h_cur = header(0);
    issue(0, 0, h_cur);
    TileHdr h_next = header(1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int blk = 0; blk < nb; ++blk) {
        const int buf = blk & 1;
        if (blk + 1 < nb) issue(blk + 1, buf ^ 1, h_next);
        const TileHdr h_blk = h_cur;
        h_cur = h_next;
        h_next = header(blk + 2);
        const unsigned char *B = lds + (size_t)buf * L::size;
        const uint16_t *gt = reinterpret_cast<const uint16_t *>(B + L::g);
        // G^T[o][t0 .. t0 + 7], o = lane % 16, t0 = 32 wave + 8 (lane / 16): two transposing reads
        // (in a 16-lane group lane m addresses row r0 + m / 4, outputs 4 (m % 4) .. + 3, and lane n
        // receives G[r0 + j][n], j = 0..3)
        const int kk = 32 * wave + 8 * (lane >> 4);
        const uint16_t *pa = gt + (kk + ((lane & 15) >> 2)) * kOS + (lane & 3) * 4;
        const uint2 lo = lds_tr16(pa), hi = lds_tr16(pa + 4 * kOS);
        const uint4 av = make_uint4(lo.x, lo.y, hi.x, hi.y);
        const int n = lane & 15;
        const uint16_t *ct = reinterpret_cast<const uint16_t *>(B + L::c);
        const uint4 bc = n < NCOL ? *reinterpret_cast<const uint4 *>(ct + n * kTB + kk) : make_uint4(0u, 0u, 0u, 0u);
        acc_m = mfma16<DT>(av, bc, acc_m);
        if constexpr (SP) {
            const uint16_t *bt = reinterpret_cast<const uint16_t *>(B + L::bt);
            const uint4 b0 = *reinterpret_cast<const uint4 *>(bt + n * kTB + kk);
            const uint4 b1 = *reinterpret_cast<const uint4 *>(bt + (16 + n) * kTB + kk);
            acc_c0 = mfma16<DT>(av, b0, acc_c0);
            acc_c1 = mfma16<DT>(av, b1, acc_c1);
            // this thread's feature: its light entries of the block
            if (tid < pw) {
                const uint32_t *off = reinterpret_cast<const uint32_t *>(B + L::off);
                const uint32_t *lrec = reinterpret_cast<const uint32_t *>(B + L::light);
                // the owner's range, clamped to the block's records whatever the offsets hold
                const uint32_t k1 = off[tid + 1] < h_blk.light_count ? off[tid + 1] : h_blk.light_count;
                const uint32_t k0 = off[tid] < k1 ? off[tid] : k1;
                const uint32_t gbase = h_blk.light_base;
#pragma unroll 2
                for (uint32_t k = k0; k < k1; ++k) {
                    const uint32_t rec = k < (uint32_t)kLightCap ? lrec[k] : a.light[gbase + k];
                    const float v = g16_to_f(rec >> 16, g_dt);
                    const uint4 *row = reinterpret_cast<const uint4 *>(gt + (rec & 511u) * kOS);
                    const uint4 w0 = row[0], w1 = row[1];
                    const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int o = 0; o < 8; ++o) {
                        s[2 * o] = fmaf(v, g16_to_f(w[o] & 0xffffu, g_dt), s[2 * o]);
                        s[2 * o + 1] = fmaf(v, g16_to_f(w[o] >> 16, g_dt), s[2 * o + 1]);
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the next block's tiles have landed
        __syncthreads();                // and every wave is done with this block's buffer
    }

    // ---- reduce the per-wave tiles over the waves, in wave order
    float *red = reinterpret_cast<float *>(lds + L::red);
    float *mfin = reinterpret_cast<float *>(lds + L::mfin);
    float *cfin = reinterpret_cast<float *>(lds + L::cfin);
    int32_t *slots = reinterpret_cast<int32_t *>(lds + L::slots);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * (lane >> 4) + r;  // D layout: rows 4 (lane / 16) .. + 3 of column lane % 16
        red[(0 * 16 + wave) * 256 + row * 16 + (lane & 15)] = acc_m[r];
        red[(1 * 16 + wave) * 256 + row * 16 + (lane & 15)] = acc_c0[r];
        red[(2 * 16 + wave) * 256 + row * 16 + (lane & 15)] = acc_c1[r];
    }
    if (tid < kPartMax) slots[tid] = -1;
    __syncthreads();
    if (SP && tid < kNC) {
        const int f = a.colmap[part * kNC + tid];
        if (f >= 0 && f < kPartMax) slots[f] = tid;
    }
    for (int i = tid; i < 3 * 256; i += kThreads) {
        const int tile = i / 256, e = i % 256;
        float sum = 0.f;
        for (int w = 0; w < 16; ++w) sum += red[(tile * 16 + w) * 256 + e];
        if (tile == 0) mfin[e] = sum;
        else cfin[(tile - 1) * 256 + e] = sum;  // [tile][o][n]: slot 16 (tile - 1) + n
    }
    __syncthreads();

    // ---- dW tile: M Q^T + scale (light + column sums), one rounding; dbias from M[:, bias_col]
    // the scale exists only with residual entries (the C ABI checks it then); without them the
    // sparse sums are zero and no scale is read
    const float scale = SP && a.bits ? *a.scale : 1.f;
    if (tid < pw) {
        const int64_t i = plo + tid;
        const uint16_t *q = static_cast<const uint16_t *>(a.q);
        const int slot = SP ? slots[tid] : -1;
        float out[kOS];
#pragma unroll
        for (int o = 0; o < kOS; ++o) {
            const float col = slot >= 0 ? cfin[(slot >> 4) * 256 + o * 16 + (slot & 15)] : 0.f;
            out[o] = scale * (s[o] + col);
        }
        // + sum_j M[o][j] Q[i][j], one rank column at a time (the M reads are LDS broadcasts)
        for (int j = 0; j < a.rank; ++j) {
            const float qj = g16_to_f(q[i * a.rank + j], g_dt);
#pragma unroll
            for (int o = 0; o < kOS; ++o) out[o] = fmaf(mfin[o * 16 + j], qj, out[o]);
        }
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
    if (a.dbias && part == 0 && tid < kOS) store_any(a.dbias, a.db_dt, o0 + tid, mfin[tid * 16 + a.bias_col]);
}

}  // namespace

// ------------------------------------------------------------------ host side
namespace {

struct TileGeom {
    int n_blocks, n_parts, part_w, ncol, bias_col;
    bool sparse;
};

bool tile_geom(const StacrGradArgs &a, TileGeom *g)
{
    if (a.dtype != STACR_DTYPE_BF16 && a.dtype != STACR_DTYPE_F16) return false;
    if (a.rows < 1 || a.d_in < 1 || a.d_out < kOS || a.d_out % kOS) return false;
    const int cols = a.rank + (a.dbias ? 1 : 0);
    if (cols > 16) return false;
    if ((uintptr_t)a.g % 16) return false;
    if (a.nnz > 0 && a.index_bytes != 4 && a.index_bytes != 8) return false;
    g->n_blocks = (int)((a.rows + kTB - 1) / kTB);
    g->n_parts = (int)((a.d_in + kPartMax - 1) / kPartMax);
    g->part_w = (int)((a.d_in + g->n_parts - 1) / g->n_parts);
    g->ncol = cols <= 8 ? 8 : 16;
    g->bias_col = a.dbias ? a.rank : -1;
    g->sparse = a.nnz > 0;
    return true;
}

enum { TW_CP, TW_BT, TW_LIGHT, TW_LOFF, TW_HDR, TW_COLMAP, TW_N };

size_t tile_layout(const StacrGradArgs &a, const TileGeom &g, size_t *off)
{
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    const size_t regions = (size_t)g.n_blocks * g.n_parts;
    take(TW_CP, (size_t)g.n_blocks * g.ncol * kTB * 2);
    take(TW_BT, g.sparse ? regions * kNC * kTB * 2 : 0);
    take(TW_LIGHT, g.sparse ? ((size_t)a.nnz + 3 * regions + 3 + kLightCap) * 4 : 0);
    take(TW_LOFF, g.sparse ? regions * kOffWords * 4 : 0);
    take(TW_HDR, g.sparse ? regions * sizeof(TileHdr) : 0);
    take(TW_COLMAP, g.sparse ? (size_t)g.n_parts * kNC * 4 : 0);
    return cur;
}

template <typename K>
void allow_lds(K kernel, size_t bytes, std::once_flag &once)
{
    std::call_once(once, [&] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)bytes);
    });
}

template <int DT, int NCOL, bool SP>
int launch_tile_grad(const TileArgs &t, int nwg, hipStream_t s)
{
    static std::once_flag once;
    constexpr size_t bytes = TileLds<NCOL, SP>::total;
    allow_lds(k_tile_grad<DT, NCOL, SP>, bytes, once);
    stacr_launch("k_dw_fused", s, [&] { k_tile_grad<DT, NCOL, SP><<<nwg, kThreads, bytes, s>>>(t); });
    return stacr_hip_check(hipGetLastError(), "weight_grad matrix-core kernel");
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
    return tile_geom(a, &g) ? tile_layout(a, g, off) : 0;
}

size_t stacr_tiles_ws_bound(int64_t rows, int64_t d_out, int64_t d_in, int64_t nnz)
{
    if (rows < 1 || d_in < 1 || d_out < kOS) return 0;
    StacrGradArgs a{};
    a.rows = rows;
    a.d_out = d_out;
    a.d_in = d_in;
    a.nnz = nnz;
    TileGeom g;
    g.n_blocks = (int)((rows + kTB - 1) / kTB);
    g.n_parts = (int)((d_in + kPartMax - 1) / kPartMax);
    g.part_w = (int)((d_in + g.n_parts - 1) / g.n_parts);
    g.ncol = 16;  // the widest coefficient tile (rank + bias column up to 16)
    g.bias_col = -1;
    g.sparse = nnz > 0;
    size_t off[TW_N];
    return tile_layout(a, g, off);
}

int stacr_tiles_launch(const StacrGradArgs &a)
{
    TileGeom g;
    if (!tile_geom(a, &g)) return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_weight_grad: matrix-core path not applicable");
    size_t off[TW_N];
    const size_t need = tile_layout(a, g, off);
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
    t.cp = reinterpret_cast<uint16_t *>(ws + off[TW_CP]);
    t.bt = g.sparse ? reinterpret_cast<uint16_t *>(ws + off[TW_BT]) : nullptr;
    t.light = g.sparse ? reinterpret_cast<uint32_t *>(ws + off[TW_LIGHT]) : nullptr;
    t.loff = g.sparse ? reinterpret_cast<uint32_t *>(ws + off[TW_LOFF]) : nullptr;
    t.hdr = g.sparse ? reinterpret_cast<TileHdr *>(ws + off[TW_HDR]) : nullptr;
    t.colmap = g.sparse ? reinterpret_cast<int32_t *>(ws + off[TW_COLMAP]) : nullptr;
    t.sparse = g.sparse ? 1 : 0;
    hipStream_t s = a.stream;
    const dim3 pgrid((unsigned)g.n_blocks, g.sparse ? (unsigned)g.n_parts : 1u);
    stacr_launch("k_dw_plan", s, [&] { k_tile_plan<<<pgrid, kThreads, 0, s>>>(t); });
    int rc = stacr_hip_check(hipGetLastError(), "weight_grad plan");
    if (rc) return rc;
    const int nwg = (int)(a.d_out / kOS) * g.n_parts;
    const bool bf = a.dtype == STACR_DTYPE_BF16;
    if (g.sparse) {
        if (g.ncol == 8)
            return bf ? launch_tile_grad<STACR_DTYPE_BF16, 8, true>(t, nwg, s) : launch_tile_grad<STACR_DTYPE_F16, 8, true>(t, nwg, s);
        return bf ? launch_tile_grad<STACR_DTYPE_BF16, 16, true>(t, nwg, s) : launch_tile_grad<STACR_DTYPE_F16, 16, true>(t, nwg, s);
    }
    if (g.ncol == 8)
        return bf ? launch_tile_grad<STACR_DTYPE_BF16, 8, false>(t, nwg, s) : launch_tile_grad<STACR_DTYPE_F16, 8, false>(t, nwg, s);
    return bf ? launch_tile_grad<STACR_DTYPE_BF16, 16, false>(t, nwg, s) : launch_tile_grad<STACR_DTYPE_F16, 16, false>(t, nwg, s);
}
