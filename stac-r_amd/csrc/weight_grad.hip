// Weight gradient from the saved factors: dW = (G^T C) Q^T + G^T R_s, dbias = sum_t G.
//
// Restates stacr/layers.py:172-198.  Accumulation is fp32 and dW is rounded once to the weight
// dtype (the reference rounds the d_out x r product and the low-rank term to G's dtype before
// adding its fp32 sparse correction; one rounding at the end is the more accurate of the two).
// Residual values are dequantized exactly as QuantizedValues.dequantize(fp32) does
// (stacr/quant.py:17-21,40-46): float(q) * scale in fp32.
//
// Two launches:
//   k_rowptr   ascending flat indices -> first residual entry of every token row (CSR offsets)
//   k_dw_fused one streaming pass over G.  A workgroup owns 16 output features (one "o-slab") and
//              a slab of at most 1024 input features; it reads G[:, o-slab] once, row block by
//              row block, and
//                * accumulates M = G^T [C | 1] in registers (packed bf16/fp16 dot products, or
//                  fp32 FMAs), which also yields dbias;
//                * adds v * G[t, o] into an LDS accumulator S[i][o] for every residual entry
//                  (t, i, v) of its rows (LDS float atomics);
//              then reduces M across its threads and writes dW = M Q^T + S for its tile.
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kOSlab = 16;         // output features per workgroup
constexpr int kAccPitch = 17;      // LDS row pitch of the accumulator: odd, so random rows hit
                                   // different banks (a pitch of 16 maps every row to 2 banks)
constexpr int kMaxISlab = 1024;    // input features per workgroup: 1024 x 17 fp32 = 68 KiB of LDS
constexpr int kBwdThreads = 512;   // 8 waves
constexpr int kPiece = 32;         // residual entries per register-accumulated piece

template <int DT, int R>
struct GradCfg {
    using T = typename Act<DT>::T;
    static constexpr bool k16 = sizeof(T) == 2;
    // output features per thread: keeps the M accumulator at <= 72 fp32 registers
    static constexpr int OT = k16 ? (R <= 8 ? 8 : (R == 16 ? 4 : 2)) : (R <= 16 ? 4 : 2);
    static constexpr int OG = kOSlab / OT;          // threads sharing one token row
    static constexpr int TP = kBwdThreads / OG;     // token pairs per block
    static constexpr int TB = 2 * TP;               // token rows per block
    static constexpr int VB = OT * (int)sizeof(T);  // bytes per thread per row
    static constexpr int NV = OT * (R + 1);         // accumulator values per thread
    // residual entries prefetched per thread and bucketed in LDS per round (8 B per entry for
    // fp32 G, 4 B packed otherwise); pieces of features split over several pieces per round
    static constexpr int EPT = k16 ? 8 : 4;
    static constexpr int ENT_CAP = EPT * kBwdThreads;
    static constexpr int HEAVY = 2 * ENT_CAP / kPiece;
};

template <int B> struct Vec;
template <> struct Vec<4> { using type = uint32_t; static constexpr int n = 1; };
template <> struct Vec<8> { using type = uint2; static constexpr int n = 2; };
template <> struct Vec<16> { using type = uint4; static constexpr int n = 4; };

template <int B>
__device__ __forceinline__ void load_words(const void *p, bool ok, uint32_t (&w)[Vec<B>::n])
{
    using V = typename Vec<B>::type;
    if (!ok) {
#pragma unroll
        for (int k = 0; k < Vec<B>::n; ++k) w[k] = 0u;
        return;
    }
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
// 16-byte vector load is used when the whole vector is in range and aligned.
template <int DT, int VB>
__device__ __forceinline__ void load_g(const typename Act<DT>::T *row, int64_t ob, int64_t d_out, bool row_ok,
                                       bool vec_ok, uint32_t (&w)[Vec<VB>::n])
{
    using T = typename Act<DT>::T;
    constexpr int OT = VB / (int)sizeof(T);
    if (row_ok && vec_ok && ob + OT <= d_out) {
        load_words<VB>(row + ob, true, w);
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

template <int IDX64>
__device__ __forceinline__ int64_t flat_at(const void *idx, int64_t k)
{
    return IDX64 ? static_cast<const int64_t *>(idx)[k] : (int64_t) static_cast<const int32_t *>(idx)[k];
}

__device__ __forceinline__ float dequant(const void *data, const float *scale, int bits, int val_dt, int64_t e)
{
    if (bits == 8) return (float)static_cast<const int8_t *>(data)[e] * scale[0];
    if (bits == 4) {
        const uint32_t byte = static_cast<const uint8_t *>(data)[e >> 1];
        int n = (int)((e & 1) ? (byte >> 4) : (byte & 0xfu));
        n = n > 7 ? n - 16 : n;
        return (float)n * scale[0];
    }
    return load_any(data, val_dt, e);
}

// rowptr[t] = first entry whose flat index is >= t * d_in (t = 0..rows).  Indices are ascending
// (stacr_save writes them so); an index outside rows x d_in maps past the last row.
template <int IDX64>
__global__ void k_rowptr(const void *__restrict__ idx, int64_t nnz, int64_t d_in, int64_t rows,
                         uint32_t *__restrict__ rowptr)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    const int64_t lim = rows * d_in;
    const int64_t f = flat_at<IDX64>(idx, e);
    const int64_t t = (f < 0 || f >= lim) ? rows : f / d_in;
    int64_t tprev = -1;
    if (e) {
        const int64_t fp = flat_at<IDX64>(idx, e - 1);
        tprev = (fp < 0 || fp >= lim) ? rows : fp / d_in;
    }
    for (int64_t tt = tprev + 1; tt <= t && tt < rows; ++tt) rowptr[tt] = (uint32_t)e;
    if (e == nnz - 1)
        for (int64_t tt = t < rows ? t + 1 : rows; tt <= rows; ++tt) rowptr[tt] = (uint32_t)nnz;
}

struct FusedArgs {
    const void *g, *coeff, *q;
    int64_t rows, d_out, d_in;
    int rank;
    const void *idx;
    const void *data;
    const float *scale;
    int bits, val_dt;
    int64_t nnz;
    const uint32_t *rowptr;
    int64_t n_slabs, n_parts, i_span;  // i_span: input features per part (<= kMaxISlab)
    int vec_ok;                        // G rows are 16-byte aligned for whole-vector loads
    int transposed;
    void *dw;
    int dw_dt;
    void *dbias;
    int db_dt;
};


// Shared-memory carve-up of k_dw_fused (byte offsets; sized for the widest configuration).
template <int DT, int R>
struct FusedLds {
    using C = GradCfg<DT, R>;
    using T = typename C::T;
    static constexpr bool k16 = C::k16;
    static constexpr size_t s_acc = 0;                                            // [1024][kAccPitch] f32
    static constexpr size_t s_gtile = s_acc + (size_t)kMaxISlab * kAccPitch * 4;  // [TB][16] T
    static constexpr size_t s_ctile = s_gtile + (size_t)C::TB * kOSlab * sizeof(T);  // [TB][R] T
    static constexpr size_t s_ent = s_ctile + (((size_t)C::TB * R * sizeof(T) + 15) & ~(size_t)15);
    static constexpr size_t ent_bytes = k16 ? 4 : 8;                              // packed (t, v)
    static constexpr size_t s_cols = s_ent + (size_t)C::ENT_CAP * ent_bytes;      // 5 x [1025] u32
    static constexpr size_t s_scr = s_cols + (size_t)5 * (kMaxISlab + 1) * 4;     // [HEAVY][16] f32
    static constexpr size_t end = s_scr + (size_t)C::HEAVY * kOSlab * 4;
};

template <int DT, int R, int IDX64>
__global__ __launch_bounds__(kBwdThreads) void k_dw_fused(FusedArgs a)
{
    using C = GradCfg<DT, R>;
    using T = typename C::T;
    using L = FusedLds<DT, R>;
    constexpr int OT = C::OT, OG = C::OG, TP = C::TP, TB = C::TB, VB = C::VB, NW = Vec<C::VB>::n;
    constexpr int CPT = (TB * R + kBwdThreads - 1) / kBwdThreads;  // C elements staged per thread
    constexpr int EPT = C::EPT, kEntCap = C::ENT_CAP;
    constexpr int NGRP = kBwdThreads / OG;                          // piece groups per pass

    extern __shared__ float lds[];
    char *base = reinterpret_cast<char *>(lds);
    float *acc = reinterpret_cast<float *>(base + L::s_acc);       // residual accumulator S[i][o]
    T *gtile = reinterpret_cast<T *>(base + L::s_gtile);            // G rows of the current block
    T *ctile = reinterpret_cast<T *>(base + L::s_ctile);            // C rows of the current block
    uint32_t *ent = reinterpret_cast<uint32_t *>(base + L::s_ent);  // bucketed entries
    uint32_t *cnt = reinterpret_cast<uint32_t *>(base + L::s_cols); // per column: entries,
    uint32_t *cstart = cnt + (kMaxISlab + 1);                       //   first bucket slot,
    uint32_t *ccur = cstart + (kMaxISlab + 1);                      //   placement cursor,
    uint32_t *tstart = ccur + (kMaxISlab + 1);                      //   first piece,
    uint32_t *hstart = tstart + (kMaxISlab + 1);                    //   first heavy-scratch slot
    float *scr = reinterpret_cast<float *>(base + L::s_scr);        // partials of split columns
    float *mred = reinterpret_cast<float *>(base + L::s_gtile);     // reused after the stream
    __shared__ uint32_t s_tot[kBwdThreads / 64];

    // workgroup -> (o-slab, part); consecutive logical ids land on the same XCD (ids are dealt
    // round-robin over 8 XCDs), so the parts of a slab and neighbouring slabs share an L2
    const int64_t nwg = a.n_slabs * a.n_parts;
    int64_t lid = blockIdx.x;
    if (nwg % 8 == 0) lid = (int64_t)(blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int64_t slab = lid / a.n_parts, part = lid - slab * a.n_parts;
    const int64_t o0 = slab * kOSlab;
    const int64_t i0 = part * a.i_span;
    const int64_t i1 = min(i0 + a.i_span, a.d_in);
    const int ni = (int)(i1 - i0);

    const int og = threadIdx.x % OG, tp = threadIdx.x / OG;
    const int64_t ob = o0 + og * OT;                      // first output feature of this thread
    const bool o_ok = ob < a.d_out;                       // thread owns at least one output feature
    const bool vec_ok = a.vec_ok != 0;
    const T *g = static_cast<const T *>(a.g);
    const T *coeff = static_cast<const T *>(a.coeff);
    const bool sparse = a.nnz > 0;
    const float qscale = (sparse && a.bits) ? a.scale[0] : 1.f;  // residual codes are scaled at flush
    const uint32_t d_in = (uint32_t)a.d_in;
    const float inv_d = 1.f / (float)a.d_in;

    for (int i = threadIdx.x; i < ni * kAccPitch; i += kBwdThreads) acc[i] = 0.f;

    float m[OT][R + 1];
#pragma unroll
    for (int o = 0; o < OT; ++o)
#pragma unroll
        for (int j = 0; j <= R; ++j) m[o][j] = 0.f;

    // ---- everything a block needs is loaded one block ahead into registers
    uint32_t wa[NW], wb[NW];          // G rows t and t+1 (this thread's output features)
    T cpre[CPT];                      // C elements of the block (cooperative)
    uint32_t pf_off[EPT];             // residual entries: flat offset from the block start
    uint32_t pf_val[EPT];             //   value bits (G's 16-bit type, or fp32 for fp32 G)
    uint32_t pf_e0 = 0, pf_e1 = 0;    // entry range of the block
    // residual entries [lo, hi) (at most kEntCap) into pf_off / pf_val
    auto load_entries = [&](uint32_t lo, uint32_t hi, int64_t tb0) {
        const int64_t fbase = tb0 * a.d_in;
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            const uint32_t e = lo + threadIdx.x + k * kBwdThreads;
            if (e < hi) {
                pf_off[k] = (uint32_t)(flat_at<IDX64>(a.idx, e) - fbase);
                if (a.bits == 8 || a.bits == 4) {
                    int qv;
                    if (a.bits == 8) {
                        qv = static_cast<const int8_t *>(a.data)[e];
                    } else {
                        const uint32_t byte = static_cast<const uint8_t *>(a.data)[e >> 1];
                        qv = (int)((e & 1) ? (byte >> 4) : (byte & 0xfu));
                        qv = qv > 7 ? qv - 16 : qv;
                    }
                    pf_val[k] = C::k16 ? (uint32_t)Act<DT>::st((float)qv) : __float_as_uint((float)qv);
                } else {
                    const float v = load_any(a.data, a.val_dt, e);
                    pf_val[k] = C::k16 ? (uint32_t)Act<DT>::st(v) : __float_as_uint(v);
                }
            }
        }
    };
    auto prefetch_entries = [&](int64_t blk) {
        const int64_t tb0 = blk * TB;
        pf_e0 = a.rowptr[min(tb0, a.rows)];
        pf_e1 = a.rowptr[min(tb0 + TB, a.rows)];
        const uint32_t hi = pf_e1 - pf_e0 > (uint32_t)kEntCap ? pf_e0 + kEntCap : pf_e1;
        load_entries(pf_e0, hi, tb0);
    };
    auto prefetch_gc = [&](int64_t blk) {
        const int64_t tb0 = blk * TB, t = tb0 + 2 * tp;
        load_g<DT, VB>(g + t * a.d_out, ob, a.d_out, o_ok && t < a.rows, vec_ok, wa);
        load_g<DT, VB>(g + (t + 1) * a.d_out, ob, a.d_out, o_ok && t + 1 < a.rows, vec_ok, wb);
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int el = threadIdx.x + c * kBwdThreads;
            const int r = el / R, j = el - (el / R) * R;
            const int64_t row = tb0 + r;
            cpre[c] = (el < TB * R && j < a.rank && row < a.rows) ? coeff[row * a.rank + j] : (T)0;
        }
    };

    // One round: bucket the staged entries [lo, hi) of this block by input feature, cut every
    // feature's run into pieces of <= kPiece entries, accumulate each piece in registers, and add
    // it into S (directly when the feature has one piece; through the scratch otherwise).
    auto scatter_round = [&](uint32_t lo, uint32_t hi) {
        for (int c = threadIdx.x; c <= ni; c += kBwdThreads) {
            cnt[c] = 0u;
            ccur[c] = 0u;
        }
        __syncthreads();
        uint32_t mycol[EPT];
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            mycol[k] = 0xffffffffu;
            const uint32_t e = lo + threadIdx.x + k * kBwdThreads;
            if (e < hi) {
                const uint32_t off = pf_off[k];
                uint32_t tl = (uint32_t)((float)off * inv_d);  // off / d_in, corrected below
                if (tl * d_in > off) --tl;
                else if ((tl + 1) * d_in <= off) ++tl;
                const int64_t col = (int64_t)(off - tl * d_in) - i0;
                if (tl < (uint32_t)TB && col >= 0 && col < ni) {
                    mycol[k] = (uint32_t)col;
                    pf_off[k] = tl;  // keep the block-local row for placement
                    atomicAdd(&cnt[col], 1u);
                }
            }
        }
        __syncthreads();
        // prefix sums over features: bucket starts, piece starts, heavy-scratch starts
        {
            const int c0 = 2 * threadIdx.x;  // ni <= 1024: two features per thread
            const uint32_t n0 = c0 < ni ? cnt[c0] : 0u, n1 = c0 + 1 < ni ? cnt[c0 + 1] : 0u;
            const uint32_t p0 = (n0 + kPiece - 1) / kPiece, p1 = (n1 + kPiece - 1) / kPiece;
            const uint32_t h0 = p0 > 1 ? p0 : 0u, h1 = p1 > 1 ? p1 : 0u;
            uint32_t tot;
            const uint32_t se = block_exclusive_scan<kBwdThreads>(n0 + n1, s_tot, &tot);
            const uint32_t sp = block_exclusive_scan<kBwdThreads>(p0 + p1, s_tot, &tot);
            const uint32_t n_pieces = tot;
            const uint32_t sh = block_exclusive_scan<kBwdThreads>(h0 + h1, s_tot, &tot);
            if (c0 < ni) {
                cstart[c0] = se;
                tstart[c0] = sp;
                hstart[c0] = sh;
            }
            if (c0 + 1 < ni) {
                cstart[c0 + 1] = se + n0;
                tstart[c0 + 1] = sp + p0;
                hstart[c0 + 1] = sh + h0;
            }
            if (threadIdx.x == 0) tstart[ni] = n_pieces;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < EPT; ++k) {
            if (mycol[k] != 0xffffffffu) {
                const uint32_t pos = cstart[mycol[k]] + atomicAdd(&ccur[mycol[k]], 1u);
                if constexpr (C::k16) {
                    ent[pos] = (pf_off[k] << 16) | (pf_val[k] & 0xffffu);
                } else {
                    ent[2 * pos] = pf_off[k];
                    ent[2 * pos + 1] = pf_val[k];
                }
            }
        }
        __syncthreads();
        const uint32_t n_pieces = tstart[ni];
        if (o_ok) {
            const int grp = threadIdx.x / OG;
            for (uint32_t task = grp; task < n_pieces; task += NGRP) {
                int lo_c = 0, hi_c = ni;  // feature c with tstart[c] <= task < tstart[c + 1]
                while (hi_c - lo_c > 1) {
                    const int mid = (lo_c + hi_c) >> 1;
                    if (tstart[mid] <= task) lo_c = mid;
                    else hi_c = mid;
                }
                const int c = lo_c;
                const uint32_t piece = task - tstart[c];
                const uint32_t n = cnt[c];
                const uint32_t e_lo = cstart[c] + piece * kPiece;
                const uint32_t e_hi = cstart[c] + min(n, (piece + 1) * kPiece);
                float pacc[OT];
#pragma unroll
                for (int o = 0; o < OT; ++o) pacc[o] = 0.f;
                for (uint32_t e = e_lo; e < e_hi; ++e) {
                    if constexpr (C::k16) {
                        const uint32_t wv = ent[e];
                        const uint32_t tl = wv >> 16;
                        uint32_t gw[NW];
                        const uint32_t *src = reinterpret_cast<const uint32_t *>(gtile + tl * kOSlab + og * OT);
#pragma unroll
                        for (int k = 0; k < NW; ++k) gw[k] = src[k];
                        const uint32_t vlo = wv & 0xffffu, vhi = wv << 16;  // (v, 0) and (0, v)
#pragma unroll
                        for (int k = 0; k < NW; ++k) {
                            pacc[2 * k] = dot2<DT>(gw[k], vlo, pacc[2 * k]);
                            pacc[2 * k + 1] = dot2<DT>(gw[k], vhi, pacc[2 * k + 1]);
                        }
                    } else {
                        const uint32_t tl = ent[2 * e];
                        const float v = __uint_as_float(ent[2 * e + 1]);
                        const float *src = reinterpret_cast<const float *>(gtile) + tl * kOSlab + og * OT;
#pragma unroll
                        for (int o = 0; o < OT; ++o) pacc[o] = fmaf(src[o], v, pacc[o]);
                    }
                }
                const uint32_t npc = (n + kPiece - 1) / kPiece;
                if (npc == 1) {
                    float *dst = acc + c * kAccPitch + og * OT;
#pragma unroll
                    for (int o = 0; o < OT; ++o) dst[o] += pacc[o] * qscale;
                } else {
                    float *dst = scr + (hstart[c] + piece) * kOSlab + og * OT;
#pragma unroll
                    for (int o = 0; o < OT; ++o) dst[o] = pacc[o];
                }
            }
        }
        __syncthreads();
        // features split into several pieces: add their partials in piece order
        for (int w = threadIdx.x; w < ni * kOSlab; w += kBwdThreads) {
            const int c = w / kOSlab, o = w - c * kOSlab;
            const uint32_t npc = (cnt[c] + kPiece - 1) / kPiece;
            if (npc > 1 && o0 + o < a.d_out) {
                float s = 0.f;
                for (uint32_t p = 0; p < npc; ++p) s += scr[(hstart[c] + p) * kOSlab + o];
                acc[c * kAccPitch + o] += s * qscale;
            }
        }
    };

    const int64_t n_blocks = (a.rows + TB - 1) / TB;
    if (n_blocks > 0) {
        prefetch_gc(0);
        if (sparse) prefetch_entries(0);
    }
    for (int64_t blk = 0; blk < n_blocks; ++blk) {
        const int64_t t0 = blk * TB;
        uint32_t ca[NW], cb[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k) { ca[k] = wa[k]; cb[k] = wb[k]; }
        const uint32_t e0 = pf_e0, e1 = pf_e1;
        __syncthreads();  // previous block's LDS tiles fully consumed
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int el = threadIdx.x + c * kBwdThreads;
            if (el < TB * R) ctile[el] = cpre[c];
        }
        {   // G rows of the block for the residual pieces
            uint32_t *ga_dst = reinterpret_cast<uint32_t *>(gtile + (2 * tp) * kOSlab + og * OT);
            uint32_t *gb_dst = reinterpret_cast<uint32_t *>(gtile + (2 * tp + 1) * kOSlab + og * OT);
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                ga_dst[k] = ca[k];
                gb_dst[k] = cb[k];
            }
        }
        __syncthreads();
        if (blk + 1 < n_blocks) prefetch_gc(blk + 1);  // overlaps with this block's arithmetic
        // ---- low rank: m[o][j] += G[t][o] C[t][j] + G[t+1][o] C[t+1][j];  m[o][R] += G[t][o] + G[t+1][o]
        if constexpr (C::k16) {
            uint32_t pr[OT];  // (G[t][o], G[t+1][o]) pairs
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                pr[2 * k] = __builtin_amdgcn_perm(cb[k], ca[k], 0x05040100u);
                pr[2 * k + 1] = __builtin_amdgcn_perm(cb[k], ca[k], 0x07060302u);
            }
            const uint32_t *rowa = reinterpret_cast<const uint32_t *>(ctile + (2 * tp) * R);
            const uint32_t *rowb = reinterpret_cast<const uint32_t *>(ctile + (2 * tp + 1) * R);
            uint32_t cv[R];  // (C[t][j], C[t+1][j]) pairs
#pragma unroll
            for (int k = 0; k < R / 2; ++k) {
                const uint32_t xa = rowa[k], xb = rowb[k];
                cv[2 * k] = __builtin_amdgcn_perm(xb, xa, 0x05040100u);
                cv[2 * k + 1] = __builtin_amdgcn_perm(xb, xa, 0x07060302u);
            }
            const uint32_t ones = DT == STACR_DTYPE_BF16 ? 0x3f803f80u : 0x3c003c00u;
#pragma unroll
            for (int o = 0; o < OT; ++o) {
#pragma unroll
                for (int j = 0; j < R; ++j) m[o][j] = dot2<DT>(pr[o], cv[j], m[o][j]);
                m[o][R] = dot2<DT>(pr[o], ones, m[o][R]);
            }
        } else {
            float ga[OT], gb[OT];
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                ga[k] = __uint_as_float(ca[k]);
                gb[k] = __uint_as_float(cb[k]);
            }
            const float *cpa = reinterpret_cast<const float *>(ctile) + (2 * tp) * R;
            const float *cpb = cpa + R;
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const float c0 = cpa[j], c1 = cpb[j];
#pragma unroll
                for (int o = 0; o < OT; ++o) m[o][j] = fmaf(gb[o], c1, fmaf(ga[o], c0, m[o][j]));
            }
#pragma unroll
            for (int o = 0; o < OT; ++o) m[o][R] += ga[o] + gb[o];
        }
        if (!sparse) continue;
        // ---- residual entries of the block: first round from the prefetched registers; blocks
        // with more than kEntCap entries continue with synchronously loaded rounds
        const uint32_t hi0 = e1 - e0 > (uint32_t)kEntCap ? e0 + kEntCap : e1;
        scatter_round(e0, hi0);
        for (uint32_t lo = hi0; lo < e1; lo += kEntCap) {
            const uint32_t hi = e1 - lo > (uint32_t)kEntCap ? lo + kEntCap : e1;
            load_entries(lo, hi, t0);
            scatter_round(lo, hi);
        }
        if (blk + 1 < n_blocks) prefetch_entries(blk + 1);
    }
    __syncthreads();

    // ---- reduce m over the TP threads that share an output group, in a fixed order.
    // Two halves of the per-thread values in turn: every thread parks its half in LDS, 8 threads
    // per output sum TP/8 rows each, one thread per output adds the 8 partial sums.
    constexpr int HALF = (C::NV + 1) / 2;
    float *psum = mred + kBwdThreads * HALF;       // [8][OG * HALF]
    float *mfin = psum + 8 * OG * HALF;            // final M: [kOSlab][R + 1]
    for (int h = 0; h < 2; ++h) {
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
    // A thread takes whole input features i (its Q row stays in registers) and all 16 outputs.
    const T *q = static_cast<const T *>(a.q);
    for (int ii = threadIdx.x; ii < ni; ii += kBwdThreads) {
        const int64_t i = i0 + ii;
        float qr[R];
#pragma unroll
        for (int j = 0; j < R; ++j) qr[j] = j < a.rank ? Act<DT>::ld(q[i * a.rank + j]) : 0.f;
#pragma unroll
        for (int oo = 0; oo < kOSlab; ++oo) {
            const int64_t o = o0 + oo;
            if (o >= a.d_out) break;
            float s = acc[ii * kAccPitch + oo];
#pragma unroll
            for (int j = 0; j < R; ++j) s = fmaf(mfin[oo * (R + 1) + j], qr[j], s);
            store_any(a.dw, a.dw_dt, a.transposed ? i * a.d_out + o : o * a.d_in + i, s);
        }
    }
    if (a.dbias && part == 0)
        for (int oo = threadIdx.x; oo < kOSlab; oo += kBwdThreads)
            if (o0 + oo < a.d_out) store_any(a.dbias, a.db_dt, o0 + oo, mfin[oo * (R + 1) + R]);
}

template <int DT, int R>
constexpr size_t fused_lds_bytes()
{
    using C = GradCfg<DT, R>;
    using L = FusedLds<DT, R>;
    constexpr int HALF = (C::NV + 1) / 2;
    constexpr size_t red = L::s_gtile + ((size_t)kBwdThreads * HALF + (size_t)8 * C::OG * HALF + (size_t)kOSlab * (R + 1)) * 4;
    return L::end > red ? L::end : red;
}

int pad_rank(int rank) { return rank <= 4 ? 4 : rank <= 8 ? 8 : rank <= 16 ? 16 : 32; }

enum { GW_ROWPTR, GW_N };

struct GPlan {
    int R;
    int64_t n_slabs, n_parts, i_span;
};

GPlan make_gplan(const StacrGradArgs &a)
{
    GPlan p{};
    p.R = pad_rank(a.rank);
    p.n_slabs = (a.d_out + kOSlab - 1) / kOSlab;
    p.n_parts = hmax<int64_t>(1, (a.d_in + kMaxISlab - 1) / kMaxISlab);
    p.i_span = (a.d_in + p.n_parts - 1) / p.n_parts;
    return p;
}

size_t glayout(const StacrGradArgs &a, const GPlan &p, size_t *off)
{
    (void)p;
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    take(GW_ROWPTR, a.nnz > 0 ? (size_t)(a.rows + 1) * sizeof(uint32_t) : 0);
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
    hipStream_t s = a.stream;
    FusedArgs f{};
    f.vec_ok = (a.d_out * (int64_t)sizeof(typename Cfg::T)) % Cfg::VB == 0 && (uintptr_t)a.g % Cfg::VB == 0;
    f.g = a.g;
    f.coeff = a.coeff;
    f.q = a.q;
    f.rows = a.rows;
    f.d_out = a.d_out;
    f.d_in = a.d_in;
    f.rank = a.rank;
    f.idx = a.idx;
    f.data = a.data;
    f.scale = a.scale;
    f.bits = a.bits;
    f.val_dt = a.val_dtype;
    f.nnz = a.nnz;
    f.n_slabs = p.n_slabs;
    f.n_parts = p.n_parts;
    f.i_span = p.i_span;
    f.transposed = a.transposed;
    f.dw = a.dw;
    f.dw_dt = a.dw_dtype;
    f.dbias = a.dbias;
    f.db_dt = a.dbias_dtype;
    if (a.nnz > 0) {
        uint32_t *rowptr = reinterpret_cast<uint32_t *>(ws + off[GW_ROWPTR]);
        f.rowptr = rowptr;
        const int cg = (int)((a.nnz + kBlock - 1) / kBlock);
        if (a.index_bytes == 8)
            stacr_launch("k_rowptr", s, [&] { k_rowptr<1><<<cg, kBlock, 0, s>>>(a.idx, a.nnz, a.d_in, a.rows, rowptr); });
        else
            stacr_launch("k_rowptr", s, [&] { k_rowptr<0><<<cg, kBlock, 0, s>>>(a.idx, a.nnz, a.d_in, a.rows, rowptr); });
    }
    constexpr size_t lds = fused_lds_bytes<DT, R>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    const unsigned nwg = (unsigned)(p.n_slabs * p.n_parts);
    if (a.index_bytes == 8) {
        raise_lds_limit(k_dw_fused<DT, R, 1>, lds);
        stacr_launch("k_dw_fused", s, [&] { k_dw_fused<DT, R, 1><<<nwg, kBwdThreads, lds, s>>>(f); });
    } else {
        raise_lds_limit(k_dw_fused<DT, R, 0>, lds);
        stacr_launch("k_dw_fused", s, [&] { k_dw_fused<DT, R, 0><<<nwg, kBwdThreads, lds, s>>>(f); });
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
    const GPlan p = make_gplan(a);
    size_t tmp[GW_N];
    return glayout(a, p, offsets ? offsets : tmp);
}

int stacr_grad_launch(const StacrGradArgs &a)
{
    const GPlan p = make_gplan(a);
    size_t off[GW_N];
    const size_t need = glayout(a, p, off);
    if (a.workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_weight_grad: workspace has %zu bytes, needs %zu",
                          a.workspace_bytes, need);
    char *ws = static_cast<char *>(a.workspace);
    switch (a.dtype) {
    case STACR_DTYPE_F32: return grad_dispatch<STACR_DTYPE_F32>(a, p, ws, off);
    case STACR_DTYPE_BF16: return grad_dispatch<STACR_DTYPE_BF16>(a, p, ws, off);
    default: return grad_dispatch<STACR_DTYPE_F16>(a, p, ws, off);
    }
}
