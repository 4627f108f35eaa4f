// Save path: coefficients, exact residual top-k selection, ordered compaction, quantization.
//
// Restates stacr/layers.py:135-148 (coeff = X.Q, _select_residual, quantize_values) as a chain
// of streaming passes over X:
//   proj_hist     X -> coeff (rounded to the activation dtype), residual r = X - coeff.Q^T in
//                 fp32, per-chunk histogram of the top 11 bits of |r|, global max |r|
//   select_step   per chunk: which histogram bin holds the k-th largest key
//   refine_hist   recompute r; histogram of the next key digit inside the chosen prefix (x2)
//   count/offsets exact 31-bit threshold known: per-workgroup survivor counts -> output offsets
//   emit          recompute r; ordered compaction in ascending flat index; quantize and write
// chunk_topk's trim to k_total (stacr/layers.py:38-40) reruns the radix select over the emitted
// list.  Ties at the threshold go to the lowest flat index.
#include <float.h>

#include <type_traits>

#include "internal.h"

using namespace stacr;

namespace {

constexpr int kHistCopies = 8;     // histogram / max-key copies of a chunk with many workgroups
constexpr int kMaxKeyStride = 32;  // max-key copies 128 bytes apart
constexpr int kCoarse = 64;        // level-0 coarse bins (32 histogram bins each)
constexpr int kEmitStage = 1024;   // survivors a batched emission workgroup stages in LDS
constexpr int kCandCap = 2048;               // candidates a workgroup keeps
constexpr int kCandPer = kCandCap / kBlock;  // candidates a thread reads (consecutive)
static_assert(kCandPer == 8, "one 16-byte vector of bf16 candidate values per thread");

struct CandMeta {
    uint32_t cut;    // level-0 bin of the workgroup's cut
    uint32_t count;  // candidates (more than kCandCap: the list overflowed and is not used)
};

__device__ __forceinline__ void wg_rows(const SaveGeom &g, int64_t wg, int64_t &chunk, int64_t &row0,
                                        int64_t &row_end)
{
    chunk = wg / g.wgs_per_chunk;
    const int64_t local = wg - chunk * g.wgs_per_chunk;
    const int64_t cstart = chunk * g.chunk_rows;
    const int64_t cend = min(cstart + g.chunk_rows, g.rows);
    row0 = cstart + local * g.rows_per_wg;
    row_end = min(row0 + g.rows_per_wg, cend);
}

// Sum R partial values over the L threads of a row slot; every thread of the slot receives the
// identical total (the xor butterfly adds commuted pairs, the cross-wave sum has a fixed order).
template <int R>
__device__ __forceinline__ void row_reduce(float (&acc)[R], int L, float *s_red)
{
    const int w = L < 64 ? L : 64;
    for (int off = w >> 1; off > 0; off >>= 1) {
#pragma unroll
        for (int j = 0; j < R; ++j) acc[j] += __shfl_xor(acc[j], off, 64);
    }
    if (L > 64) {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < R; ++j) s_red[wave * R + j] = acc[j];
        }
        __syncthreads();
        const int per = L >> 6, first = (wave / per) * per;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            float s = 0.f;
            for (int k = 0; k < per; ++k) s += s_red[(first + k) * R + j];
            acc[j] = s;
        }
        __syncthreads();
    }
}

// Basis columns of one vector, either cached in registers or read from the padded fp32 copy.
template <int R, int V, bool QREG>
struct QCols {
    float q[QREG ? V : 1][QREG ? R : 1];
    __device__ __forceinline__ void init(const float *__restrict__ qp, int64_t col, int64_t d)
    {
        if constexpr (QREG) {
            if (col + V <= d) {  // V * R contiguous floats, 16-byte aligned: vector loads, no branches
                const float4 *src = reinterpret_cast<const float4 *>(qp + col * R);
#pragma unroll
                for (int k = 0; k < V * R / 4; ++k) {
                    const float4 v = src[k];
                    q[(4 * k) / R][(4 * k) % R] = v.x;
                    q[(4 * k + 1) / R][(4 * k + 1) % R] = v.y;
                    q[(4 * k + 2) / R][(4 * k + 2) % R] = v.z;
                    q[(4 * k + 3) / R][(4 * k + 3) % R] = v.w;
                }
                return;
            }
#pragma unroll
            for (int e = 0; e < V; ++e)
#pragma unroll
                for (int j = 0; j < R; ++j)
                    q[e][j] = (col + e < d) ? qp[(col + e) * R + j] : 0.f;
        }
    }
    __device__ __forceinline__ float get(const float *__restrict__ qp, int64_t col, int e, int j) const
    {
        if constexpr (QREG) return q[e][j];
        else return qp[(col + e) * R + j];
    }
};

// Residual of one vector in the activation dtype, as both engines form it with dtype-native torch
// ops (stacr/layers.py:32,73 and stacr/adaptive.py:1518-1519): p = sum_j c_j q_j as an fp32
// fused multiply-add chain from 0 (j ascending) rounded to the dtype, then r = x - p rounded to the
// dtype.  For fp32 the roundings are the identity.  The oracle repeats this order.
template <int DT, int R, int V, bool QREG>
__device__ __forceinline__ void residuals(const float (&xv)[V], const float (&c)[R],
                                          const QCols<R, V, QREG> &qc, const float *__restrict__ qp,
                                          int64_t col, float (&r)[V])
{
#pragma unroll
    for (int e = 0; e < V; ++e) {
        float p = 0.f;
#pragma unroll
        for (int j = 0; j < R; ++j) p = fmaf(c[j], qc.get(qp, col, e, j), p);
        r[e] = Act<DT>::rnd(xv[e] - Act<DT>::rnd(p));
    }
}

template <int DT, int R>
__device__ __forceinline__ void load_coeff(const typename Act<DT>::T *__restrict__ coeff, int64_t row,
                                           int rank, bool active, float (&c)[R])
{
#pragma unroll
    for (int j = 0; j < R; ++j)
        c[j] = (active && j < rank) ? Act<DT>::ld(coeff[row * rank + j]) : 0.f;
}

struct OutSpec {
    void *idx;
    int idx_bytes;   // 2, 4 or 8
    void *data;   // int8 (bits 8), int8 staging (bits 4), activation dtype (bits 0)
    int bits;
    uint32_t *list_rbits;  // trim path: chunk survivors as (fp32 bits, flat index)
    uint32_t *list_idx;
    uint32_t cap;          // entries the destination holds; positions at or past it are dropped
};

__device__ __forceinline__ float quant_scale(uint32_t maxkey, int bits, float amax_rounded)
{
    (void)maxkey;
    const float qmax = bits == 4 ? 7.f : 127.f;
    float s = __fdiv_rn(amax_rounded, qmax);
    return s < FLT_MIN ? FLT_MIN : s;  // NaN propagates (comparison is false)
}

__device__ __forceinline__ int8_t quantize_one(float v, float scale, int bits)
{
    const float qmax = bits == 4 ? 7.f : 127.f;
    float t = rintf(__fdiv_rn(v, scale));  // round half to even, as torch.round
    t = fminf(fmaxf(t, -qmax - 1.f), qmax);
    return (int8_t)(int)t;
}

template <int DT>
__device__ __forceinline__ void write_entry(const OutSpec &o, uint32_t pos, uint32_t flat, float r, float scale)
{
    if (o.idx_bytes == 8) static_cast<int64_t *>(o.idx)[pos] = (int64_t)flat;
    else if (o.idx_bytes == 4) static_cast<int32_t *>(o.idx)[pos] = (int32_t)flat;
    else static_cast<int16_t *>(o.idx)[pos] = (int16_t)flat;
    const float v = Act<DT>::rnd(r);
    if (o.bits == 0) static_cast<typename Act<DT>::T *>(o.data)[pos] = Act<DT>::st(v);
    else static_cast<int8_t *>(o.data)[pos] = quantize_one(v, scale, o.bits);
}

// ------------------------------------------------------------------ kernels
__global__ void k_zero_u32(uint32_t *p, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Set-up of a save: the padded fp32 basis (its first `rank` columns of rows q_ld apart), and the
// histograms and max key cleared (one launch).
template <int DT>
__global__ void k_prep(const typename Act<DT>::T *__restrict__ q, int64_t d, int rank, int q_ld, int R,
                       float *__restrict__ qp, uint32_t *__restrict__ zero, int64_t n_zero, uint32_t *__restrict__ zero2,
                       int64_t n_zero2)
{
    const int64_t n = d * R;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    float *qpt = qp + n;  // the same values transposed, [R][d]: the batched passes read it per rank
    // 16-bit types: also the transposed copy in the activation dtype (the projection's dot products)
    typename Act<DT>::T *qph = reinterpret_cast<typename Act<DT>::T *>(qpt + n);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) {
        {   // padded copy: element i is (row i / R, column i % R)
            const int64_t row = i / R;
            const int j = (int)(i - row * R);
            qp[i] = j < rank ? Act<DT>::ld(q[row * q_ld + j]) : 0.f;
        }
        {   // transposed copies: element i is (column i / d, row i % d), so consecutive threads write
            // consecutive addresses
            const int j = (int)(i / d);
            const int64_t row = i - (int64_t)j * d;
            const typename Act<DT>::T raw = j < rank ? q[row * q_ld + j] : (typename Act<DT>::T)0;
            qpt[i] = j < rank ? Act<DT>::ld(raw) : 0.f;
            if constexpr (sizeof(typename Act<DT>::T) == 2) qph[i] = raw;
        }
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_zero; i += step) zero[i] = 0u;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_zero2; i += step) zero2[i] = 0u;
}

// One radix level of one chunk, computed by a whole workgroup: the bin holding the need-th largest
// key among those matching `prefix`.  Every thread calls it and receives the new state.
__device__ SelState block_select(int lvl, const uint32_t *__restrict__ h, uint32_t prefix, uint32_t need,
                                 uint32_t *s_tot, SelState *s_res)
{
    const int per = kDigitBins[lvl] / kBlock;
    const int bits = lvl == 2 ? 9 : 11;
    // thread t looks at the bins of owner 255 - t so that the exclusive scan counts the bins above
    const int owner = kBlock - 1 - threadIdx.x;
    uint32_t local = 0u;
    for (int i = 0; i < per; ++i) local += h[owner * per + i];
    if (threadIdx.x == 0) *s_res = SelState{prefix << bits, need};
    uint32_t total;
    const uint32_t above = block_exclusive_scan(local, s_tot, &total);
    if (above < need && above + local >= need) {
        uint32_t run = above;
        for (int i = per - 1; i >= 0; --i) {
            const int b = owner * per + i;
            if (run + h[b] >= need) {
                *s_res = SelState{(prefix << bits) | (uint32_t)b, need - run};
                break;
            }
            run += h[b];
        }
    }
    __syncthreads();
    const SelState r = *s_res;
    __syncthreads();  // s_res is free again
    return r;
}

// Level lvl's state of a chunk, from its histogram and the previous level's state (level 0: the
// chunk's k).  The first workgroup of the chunk records it for the kernels that follow.
__device__ SelState chunk_select(int lvl, const uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                 int64_t chunk, int64_t n_chunks, uint32_t k_full, uint32_t k_last, bool record,
                                 uint32_t *s_tot, SelState *s_res)
{
    uint32_t need, prefix;
    if (lvl == 0) {
        need = chunk == n_chunks - 1 ? k_last : k_full;
        prefix = 0u;
    } else {
        const SelState sp = state[chunk * 3 + lvl - 1];
        need = sp.need;
        prefix = sp.prefix;
    }
    const SelState r = block_select(lvl, hist + (chunk * 3 + lvl) * kBins, prefix, need, s_tot, s_res);
    if (record && threadIdx.x == 0) state[chunk * 3 + lvl] = r;
    return r;
}

// The same as a kernel, one workgroup per chunk (the trim pass over the candidate list).
__global__ __launch_bounds__(kBlock) void k_select_step(int lvl, const uint32_t *__restrict__ hist,
                                                        SelState *__restrict__ state, int64_t n_chunks,
                                                        uint32_t k_full, uint32_t k_last)
{
    __shared__ uint32_t s_tot[kWaves];
    __shared__ SelState s_res;
    chunk_select(lvl, hist, state, blockIdx.x, n_chunks, k_full, k_last, true, s_tot, &s_res);
}

// A workgroup's output offset and tie budget: its chunk's earlier workgroups in order, ties handed
// out first come (the per-workgroup form of k_offsets).
__device__ WgOffset wg_offset(const WgCount *__restrict__ counts, int64_t chunk, int64_t w, int64_t wgs_per_chunk,
                              uint32_t need_eq, uint32_t chunk_k, uint32_t *s_tot)
{
    uint32_t gt = 0u, eq = 0u;
    for (int64_t v = threadIdx.x; v < w; v += kBlock) {
        const WgCount c = counts[chunk * wgs_per_chunk + v];
        gt += c.gt;
        eq += c.eq;
    }
    const uint32_t gt_before = block_sum(gt, s_tot);
    const uint32_t eq_before = block_sum(eq, s_tot);
    const WgCount mine = counts[chunk * wgs_per_chunk + w];
    const uint32_t take = eq_before >= need_eq ? 0u : min(mine.eq, need_eq - eq_before);
    return WgOffset{(uint32_t)chunk * chunk_k + gt_before + min(need_eq, eq_before), take};
}

// Pass 1: coefficients, first-digit histogram, max key.
template <int DT, int R, int V, bool QREG>
__global__ __launch_bounds__(kBlock) void k_proj_hist(SaveGeom g, const typename Act<DT>::T *__restrict__ x,
                                                      const float *__restrict__ qp,
                                                      typename Act<DT>::T *__restrict__ coeff,
                                                      uint32_t *__restrict__ hist, uint32_t *__restrict__ maxkey,
                                                      int do_hist, const typename Act<DT>::T *__restrict__ coeff_in)
{
    using A = Act<DT>;
    __shared__ uint32_t s_hist[kBins];
    __shared__ float s_red[kWaves * R];
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;

    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    QCols<R, V, QREG> qc;
    qc.init(qp, (int64_t)u * V, g.d);
    uint32_t kmax = 0u;
    __syncthreads();

    for (int64_t base = row0; base < row_end; base += g.rpi) {
        const int64_t row = base + slot;
        const bool active = row < row_end;
        const typename A::T *xr = x + row * g.d;
        float xkeep[V];
        float c[R];
        if (coeff_in) {
            // coefficients supplied by the caller (selection on a given projection)
            load_coeff<DT, R>(coeff_in, row, g.rank, active, c);
        } else {
            float acc[R];
#pragma unroll
            for (int j = 0; j < R; ++j) acc[j] = 0.f;
            for (int m = 0; m < g.mv; ++m) {
                const int64_t col = ((int64_t)m * g.L + u) * V;
                if (active && col < g.d) {
                    float xv[V];
                    load_vec<DT, V>(xr + col, xv);
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        xkeep[e] = xv[e];
#pragma unroll
                        for (int j = 0; j < R; ++j) acc[j] = fmaf(xv[e], qc.get(qp, col, e, j), acc[j]);
                    }
                }
            }
            row_reduce<R>(acc, g.L, s_red);
#pragma unroll
            for (int j = 0; j < R; ++j) c[j] = j < g.rank ? A::rnd(acc[j]) : 0.f;
            if (active && u == 0)
                for (int j = 0; j < g.rank; ++j) coeff[row * g.rank + j] = A::st(c[j]);
        }
        if (!do_hist) continue;
        for (int m = 0; m < g.mv; ++m) {
            const int64_t col = ((int64_t)m * g.L + u) * V;
            if (active && col < g.d) {
                float xv[V], r[V];
                if (QREG && !coeff_in) {
#pragma unroll
                    for (int e = 0; e < V; ++e) xv[e] = xkeep[e];
                } else {
                    load_vec<DT, V>(xr + col, xv);
                }
                residuals<DT, R, V, QREG>(xv, c, qc, qp, col, r);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                    atomicAdd(&s_hist[key >> kDigitShift[0]], 1u);
                    kmax = max(kmax, key);
                }
            }
        }
    }
    if (!do_hist) return;
    __syncthreads();
    uint32_t *gh = hist + (chunk * 3 + 0) * kBins;
    for (int b = threadIdx.x; b < kBins; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    if ((threadIdx.x & 63) == 0 && kmax) atomicMax(maxkey, kmax);
}

// Passes 2 and 3: histogram of digit `lvl` among keys matching the chunk's prefix so far.
template <int DT, int R, int V, bool QREG>
__global__ __launch_bounds__(kBlock) void k_refine_hist(SaveGeom g, int lvl, const typename Act<DT>::T *__restrict__ x,
                                                        const float *__restrict__ qp,
                                                        const typename Act<DT>::T *__restrict__ coeff,
                                                        uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                                        uint32_t k_full, uint32_t k_last)
{
    __shared__ uint32_t s_hist[kBins];
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    __shared__ uint32_t s_tot[kWaves];
    __shared__ SelState s_res;
    const uint32_t prefix = chunk_select(lvl - 1, hist, state, chunk, g.n_chunks, k_full, k_last,
                                         blockIdx.x % g.wgs_per_chunk == 0, s_tot, &s_res).prefix;
    const int match_shift = kDigitShift[lvl - 1], dshift = kDigitShift[lvl];
    const uint32_t dmask = (uint32_t)kDigitBins[lvl] - 1u;
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    QCols<R, V, QREG> qc;
    qc.init(qp, (int64_t)u * V, g.d);
    __syncthreads();
    for (int64_t base = row0; base < row_end; base += g.rpi) {
        const int64_t row = base + slot;
        const bool active = row < row_end;
        float c[R];
        load_coeff<DT, R>(coeff, row, g.rank, active, c);
        for (int m = 0; m < g.mv; ++m) {
            const int64_t col = ((int64_t)m * g.L + u) * V;
            if (active && col < g.d) {
                float xv[V], r[V];
                load_vec<DT, V>(x + row * g.d + col, xv);
                residuals<DT, R, V, QREG>(xv, c, qc, qp, col, r);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                    if ((key >> match_shift) == prefix) atomicAdd(&s_hist[(key >> dshift) & dmask], 1u);
                }
            }
        }
    }
    __syncthreads();
    uint32_t *gh = hist + (chunk * 3 + lvl) * kBins;
    for (int b = threadIdx.x; b < kDigitBins[lvl]; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
}

template <int DT, int R, int V, bool QREG>
__global__ __launch_bounds__(kBlock) void k_count(SaveGeom g, const typename Act<DT>::T *__restrict__ x,
                                                  const float *__restrict__ qp,
                                                  const typename Act<DT>::T *__restrict__ coeff,
                                                  const uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                                  WgCount *__restrict__ counts, uint32_t k_full, uint32_t k_last)
{
    __shared__ uint32_t s_tot[kWaves];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    __shared__ SelState s_res;
    const uint32_t T = chunk_select(2, hist, state, chunk, g.n_chunks, k_full, k_last,
                                    blockIdx.x % g.wgs_per_chunk == 0, s_tot, &s_res).prefix;
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    QCols<R, V, QREG> qc;
    qc.init(qp, (int64_t)u * V, g.d);
    uint32_t gt = 0u, eq = 0u;
    for (int64_t base = row0; base < row_end; base += g.rpi) {
        const int64_t row = base + slot;
        const bool active = row < row_end;
        float c[R];
        load_coeff<DT, R>(coeff, row, g.rank, active, c);
        for (int m = 0; m < g.mv; ++m) {
            const int64_t col = ((int64_t)m * g.L + u) * V;
            if (active && col < g.d) {
                float xv[V], r[V];
                load_vec<DT, V>(x + row * g.d + col, xv);
                residuals<DT, R, V, QREG>(xv, c, qc, qp, col, r);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                    gt += key > T;
                    eq += key == T;
                }
            }
        }
    }
    const uint32_t tg = block_sum(gt, s_tot);
    const uint32_t te = block_sum(eq, s_tot);
    if (threadIdx.x == 0) counts[blockIdx.x] = WgCount{tg, te};
}

// Output offsets: per chunk, scan the workgroups in order; ties are handed out first come.
__global__ __launch_bounds__(kBlock) void k_offsets(const WgCount *__restrict__ counts, WgOffset *__restrict__ offs,
                                                    const SelState *__restrict__ state, int64_t wgs_per_chunk,
                                                    uint32_t chunk_k)
{
    __shared__ uint32_t s_tot[kWaves];
    const int64_t chunk = blockIdx.x;
    const uint32_t need_eq = state[chunk * 3 + 2].need;
    const uint32_t base = (uint32_t)chunk * chunk_k;
    uint32_t carry_eq = 0u, carry_sel = 0u;
    for (int64_t w0 = 0; w0 < wgs_per_chunk; w0 += kBlock) {
        const int64_t w = w0 + threadIdx.x;
        const WgCount c = w < wgs_per_chunk ? counts[chunk * wgs_per_chunk + w] : WgCount{0u, 0u};
        uint32_t tot_eq, tot_sel;
        const uint32_t eq_before = carry_eq + block_exclusive_scan(c.eq, s_tot, &tot_eq);
        const uint32_t take = eq_before >= need_eq ? 0u : min(c.eq, need_eq - eq_before);
        const uint32_t sel = c.gt + take;
        const uint32_t sel_before = carry_sel + block_exclusive_scan(sel, s_tot, &tot_sel);
        if (w < wgs_per_chunk) offs[chunk * wgs_per_chunk + w] = WgOffset{base + sel_before, take};
        carry_eq += tot_eq;
        carry_sel += tot_sel;
    }
}

template <int DT, int R, int V, bool QREG>
__global__ __launch_bounds__(kBlock) void k_emit(SaveGeom g, const typename Act<DT>::T *__restrict__ x,
                                                 const float *__restrict__ qp,
                                                 const typename Act<DT>::T *__restrict__ coeff,
                                                 const SelState *__restrict__ state, const WgCount *__restrict__ counts, uint32_t chunk_k,
                                                 const uint32_t *__restrict__ maxkey, OutSpec o, float *scale_out,
                                                 int to_list)
{
    __shared__ uint32_t s_tot[kWaves];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const uint32_t T = state[chunk * 3 + 2].prefix;
    __shared__ uint32_t s_off[kWaves];
    const WgOffset wo = wg_offset(counts, chunk, blockIdx.x - chunk * g.wgs_per_chunk, g.wgs_per_chunk,
                                  state[chunk * 3 + 2].need, chunk_k, s_off);
    const float amax = Act<DT>::rnd(__uint_as_float(*maxkey));
    const float scale = o.bits ? quant_scale(*maxkey, o.bits, amax) : 1.f;
    if (!to_list && blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    QCols<R, V, QREG> qc;
    qc.init(qp, (int64_t)u * V, g.d);
    uint32_t cur_gt = 0u, cur_eq = 0u;
    for (int64_t base = row0; base < row_end; base += g.rpi) {
        const int64_t row = base + slot;
        const bool active = row < row_end;
        float c[R];
        load_coeff<DT, R>(coeff, row, g.rank, active, c);
        for (int m = 0; m < g.mv; ++m) {
            const int64_t col = ((int64_t)m * g.L + u) * V;
            const bool live = active && col < g.d;
            float r[V];
            uint32_t ngt = 0u, neq = 0u;
            if (live) {
                float xv[V];
                load_vec<DT, V>(x + row * g.d + col, xv);
                residuals<DT, R, V, QREG>(xv, c, qc, qp, col, r);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                    ngt += key > T;
                    neq += key == T;
                }
            }
            uint32_t tot;
            const uint32_t ex = block_exclusive_scan(ngt | (neq << 16), s_tot, &tot);
            if (live && (ngt | neq)) {
                uint32_t gb = cur_gt + (ex & 0xffffu), eb = cur_eq + (ex >> 16);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                    const bool is_gt = key > T, is_eq = key == T;
                    if (is_gt || (is_eq && eb < wo.take)) {
                        const uint32_t pos = wo.off + gb + min(eb, wo.take);
                        const uint32_t flat = (uint32_t)(row * g.d + col + e);
                        if (pos >= o.cap) {
                            // unreachable when the counts are consistent; never write out of bounds
                        } else if (to_list) {
                            o.list_rbits[pos] = __float_as_uint(r[e]);
                            o.list_idx[pos] = flat;
                        } else {
                            write_entry<DT>(o, pos, flat, r[e], scale);
                        }
                    }
                    gb += is_gt;
                    eb += is_eq;
                }
            }
            cur_gt += tot & 0xffffu;
            cur_eq += tot >> 16;
        }
    }
}

// ------------------------------------------------------------------ batched fast path
// Rows of d <= 256 * V features whose vectors are aligned: every thread holds one V-wide vector
// of a row and the basis rows of its V columns in registers; L = 64 * W threads (W waves) share a
// row and 256 / L row slots run side by side.  A batch is NB = 64 / R iterations of the slots, and
// everything a batch needs (NB vectors of X per thread, NB coefficient rows) is loaded before any
// of it is used, so a batch costs one memory round trip and at most two barriers.
template <int R> struct Batch {
    static constexpr int NB = 64 / R;  // iterations per batch: NB * R = 64 values per row slot
};

// Raw V-wide vector of X (one 16-byte load), zero when the row is outside the workgroup's range.
template <int DT, int V>
__device__ __forceinline__ uint4 load_raw(const typename Act<DT>::T *__restrict__ p, bool ok)
{
    static_assert(V * sizeof(typename Act<DT>::T) == 16, "fast path uses 16-byte vectors");
    return ok ? *reinterpret_cast<const uint4 *>(p) : make_uint4(0u, 0u, 0u, 0u);
}

template <int DT, int V>
__device__ __forceinline__ void unpack_raw(const uint4 &w, float (&x)[V])
{
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
    if constexpr (V == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(u[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = Act<DT>::ld((typename Act<DT>::T)((u[e / 2] >> (16 * (e & 1))) & 0xffffu));
    }
}

// V residuals of a 16-bit type (each exactly representable) packed as one 16-byte vector
template <int DT, int V>
__device__ __forceinline__ uint4 pack_raw(const float (&v)[V])
{
    static_assert(V == 8 && sizeof(typename Act<DT>::T) == 2, "16-bit vectors of 8");
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        u[k] = (uint32_t)Act<DT>::st(v[2 * k]) | ((uint32_t)Act<DT>::st(v[2 * k + 1]) << 16);
    return make_uint4(u[0], u[1], u[2], u[3]);
}

// Coefficients of the NB rows of a batch for this thread's slot, as the activation dtype rounds
// them.  Pass 1 computes them (acc holds the thread's partial sums, flattened i * R + j) and
// writes them to `coeff`; the later passes load them.  s_c holds [slot][64] floats.
template <int DT, int R>
__device__ __forceinline__ void batch_coeff_from_acc(float (&acc)[64], int W, int slot, float *s_part, float *s_c,
                                                     int64_t base, int rpi, int64_t row_end, int rank,
                                                     typename Act<DT>::T *__restrict__ coeff, float (&c)[64])
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float part = wave_reduce_scatter64(acc);
    if (W > 1) s_part[wave * 64 + lane] = part;
    __syncthreads();
    const int w0 = slot * W;  // first wave of the slot
    if (wave == w0) {
        float tot = part;
        for (int w = 1; w < W; ++w) tot += s_part[(w0 + w) * 64 + lane];
        const float cv = Act<DT>::rnd(tot);
        s_c[slot * 64 + lane] = cv;
        const int i = lane / R, j = lane % R;
        const int64_t row = base + (int64_t)i * rpi + slot;  // row i of the batch (computed, not indexed)
        if (j < rank && row < row_end) coeff[row * rank + j] = Act<DT>::st(cv);
    }
    __syncthreads();
    const float4 *src = reinterpret_cast<const float4 *>(s_c + slot * 64);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float4 v = src[k];
        c[4 * k] = v.x; c[4 * k + 1] = v.y; c[4 * k + 2] = v.z; c[4 * k + 3] = v.w;
    }
}

template <int DT, int R>
__device__ __forceinline__ void batch_coeff_load(const typename Act<DT>::T *__restrict__ coeff, int rank,
                                                 const int64_t (&rows)[Batch<R>::NB], int64_t row_end, bool vec,
                                                 float (&c)[64])
{
    constexpr int NB = Batch<R>::NB;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool ok = rows[i] < row_end;
        if (vec && sizeof(typename Act<DT>::T) * R % 16 == 0) {  // rank == R, 16-byte aligned rows
            constexpr int NW = (int)(sizeof(typename Act<DT>::T) * R / 16) > 0 ? (int)(sizeof(typename Act<DT>::T) * R / 16) : 1;
            const uint4 *src = reinterpret_cast<const uint4 *>(coeff + rows[i] * R);
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                const uint4 w = ok ? src[k] : make_uint4(0u, 0u, 0u, 0u);
                if constexpr (sizeof(typename Act<DT>::T) == 4) {
                    c[i * R + 4 * k] = __uint_as_float(w.x); c[i * R + 4 * k + 1] = __uint_as_float(w.y);
                    c[i * R + 4 * k + 2] = __uint_as_float(w.z); c[i * R + 4 * k + 3] = __uint_as_float(w.w);
                } else {
                    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        c[i * R + 8 * k + e] = Act<DT>::ld((typename Act<DT>::T)((u[e / 2] >> (16 * (e & 1))) & 0xffffu));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < R; ++j) c[i * R + j] = (ok && j < rank) ? Act<DT>::ld(coeff[rows[i] * rank + j]) : 0.f;
        }
    }
}

// Residual of one vector with the basis in registers (arithmetic as in residuals above).
template <int DT, int R, int V>
__device__ __forceinline__ void batch_residual(const float (&xv)[V], const float *c, const float (&q)[V][R],
                                               float (&r)[V])
{
#pragma unroll
    for (int e = 0; e < V; ++e) {
        float p = 0.f;
#pragma unroll
        for (int j = 0; j < R; ++j) p = fmaf(c[j], q[e][j], p);
        r[e] = Act<DT>::rnd(xv[e] - Act<DT>::rnd(p));
    }
}

struct FastGeom {
    int W;       // waves per row slot
    int c_vec;   // coefficient rows are exactly R wide and 16-byte aligned
};

// The rows of batch `base` for this thread: base + i * rpi + slot.
template <int R>
__device__ __forceinline__ void batch_rows(const SaveGeom &g, int64_t base, int slot, int64_t (&rows)[Batch<R>::NB])
{
#pragma unroll
    for (int i = 0; i < Batch<R>::NB; ++i) rows[i] = base + (int64_t)i * g.rpi + slot;
}

// Fast-path loads are unconditional, from rows and columns clamped into range, and the values
// outside the workgroup's rows or the matrix's columns are zeroed where they are used: a load
// whose value is merged from divergent paths is waited for as soon as it is issued, whereas these
// stay in flight together (histogram words for the selection first, then X, C and the basis) and
// overlap the selection arithmetic.
template <int DT, int R, int V, bool LOADC>
struct FastLoads {
    using T = typename Act<DT>::T;
    static constexpr int NB = Batch<R>::NB;
    static constexpr bool kCVec = LOADC && sizeof(T) * R % 16 == 0;        // whole 16-byte C rows
    static constexpr int NWC = kCVec ? (int)(sizeof(T) * R / 16) : 1;
    int64_t rows[NB];
    uint4 raw[NB];
    uint4 craw[kCVec ? NB : 1][NWC];

    __device__ __forceinline__ void issue(const SaveGeom &g, int slot, int64_t base, int64_t row_end, int64_t colc,
                                          const T *__restrict__ x, const T *__restrict__ coeff, bool cvec)
    {
        // rows clamped to row_end - 1, a row of the matrix even for a trailing workgroup with no rows
        // (row_end is at least 1)
        batch_rows<R>(g, base, slot, rows);
#pragma unroll
        for (int i = 0; i < NB; ++i)
            raw[i] = *reinterpret_cast<const uint4 *>(x + min(rows[i], row_end - 1) * g.d + colc);
        if constexpr (kCVec) {
            // without whole C rows (cvec false) the same loads read the row's start in X instead
            // (valid memory: a batched-path X row is wider than NWC vectors) and are not used
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int64_t row = min(rows[i], row_end - 1);
                const uint4 *src = reinterpret_cast<const uint4 *>(cvec ? coeff + row * R : x + row * g.d);
#pragma unroll
                for (int k = 0; k < NWC; ++k) craw[i][k] = src[k];
            }
        }
    }
    // vector i as floats (zero outside the rows / columns)
    __device__ __forceinline__ void x_at(int i, bool live, float (&xv)[V]) const
    {
        unpack_raw<DT, V>(live ? raw[i] : make_uint4(0u, 0u, 0u, 0u), xv);
    }
    // coefficient row of vector i (the loaded one when cvec, else read now), zero outside the rows
    __device__ __forceinline__ void coeff_row(int i, const T *__restrict__ coeff, int rank, int64_t row_end,
                                              bool cvec, float (&c)[R]) const
    {
        const bool ok = rows[i] < row_end;
        if (kCVec && cvec) {
#pragma unroll
            for (int k = 0; k < NWC; ++k) {
                const uint4 w = ok ? craw[kCVec ? i : 0][k] : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t u[4] = {w.x, w.y, w.z, w.w};
                if constexpr (sizeof(T) == 4) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) c[4 * k + e] = __uint_as_float(u[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) c[8 * k + e] = Act<DT>::ld((T)((u[e / 2] >> (16 * (e & 1))) & 0xffffu));
                }
            }
        } else {
            load_coeff<DT, R>(coeff, rows[i], rank, ok, c);
        }
    }
};

// Basis values of this thread's columns from a clamped column (zeroed where the column is outside
// the matrix, at the first use), read from the transposed copy qpt[j][col]: per rank, the lanes of
// a wave read consecutive 16- or 32-byte pieces of one row, not 256-byte-strided blocks.
template <int R, int V>
__device__ __forceinline__ void basis_issue(const float *__restrict__ qpt, int64_t d, int64_t colc, float (&q)[V][R])
{
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
        for (int h = 0; h < V / 4; ++h) {
            const float4 v = *reinterpret_cast<const float4 *>(qpt + j * d + colc + 4 * h);
            q[4 * h][j] = v.x;
            q[4 * h + 1][j] = v.y;
            q[4 * h + 2][j] = v.z;
            q[4 * h + 3][j] = v.w;
        }
    }
}
template <int R, int V>
__device__ __forceinline__ void basis_mask(bool col_ok, float (&q)[V][R])
{
#pragma unroll
    for (int e = 0; e < V; ++e)
#pragma unroll
        for (int j = 0; j < R; ++j) q[e][j] = col_ok ? q[e][j] : 0.f;
}

// The bins a thread reads for a block_select, loaded ahead.
struct HistPre {
    uint32_t v[kBins / kBlock];
};
// PER: bins per thread, 8 for the 11-bit levels, 2 for the last.  HC: histogram copies (kBins
// apart) summed on the way in.
template <int PER, int HC>
__device__ __forceinline__ void hist_issue(const uint32_t *__restrict__ h, HistPre &p)
{
    const int owner = kBlock - 1 - threadIdx.x;
    if constexpr (PER == 8) {
        uint4 a[HC], b[HC];
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint4 *src = reinterpret_cast<const uint4 *>(h + c * kBins + owner * 8);
            a[c] = src[0];
            b[c] = src[1];
        }
        p.v[0] = a[0].x; p.v[1] = a[0].y; p.v[2] = a[0].z; p.v[3] = a[0].w;
        p.v[4] = b[0].x; p.v[5] = b[0].y; p.v[6] = b[0].z; p.v[7] = b[0].w;
#pragma unroll
        for (int c = 1; c < HC; ++c) {
            p.v[0] += a[c].x; p.v[1] += a[c].y; p.v[2] += a[c].z; p.v[3] += a[c].w;
            p.v[4] += b[c].x; p.v[5] += b[c].y; p.v[6] += b[c].z; p.v[7] += b[c].w;
        }
    } else {
        static_assert(PER == 2, "level bins per thread");
        uint2 a[HC];
#pragma unroll
        for (int c = 0; c < HC; ++c) a[c] = *reinterpret_cast<const uint2 *>(h + c * kBins + owner * 2);
        p.v[0] = a[0].x; p.v[1] = a[0].y;
#pragma unroll
        for (int c = 1; c < HC; ++c) { p.v[0] += a[c].x; p.v[1] += a[c].y; }
#pragma unroll
        for (int i = 2; i < kBins / kBlock; ++i) p.v[i] = 0u;
    }
}
// block_select on the prefetched bins (same result as block_select on the histogram)
__device__ SelState block_select_pre(int lvl, const HistPre &p, uint32_t prefix, uint32_t need, uint32_t *s_tot,
                                     SelState *s_res)
{
    const int per = kDigitBins[lvl] / kBlock;
    const int bits = lvl == 2 ? 9 : 11;
    const int owner = kBlock - 1 - threadIdx.x;
    uint32_t local = 0u;
#pragma unroll
    for (int i = 0; i < kBins / kBlock; ++i) local += i < per ? p.v[i] : 0u;
    if (threadIdx.x == 0) *s_res = SelState{prefix << bits, need};
    uint32_t total;
    const uint32_t above = block_exclusive_scan(local, s_tot, &total);
    if (above < need && above + local >= need) {
        uint32_t run = above;
        bool found = false;
#pragma unroll
        for (int i = kBins / kBlock - 1; i >= 0; --i) {
            if (i < per && !found) {
                if (run + p.v[i] >= need) {
                    *s_res = SelState{(prefix << bits) | (uint32_t)(owner * per + i), need - run};
                    found = true;
                } else {
                    run += p.v[i];
                }
            }
        }
    }
    __syncthreads();
    const SelState r = *s_res;
    __syncthreads();  // s_res is free again
    return r;
}

// Pass 1 (batched): coefficients, first-digit histogram, max key; SR: the residual is also
// stored (16-bit types, where it is exact in the activation dtype) for the later passes to read.
template <int DT, int R, int V, bool SR>
__global__ __launch_bounds__(kBlock) void k_proj_hist_b(SaveGeom g, FastGeom fg, const typename Act<DT>::T *__restrict__ x,
                                                        const float *__restrict__ qp, typename Act<DT>::T *__restrict__ coeff,
                                                        uint32_t *__restrict__ hist, uint32_t *__restrict__ maxkey,
                                                        int do_hist, const typename Act<DT>::T *__restrict__ coeff_in,
                                                        typename Act<DT>::T *__restrict__ rout, uint32_t *__restrict__ coarse)
{
    constexpr int NB = Batch<R>::NB;
    __shared__ uint32_t s_hist[kBins];
    __shared__ __align__(16) float s_part[kWaves * 64];
    __shared__ __align__(16) float s_c[kWaves * 64];
    __shared__ uint32_t s_wmax[kWaves];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    if (row0 >= row_end) return;  // a trailing workgroup with no rows (uniform)
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int64_t col = (int64_t)u * V, colc = min(col, g.d - V);
    const bool col_ok = col < g.d;
    FastLoads<DT, R, V, false> ld;
    ld.issue(g, slot, row0, row_end, colc, x, nullptr, false);
    // 16-bit types read the basis as 16-bit words: the projection takes them as v_dot2 operands
    // (two products a step, fp32 sums) and the residual widens the same values to fp32
    constexpr bool kPair = sizeof(typename Act<DT>::T) == 2 && V == 8;
    float q[V][R];
    uint4 qw[kPair ? R : 1];
    if constexpr (kPair) {
        const typename Act<DT>::T *qph = reinterpret_cast<const typename Act<DT>::T *>(qp + 2 * g.d * R);
#pragma unroll
        for (int j = 0; j < R; ++j) qw[j] = *reinterpret_cast<const uint4 *>(qph + j * g.d + colc);
    } else {
        basis_issue<R, V>(qp + g.d * R, g.d, colc, q);
    }
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    uint32_t kmax = 0u;
    __syncthreads();
    if constexpr (kPair) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const uint32_t w[4] = {qw[j].x, qw[j].y, qw[j].z, qw[j].w};
#pragma unroll
            for (int e = 0; e < V; ++e) q[e][j] = Act<DT>::ld((typename Act<DT>::T)((w[e / 2] >> (16 * (e & 1))) & 0xffffu));
        }
    }
    basis_mask<R, V>(col_ok, q);
    {   // the workgroup's rows are one batch (the plan sizes them so)
        float c[64];
        if (coeff_in) {
            batch_coeff_load<DT, R>(coeff_in, g.rank, ld.rows, row_end, fg.c_vec != 0, c);
        } else {
            float acc[64];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const bool live = col_ok && ld.rows[i] < row_end;
                if constexpr (kPair) {
                    const uint4 xr = live ? ld.raw[i] : make_uint4(0u, 0u, 0u, 0u);
                    const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
                    for (int j = 0; j < R; ++j) {
                        const uint32_t w[4] = {qw[j].x, qw[j].y, qw[j].z, qw[j].w};
                        float s = 0.f;
#pragma unroll
                        for (int k = 0; k < 4; ++k) s = dot2<DT>(xw[k], w[k], s);
                        acc[i * R + j] = s;
                    }
                } else {
                    float xv[V];
                    ld.x_at(i, live, xv);
#pragma unroll
                    for (int j = 0; j < R; ++j) {
                        float s = 0.f;
#pragma unroll
                        for (int e = 0; e < V; ++e) s = fmaf(xv[e], q[e][j], s);
                        acc[i * R + j] = s;
                    }
                }
            }
            batch_coeff_from_acc<DT, R>(acc, fg.W, slot, s_part, s_c, row0, g.rpi, row_end, g.rank, coeff, c);
        }
        if (!do_hist) return;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (!(col_ok && ld.rows[i] < row_end)) continue;
            float xv[V], r[V];
            ld.x_at(i, true, xv);
            batch_residual<DT, R, V>(xv, c + i * R, q, r);
            if constexpr (SR) *reinterpret_cast<uint4 *>(rout + ld.rows[i] * g.d + col) = pack_raw<DT, V>(r);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                atomicAdd(&s_hist[key >> kDigitShift[0]], 1u);
                kmax = max(kmax, key);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    if ((threadIdx.x & 63) == 0) s_wmax[threadIdx.x >> 6] = kmax;
    __syncthreads();
    // this workgroup's copy of the chunk histogram and of the max key (one atomic per workgroup)
    const int copy = (int)(blockIdx.x % g.hcopies);
    uint32_t *gh = hist + ((chunk * 3 + 0) * g.hcopies + copy) * kBins;
    for (int b = threadIdx.x; b < kBins; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
    if (threadIdx.x < kCoarse) {  // the same counts in 64 bins of 32
        uint32_t sum = 0u;
#pragma unroll 8
        for (int b = 0; b < kBins / kCoarse; ++b) sum += s_hist[threadIdx.x * (kBins / kCoarse) + b];
        if (sum) atomicAdd(&coarse[(chunk * g.hcopies + copy) * kCoarse + threadIdx.x], sum);
    }
    if (threadIdx.x == 0) {
        uint32_t m = 0u;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) m = max(m, s_wmax[w]);
        if (m) atomicMax(maxkey + copy * kMaxKeyStride, m);
    }
}

// Pass 1 for 16-bit rows the batched kernels do not take (2048 < d <= 8192, or rank 16): the
// workgroup's NT threads share each row, thread u holding the MV vectors at columns
// (m * NT + u) * 8, and the basis stays as packed 16-bit words (the projection's v_dot2 operands;
// the residual widens one vector's worth at a time).  The workgroup's rows are one batch of
// 64 / R rows.  Outputs as k_proj_hist_b with the residual stored: coefficients, the residual
// (exact in the activation dtype), the level-0 histogram with its coarse sums, and the max key.
// The later passes read the stored residual as a matrix of f * rows rows of d / f columns (the
// same memory, the same flat indices), so they never need the basis or C.
//
// Optional outputs (NULL: none): y_out, the fp32 projections before rounding of the basis's first
// y_cols columns (the basis copy may hold more columns than the rank, g.rank: those are projected
// for y_out only and take no part in the coefficients or the residual); epart, the workgroup's
// energy partial [kEnergyStride]: sum of rnd(x^2) over its elements, sum of rnd(c^2) and, per basis
// column j < g.rank, the sum of c_j^2 over its rows (C as saved; bf16 only).
template <int DT, int R, int MV, int NT>
__global__ __launch_bounds__(NT) void k_proj_hist_w(SaveGeom g, int c_vec, const typename Act<DT>::T *__restrict__ x,
                                                    const float *__restrict__ qp, typename Act<DT>::T *__restrict__ coeff,
                                                    uint32_t *__restrict__ hist, uint32_t *__restrict__ maxkey,
                                                    int do_hist, const typename Act<DT>::T *__restrict__ coeff_in,
                                                    typename Act<DT>::T *__restrict__ rout, uint32_t *__restrict__ coarse,
                                                    float *__restrict__ y_out, int y_cols, float *__restrict__ epart)
{
    using T = typename Act<DT>::T;
    static_assert(sizeof(T) == 2, "16-bit activations");
    constexpr int V = 8, NB = Batch<R>::NB, W = NT / 64;
    static_assert(NB * R == 64 && NT % 64 == 0 && kBins % NT == 0, "batch and block shape");
    __shared__ uint32_t s_hist[kBins];
    __shared__ __align__(16) float s_part[W * 64];
    __shared__ __align__(16) float s_c[64];
    __shared__ uint32_t s_wmax[W];
    __shared__ float s_ex[W];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    if (row0 >= row_end) {  // a trailing workgroup with no rows (uniform): its energy partial is zero
        if (epart && threadIdx.x < kEnergyStride) epart[(int64_t)blockIdx.x * kEnergyStride + threadIdx.x] = 0.f;
        return;
    }
    const int u = threadIdx.x, lane = u & 63, wave = u >> 6;
    int64_t col[MV], colc[MV];
    bool col_ok[MV];
#pragma unroll
    for (int m = 0; m < MV; ++m) {
        col[m] = (int64_t)(m * NT + u) * V;
        colc[m] = min(col[m], g.d - V);
        col_ok[m] = col[m] < g.d;
    }
    // every load issued before any is used: X rows clamped into the workgroup's range, columns
    // clamped into the row (values outside are zeroed where used)
    int64_t rows[NB];
    uint4 raw[NB][MV];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        rows[i] = row0 + i;
        const T *src = x + min(rows[i], row_end - 1) * g.d;
#pragma unroll
        for (int m = 0; m < MV; ++m) raw[i][m] = *reinterpret_cast<const uint4 *>(src + colc[m]);
    }
    const T *qph = reinterpret_cast<const T *>(qp + 2 * g.d * R);  // [R][d] in the activation dtype
    uint4 qw[MV][R];
#pragma unroll
    for (int m = 0; m < MV; ++m)
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const uint4 w = *reinterpret_cast<const uint4 *>(qph + j * g.d + colc[m]);
            qw[m][j] = col_ok[m] ? w : make_uint4(0u, 0u, 0u, 0u);
        }
    for (int b = u; b < kBins; b += NT) s_hist[b] = 0u;
    uint32_t kmax = 0u;
    float c[64];
    if (coeff_in) {
        batch_coeff_load<DT, R>(coeff_in, g.rank, rows, row_end, c_vec != 0, c);
    } else {
        float acc[64];
#pragma unroll
        for (int k = 0; k < 64; ++k) acc[k] = 0.f;
#pragma unroll
        for (int m = 0; m < MV; ++m) {  // vector by vector: vector m's basis words die after it
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const uint4 xr = rows[i] < row_end && col_ok[m] ? raw[i][m] : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
                for (int j = 0; j < R; ++j) {
                    const uint32_t w[4] = {qw[m][j].x, qw[m][j].y, qw[m][j].z, qw[m][j].w};
                    float sum = acc[i * R + j];
#pragma unroll
                    for (int k = 0; k < 4; ++k) sum = dot2<DT>(xw[k], w[k], sum);
                    acc[i * R + j] = sum;
                }
            }
        }
        // lane l of every wave: the wave's total of value l = (row l / R, basis column l % R); the
        // first wave adds the other waves' totals in wave order and rounds once
        const float part = wave_reduce_scatter64(acc);
        s_part[wave * 64 + lane] = part;
        __syncthreads();
        if (wave == 0) {
            float tot = part;
            for (int w = 1; w < W; ++w) tot += s_part[w * 64 + lane];
            const int i = lane / R, j = lane % R;
            const int64_t row = row0 + i;
            if (y_out && j < y_cols && row < row_end) y_out[row * y_cols + j] = tot;
            const float cv = j < g.rank ? Act<DT>::rnd(tot) : 0.f;  // (columns past the rank: Y only)
            s_c[lane] = cv;
            if (j < g.rank && row < row_end) coeff[row * g.rank + j] = Act<DT>::st(cv);
        }
        __syncthreads();
        const float4 *src = reinterpret_cast<const float4 *>(s_c);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float4 v = src[k];
            c[4 * k] = v.x; c[4 * k + 1] = v.y; c[4 * k + 2] = v.z; c[4 * k + 3] = v.w;
        }
    }
    if constexpr (DT == STACR_DTYPE_BF16) {  // (fp16: the energies take a pass of their own)
    if (epart) {
        // energies: sum of rnd(x^2) over this thread's elements, then over the workgroup in wave order
        float ex = 0.f;
#pragma unroll
        for (int m = 0; m < MV; ++m)
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const uint4 xr = rows[i] < row_end && col_ok[m] ? raw[i][m] : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const float xe = Act<DT>::ld((T)((xw[e >> 1] >> (16 * (e & 1))) & 0xffffu));
                    ex += Act<DT>::rnd(xe * xe);
                }
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ex += __shfl_xor(ex, off, 64);
        if (lane == 0) s_ex[wave] = ex;
        // C as saved: lane (i, j) of wave 0
        if (wave == 0) {
            const int i = lane / R, j = lane % R;
            const int64_t row = row0 + i;
            float cv = 0.f;
            if (j < g.rank && row < row_end) cv = coeff_in ? Act<DT>::ld(coeff_in[row * g.rank + j]) : s_c[lane];
            float sc = Act<DT>::rnd(cv * cv), cj = cv * cv;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sc += __shfl_xor(sc, off, 64);
#pragma unroll
            for (int off = 32; off >= R; off >>= 1) cj += __shfl_xor(cj, off, 64);  // over the rows i
            float *ep = epart + (int64_t)blockIdx.x * kEnergyStride;
            if (lane < g.rank) ep[2 + lane] = cj;
            if (lane == 0) ep[1] = sc;
        }
        __syncthreads();
        if (u == 0) {
            float t = s_ex[0];
            for (int w = 1; w < W; ++w) t += s_ex[w];
            epart[(int64_t)blockIdx.x * kEnergyStride] = t;
        }
    }
    }
    if (!do_hist) return;
    if (coeff_in) __syncthreads();  // the histogram is clear
    // Residual r = rnd(x - rnd(sum_j c_j q_j)) (an fp32 fused-multiply-add chain over j, as in
    // batch_residual), element by element across the batch's rows, packed in the activation
    // dtype as it is formed.  The basis words of vectors m >= 1 are read again here (from L2: the
    // basis is shared by every workgroup) rather than kept from the projection, which leaves room
    // for the batch's coefficients in registers.
#pragma unroll
    for (int m = 0; m < MV; ++m) {
        uint4 qm[R];
        if (m == 0) {
#pragma unroll
            for (int j = 0; j < R; ++j) qm[j] = qw[0][j];
        } else {
            int64_t o = colc[m];
            asm volatile("" : "+v"(o));  // a fresh load, not the projection's registers
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const uint4 w = *reinterpret_cast<const uint4 *>(qph + j * g.d + o);
                qm[j] = col_ok[m] ? w : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        uint32_t rp[NB][4];
#pragma unroll
        for (int i = 0; i < NB; ++i) rp[i][0] = rp[i][1] = rp[i][2] = rp[i][3] = 0u;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            float qe[R];
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const uint32_t w = e < 2 ? qm[j].x : e < 4 ? qm[j].y : e < 6 ? qm[j].z : qm[j].w;
                qe[j] = Act<DT>::ld((T)((w >> (16 * (e & 1))) & 0xffffu));
            }
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const uint4 xr = raw[i][m];
                const uint32_t xw = e < 2 ? xr.x : e < 4 ? xr.y : e < 6 ? xr.z : xr.w;
                const float xe = Act<DT>::ld((T)((xw >> (16 * (e & 1))) & 0xffffu));
                float pj = 0.f;
#pragma unroll
                for (int j = 0; j < R; ++j) pj = fmaf(c[i * R + j], qe[j], pj);
                rp[i][e >> 1] |= (uint32_t)Act<DT>::st(xe - Act<DT>::rnd(pj)) << (16 * (e & 1));
            }
        }
        if (!col_ok[m]) continue;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (rows[i] >= row_end) continue;
            *reinterpret_cast<uint4 *>(rout + rows[i] * g.d + col[m]) = make_uint4(rp[i][0], rp[i][1], rp[i][2], rp[i][3]);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const float rv = Act<DT>::ld((T)((rp[i][e >> 1] >> (16 * (e & 1))) & 0xffffu));
                const uint32_t key = __float_as_uint(rv) & 0x7fffffffu;
                atomicAdd(&s_hist[key >> kDigitShift[0]], 1u);
                kmax = max(kmax, key);
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    if (lane == 0) s_wmax[wave] = kmax;
    __syncthreads();
    const int copy = (int)(blockIdx.x % g.hcopies);
    uint32_t *gh = hist + ((chunk * 3 + 0) * g.hcopies + copy) * kBins;
    for (int b = u; b < kBins; b += NT)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
    if (u < kCoarse) {
        uint32_t sum = 0u;
#pragma unroll 8
        for (int b = 0; b < kBins / kCoarse; ++b) sum += s_hist[u * (kBins / kCoarse) + b];
        if (sum) atomicAdd(&coarse[(chunk * g.hcopies + copy) * kCoarse + u], sum);
    }
    if (u == 0) {
        uint32_t mx = 0u;
#pragma unroll
        for (int w = 0; w < W; ++w) mx = max(mx, s_wmax[w]);
        if (mx) atomicMax(maxkey + copy * kMaxKeyStride, mx);
    }
}

// The level-0 selection from the coarse histogram (64 bins of 32) and then the chosen coarse bin's
// 32 histogram bins, each summed over the HC copies, made by every wave on its own with suffix
// sums across lanes and a ballot (no barrier): the same bin and need as block_select at level 0.
// cv: this lane's coarse bin (lane) in each copy, loaded ahead by the caller.
template <int HC>
__device__ __forceinline__ SelState select_level0(const uint32_t (&cv)[HC], const uint32_t *__restrict__ fine, SelState s0)
{
    constexpr int FB = kBins / kCoarse;
    const int lane = threadIdx.x & 63;
    uint32_t suf = 0u;
#pragma unroll
    for (int h = 0; h < HC; ++h) suf += cv[h];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_down(suf, off, 64);
        if (lane + off < 64) suf += y;
    }
    const uint64_t m = __ballot(suf >= s0.need);
    if (m == 0ull) return SelState{0u, s0.need};  // fewer keys than the need (block_select's default)
    const int cb = 63 - __clzll(m);
    const uint32_t need1 = s0.need - (cb < 63 ? (uint32_t)__shfl((int)suf, cb + 1, 64) : 0u);
    const int fl = lane & (FB - 1);
    uint32_t sf = 0u;
#pragma unroll
    for (int h = 0; h < HC; ++h) sf += fine[h * kBins + cb * FB + fl];
#pragma unroll
    for (int off = 1; off < FB; off <<= 1) {
        const uint32_t y = __shfl_down(sf, off, FB);
        if (fl + off < FB) sf += y;
    }
    const uint64_t mf = __ballot(sf >= need1) & ((1ull << FB) - 1);
    const int fb = mf ? 63 - __clzll(mf) : 0;
    const uint32_t above = fb < FB - 1 ? (uint32_t)__shfl((int)sf, fb + 1, 64) : 0u;
    return SelState{(uint32_t)(cb * FB + fb), need1 - above};
}

// The previous level's state of the workgroup's chunk (level 0: its k).
__device__ __forceinline__ SelState prev_state(int lvl, const SelState *__restrict__ state, int64_t chunk,
                                               int64_t n_chunks, uint32_t k_full, uint32_t k_last)
{
    if (lvl == 0) return SelState{0u, chunk == n_chunks - 1 ? k_last : k_full};
    return state[chunk * 3 + lvl - 1];
}

// Passes 2 and 3 (batched): histogram of digit `lvl` among keys matching the prefix so far.
// CAND (bf16, stored residual, level 1): the pass also writes the workgroup's elements in bin B0
// and above, in ascending flat order, as its candidate list for k_emit_cand (cut = B0).
template <int DT, int R, int V, int HC, bool RIN, int LVL, bool CAND = false>
__global__ __launch_bounds__(kBlock) void k_refine_hist_b(SaveGeom g, FastGeom fg,
                                                          const typename Act<DT>::T *__restrict__ x,
                                                          const float *__restrict__ qp,
                                                          const typename Act<DT>::T *__restrict__ coeff,
                                                          uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                                          uint32_t k_full, uint32_t k_last, uint32_t *__restrict__ maxkey,
                                                          uint32_t *__restrict__ fold, int64_t fold_stride,
                                                          const uint32_t *__restrict__ coarse,
                                                          uint32_t *__restrict__ cand_idx = nullptr,
                                                          uint16_t *__restrict__ cand_val = nullptr,
                                                          CandMeta *__restrict__ meta = nullptr)
{
    static_assert(!CAND || (DT == STACR_DTYPE_BF16 && RIN && LVL == 1), "lists from the stored bf16 residual");
    constexpr int NB = Batch<R>::NB;
    constexpr bool kFold = DT == STACR_DTYPE_BF16;  // per-workgroup records for the emission pass
    constexpr int lvl = LVL;                         // the key digit histogrammed here (1 or 2)
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_tot[kWaves];
    __shared__ uint32_t s_above[kWaves];
    __shared__ SelState s_res;
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const bool has_rows = row0 < row_end;
    const SelState sp = prev_state(lvl - 1, state, chunk, g.n_chunks, k_full, k_last);
    HistPre hp;
    static_assert(kDigitBins[0] / kBlock == 8 && kDigitBins[1] / kBlock == 8 && kDigitBins[2] / kBlock == 2, "bins per thread");
    // level 1 selects level 0 from the coarse histogram (below); level 2 scans the histogram.  The
    // words go out before X.
    uint32_t cv[HC];
    if constexpr (LVL == 1) {
#pragma unroll
        for (int h = 0; h < HC; ++h) cv[h] = coarse[(chunk * HC + h) * kCoarse + (threadIdx.x & 63)];
    } else {
        hist_issue<8, HC>(hist + (chunk * 3 + lvl - 1) * HC * kBins, hp);
    }
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int64_t col = (int64_t)u * V, colc = min(col, g.d - V);
    const bool col_ok = col < g.d;
    FastLoads<DT, R, V, !RIN> ld;  // RIN: x is the stored residual
    // issued whether or not the workgroup has rows: a load under a branch makes every later wait
    // count as if it had not been issued, so waiting for the histogram words would wait for X too
    ld.issue(g, slot, row0, row_end, colc, x, coeff, fg.c_vec != 0);
    float q[V][R];
    if constexpr (!RIN) basis_issue<R, V>(qp + g.d * R, g.d, colc, q);
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    // the chunk's first workgroup records the selection for the passes that follow
    SelState sel;
    if constexpr (LVL == 1) sel = select_level0<HC>(cv, hist + chunk * 3 * HC * kBins, sp);
    else sel = block_select_pre(lvl - 1, hp, sp.prefix, sp.need, s_tot, &s_res);
    if (blockIdx.x % g.wgs_per_chunk == 0 && threadIdx.x == 0) state[chunk * 3 + lvl - 1] = sel;
    if (HC > 1 && lvl == 1 && blockIdx.x == 0 && threadIdx.x == 0) {  // fold the max key's copies into the first
        uint32_t m = maxkey[0];
#pragma unroll
        for (int c = 1; c < HC; ++c) m = max(m, maxkey[c * kMaxKeyStride]);
        maxkey[0] = m;
    }
    const bool fold_rec = kFold && lvl == 1;
    if (!has_rows) {
        if (fold_rec && threadIdx.x <= 16) fold[threadIdx.x * fold_stride + blockIdx.x] = 0u;
        return;
    }
    const uint32_t prefix = sel.prefix;
    const int match_shift = kDigitShift[lvl - 1], dshift = kDigitShift[lvl];
    const uint32_t dmask = (uint32_t)kDigitBins[lvl] - 1u;
    if constexpr (!RIN) basis_mask<R, V>(col_ok, q);
    uint32_t above = 0u;
    uint32_t cmsk[CAND ? NB : 1];  // CAND: elements of vector i in bin B0 and above
    {   // the workgroup's rows are one batch
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if constexpr (CAND) cmsk[i] = 0u;
            if (!(col_ok && ld.rows[i] < row_end)) continue;
            float r[V];
            if constexpr (RIN) {
                ld.x_at(i, true, r);  // the stored residual
            } else {
                float xv[V], ci[R];
                ld.x_at(i, true, xv);
                ld.coeff_row(i, coeff, g.rank, row_end, fg.c_vec != 0, ci);
                batch_residual<DT, R, V>(xv, ci, q, r);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                if ((key >> match_shift) == prefix) atomicAdd(&s_hist[(key >> dshift) & dmask], 1u);
                if (kFold) above += (key >> match_shift) > prefix;
                if constexpr (CAND) cmsk[i] |= (key >> match_shift) >= prefix ? 1u << e : 0u;
            }
        }
    }
    if constexpr (CAND) {
        // the list: (iteration, wave, lane, element) order is ascending flat order
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        uint32_t incl[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) incl[i] = wave_inclusive_scan((uint32_t)__popc(cmsk[i]));
        __shared__ uint32_t s_cwt[kWaves * NB];
        if (lane == 63)
#pragma unroll
            for (int i = 0; i < NB; ++i) s_cwt[wave * NB + i] = incl[i];
        __syncthreads();
        uint32_t before_iter = 0u;
        uint32_t *ci = cand_idx + (int64_t)blockIdx.x * kCandCap;
        uint16_t *cv = cand_val + (int64_t)blockIdx.x * kCandCap;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            uint32_t waves_before = 0u, iter_total = 0u;
#pragma unroll
            for (int wv = 0; wv < kWaves; ++wv) {
                const uint32_t t = s_cwt[wv * NB + i];
                waves_before += wv < wave ? t : 0u;
                iter_total += t;
            }
            uint32_t pos = before_iter + waves_before + incl[i] - (uint32_t)__popc(cmsk[i]);
            if (cmsk[i]) {
                const uint4 raw = ld.raw[i];
                const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
                for (uint32_t m = cmsk[i]; m != 0u; m &= m - 1u, ++pos) {
                    const int e = __builtin_ctz(m);
                    uint32_t word = wd[0];
#pragma unroll
                    for (int k = 1; k < 4; ++k) word = (e >> 1) == k ? wd[k] : word;
                    if (pos < (uint32_t)kCandCap) {
                        ci[pos] = (uint32_t)(ld.rows[i] * g.d + col + e);
                        cv[pos] = (uint16_t)((word >> (16 * (e & 1))) & 0xffffu);
                    }
                }
            }
            before_iter += iter_total;
        }
        if (threadIdx.x == 0) meta[blockIdx.x] = CandMeta{prefix, before_iter};
    }
    if (kFold) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) above += (uint32_t)__shfl_xor((int)above, off, 64);
        if ((threadIdx.x & 63) == 0) s_above[threadIdx.x >> 6] = above;
    }
    __syncthreads();
    if (fold_rec && threadIdx.x <= 16) {  // cum[b] for b = threadIdx.x (16: above B0 only)
        uint32_t c = 0u;
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) c += s_above[wv];
        for (int b = threadIdx.x; b < 16; ++b) c += s_hist[b << 7];
        fold[threadIdx.x * fold_stride + blockIdx.x] = c;
    }
    uint32_t *gh = hist + ((chunk * 3 + lvl) * HC + blockIdx.x % HC) * kBins;
    for (int b = threadIdx.x; b < kDigitBins[lvl]; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
}

// Survivor counts (batched).
template <int DT, int R, int V, int HC, bool RIN>
__global__ __launch_bounds__(kBlock) void k_count_b(SaveGeom g, FastGeom fg, const typename Act<DT>::T *__restrict__ x,
                                                    const float *__restrict__ qp,
                                                    const typename Act<DT>::T *__restrict__ coeff,
                                                    const uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                                  WgCount *__restrict__ counts, uint32_t k_full, uint32_t k_last)
{
    constexpr int NB = Batch<R>::NB;
    // A 16-bit residual widened to fp32 has key bits 8..0 clear, so the last radix level always
    // picks bin 0 with the need unchanged: for those types this pass makes the level-1 selection
    // and derives the final state from it (the second refine pass is not launched).
    constexpr int kLvl = sizeof(typename Act<DT>::T) == 2 ? 1 : 2;
    __shared__ uint32_t s_tot[kWaves];
    __shared__ SelState s_res;
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const bool has_rows = row0 < row_end;
    const SelState sp = prev_state(kLvl, state, chunk, g.n_chunks, k_full, k_last);
    HistPre hp;
    if constexpr (kLvl == 1) hist_issue<8, HC>(hist + (chunk * 3 + 1) * HC * kBins, hp);
    else hist_issue<2, HC>(hist + (chunk * 3 + 2) * HC * kBins, hp);
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int64_t col = (int64_t)u * V, colc = min(col, g.d - V);
    const bool col_ok = col < g.d;
    FastLoads<DT, R, V, !RIN> ld;  // RIN: x is the stored residual
    // issued whether or not the workgroup has rows: a load under a branch makes every later wait
    // count as if it had not been issued, so waiting for the histogram words would wait for X too
    ld.issue(g, slot, row0, row_end, colc, x, coeff, fg.c_vec != 0);
    float q[V][R];
    if constexpr (!RIN) basis_issue<R, V>(qp + g.d * R, g.d, colc, q);
    SelState sel = block_select_pre(kLvl, hp, sp.prefix, sp.need, s_tot, &s_res);
    if (kLvl == 1) {
        if (blockIdx.x % g.wgs_per_chunk == 0 && threadIdx.x == 0) state[chunk * 3 + 1] = sel;
        sel = SelState{sel.prefix << kDigitShift[1], sel.need};
    }
    if (blockIdx.x % g.wgs_per_chunk == 0 && threadIdx.x == 0) state[chunk * 3 + 2] = sel;
    const uint32_t T = sel.prefix;
    if constexpr (!RIN) basis_mask<R, V>(col_ok, q);
    uint32_t gt = 0u, eq = 0u;
    if (has_rows) {  // the workgroup's rows are one batch; a workgroup with none only reports zeros
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (!(col_ok && ld.rows[i] < row_end)) continue;
            float r[V];
            if constexpr (RIN) {
                ld.x_at(i, true, r);  // the stored residual
            } else {
                float xv[V], ci[R];
                ld.x_at(i, true, xv);
                ld.coeff_row(i, coeff, g.rank, row_end, fg.c_vec != 0, ci);
                batch_residual<DT, R, V>(xv, ci, q, r);
            }
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                gt += key > T;
                eq += key == T;
            }
        }
    }
    const uint32_t tg = block_sum(gt, s_tot);
    const uint32_t te = block_sum(eq, s_tot);
    if (threadIdx.x == 0) counts[blockIdx.x] = WgCount{tg, te};
}

// bf16 fold.  A bf16 residual widened to fp32 has key bits 15..0 clear, so inside the level-0 bin
// B0 only bits 19..16 vary: the level-1 histogram has 16 live bins (b << 7).  The refine pass
// records, per workgroup w, cum[b][w] = (its keys above B0) + (its keys in B0 with bits 19..16
// >= b) for b = 0..16 (cum[16]: above B0 only).  Once the level-1 bin b1 is chosen, the threshold
// is T = B0 << 20 | b1 << 16, and a workgroup has cum[b1 + 1] keys above T and cum[b1] -
// cum[b1 + 1] equal to it, so the emission pass needs no separate count pass.
//
// The level-1 selection from the 16 live bins (hw: this lane's bin (lane & 15) in each histogram
// copy), made by every wave on its own: suffix sums across 16 lanes, then the highest bin whose
// suffix reaches the need.  Returns the final (31-bit) state; the same result as the generic
// level-1 and level-2 selections.
template <int HC>
__device__ __forceinline__ SelState fold_select(const uint32_t (&hw)[HC], SelState s0, SelState *sel1)
{
    const int b = threadIdx.x & 15;
    uint32_t suf = 0u;
#pragma unroll
    for (int c = 0; c < HC; ++c) suf += hw[c];
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        const uint32_t y = __shfl_down(suf, off, 16);
        if (b + off < 16) suf += y;
    }
    const uint64_t m = __ballot(suf >= s0.need) & 0xffffull;  // lanes 0..15 hold bins 0..15
    const int b1 = m ? 63 - __clzll(m) : 0;                   // m != 0: B0 holds at least need keys
    const uint32_t above = b1 < 15 ? (uint32_t)__shfl((int)suf, b1 + 1, 64) : 0u;
    *sel1 = SelState{(s0.prefix << 11) | ((uint32_t)b1 << 7), s0.need - above};
    return SelState{sel1->prefix << kDigitShift[1], sel1->need};
}

// Ordered compaction (batched).  Elements are enumerated as (iteration, slot, thread, element),
// which is ascending flat index: one multi-value block scan per batch gives every thread the
// number of survivors (gt in the low half, ties in the high half) before each of its vectors.
// Loads go out in the order they are waited for (the selection's histogram words or the earlier
// workgroups' counts, then X, C and the basis); the offset sums come after the residuals, so the
// loads they need are hidden behind that arithmetic; survivors are kept as per-iteration bit masks
// and only the set bits are visited when writing.
template <int DT, int R, int V, int HC, bool RIN>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2))) void k_emit_b(SaveGeom g, FastGeom fg, const typename Act<DT>::T *__restrict__ x,
                                                   const float *__restrict__ qp,
                                                   const typename Act<DT>::T *__restrict__ coeff,
                                                   SelState *__restrict__ state, const WgCount *__restrict__ counts, uint32_t chunk_k,
                                                   const uint32_t *__restrict__ maxkey, OutSpec o, float *scale_out,
                                                   int to_list, const uint32_t *__restrict__ hist,
                                                   const uint32_t *__restrict__ fold, int64_t fold_stride)
{
    constexpr int NB = Batch<R>::NB;
    constexpr bool kFold = DT == STACR_DTYPE_BF16;  // bf16: the selection ends here (no count pass)
    static_assert(V <= 8, "survivor masks hold 8 elements per vector");
    __shared__ uint32_t s_wt[kWaves * NB];
    __shared__ uint32_t s_off[kWaves];
    // the workgroup's survivors at their local rank, written out by consecutive threads afterwards
    // (when they fit; otherwise each is written where it is found)
    __shared__ uint32_t s_flat[kEmitStage], s_rv[kEmitStage];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const int64_t w = blockIdx.x - chunk * g.wgs_per_chunk;
    const int64_t wg0 = chunk * g.wgs_per_chunk;  // the chunk's first workgroup
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t col = (int64_t)u * V, colc = min(col, g.d - V);
    const bool col_ok = col < g.d;
    const bool has_rows = row0 < row_end;
    uint32_t hw[kFold ? HC : 1];
    WgCount pre[2];
    if constexpr (kFold) {
        const uint32_t *h1 = hist + (chunk * 3 + 1) * HC * kBins + ((threadIdx.x & 15) << 7);
#pragma unroll
        for (int c = 0; c < HC; ++c) hw[c] = h1[c * kBins];
    } else {
        // counts of the chunk's earlier workgroups (at most two per thread in the usual geometry;
        // the offset block reads any further ones itself)
#pragma unroll
        for (int k = 0; k < 2; ++k) pre[k] = counts[wg0 + min((int64_t)threadIdx.x + k * kBlock, w)];
    }
    FastLoads<DT, R, V, !RIN> ld;  // RIN: x is the stored residual
    // issued whether or not the workgroup has rows: a load under a branch makes every later wait
    // count as if it had not been issued, so waiting for the histogram words would wait for X too
    ld.issue(g, slot, row0, row_end, colc, x, coeff, fg.c_vec != 0);
    float q[V][R];
    if constexpr (!RIN) basis_issue<R, V>(qp + g.d * R, g.d, colc, q);
    SelState st;
    uint32_t rhi[2] = {0u, 0u}, rlo[2] = {0u, 0u};
    const uint32_t *fhi = fold, *flo = fold;
    if constexpr (kFold) {
        SelState sel1;
        st = fold_select<HC>(hw, state[chunk * 3 + 0], &sel1);
        if (w == 0 && threadIdx.x == 0) {
            state[chunk * 3 + 1] = sel1;
            state[chunk * 3 + 2] = st;
        }
        // the earlier workgroups' counts above / equal to the threshold (clamped reads, masked at use)
        const uint32_t b1 = (st.prefix >> 16) & 15u;
        fhi = fold + (int64_t)(b1 + 1) * fold_stride + wg0;
        flo = fold + (int64_t)b1 * fold_stride + wg0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t v = min((int64_t)threadIdx.x + k * kBlock, w);
            rhi[k] = fhi[v];
            rlo[k] = flo[v];
        }
    } else {
        st = state[chunk * 3 + 2];
    }
    const uint32_t mk = *maxkey;
    const uint32_t T = st.prefix;
    const float amax = Act<DT>::rnd(__uint_as_float(mk));
    const float scale = o.bits ? quant_scale(mk, o.bits, amax) : 1.f;
    if (!to_list && blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    if (!has_rows) return;  // uniform: a trailing workgroup with no rows writes nothing
    if constexpr (!RIN) basis_mask<R, V>(col_ok, q);
    float r[NB][V];
    uint32_t msk[NB];  // survivors of iteration i: bits 0..7 above T, bits 8..15 equal to T
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const bool live = col_ok && ld.rows[i] < row_end;
        if constexpr (RIN) {
            ld.x_at(i, live, r[i]);  // the stored residual (zero outside the rows / columns)
        } else {
            float xv[V], ci[R];
            ld.x_at(i, live, xv);
            ld.coeff_row(i, coeff, g.rank, row_end, fg.c_vec != 0, ci);
            batch_residual<DT, R, V>(xv, ci, q, r[i]);
        }
        uint32_t m = 0u;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t key = __float_as_uint(r[i][e]) & 0x7fffffffu;
            m |= (live && key > T) ? 1u << e : 0u;
            m |= (live && key == T) ? 0x100u << e : 0u;
        }
        msk[i] = m;
    }
    // the workgroup's output offset and tie budget, and its number of survivors
    WgOffset wo;
    uint32_t n_out;
    {
        uint32_t gt = 0u, eq = 0u;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t v = threadIdx.x + k * kBlock;
            const WgCount c = kFold ? WgCount{rhi[k], rlo[k] - rhi[k]} : pre[k];
            gt += v < w ? c.gt : 0u;
            eq += v < w ? c.eq : 0u;
        }
        for (int64_t v = threadIdx.x + 2 * kBlock; v < w; v += kBlock) {
            const WgCount c = kFold ? WgCount{fhi[v], flo[v] - fhi[v]} : counts[wg0 + v];
            gt += c.gt;
            eq += c.eq;
        }
        const uint32_t gt_before = block_sum(gt, s_off);
        const uint32_t eq_before = block_sum(eq, s_off);
        const WgCount mine = kFold ? WgCount{fhi[w], flo[w] - fhi[w]} : counts[wg0 + w];
        const uint32_t take = eq_before >= st.need ? 0u : min(mine.eq, st.need - eq_before);
        wo = WgOffset{(uint32_t)chunk * chunk_k + gt_before + min(st.need, eq_before), take};
        n_out = mine.gt + take;
    }
    const bool staged = n_out <= (uint32_t)kEmitStage;  // uniform
    uint32_t cnt[NB], incl[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        cnt[i] = (uint32_t)__popc(msk[i] & 0xffu) | ((uint32_t)__popc(msk[i] >> 8) << 16);
        incl[i] = wave_inclusive_scan(cnt[i]);  // over the wave's lanes, one per iteration
    }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < NB; ++i) s_wt[wave * NB + i] = incl[i];
    __syncthreads();
    uint32_t before_iter = 0u;  // survivors of the batch's earlier iterations (all waves)
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        uint32_t waves_before = 0u, iter_total = 0u;
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) {
            const uint32_t t = s_wt[wv * NB + i];
            waves_before += wv < wave ? t : 0u;
            iter_total += t;
        }
        const uint32_t ex = before_iter + waves_before + incl[i] - cnt[i];
        uint32_t gb = ex & 0xffffu, eb = ex >> 16;
        // this vector's survivors in element order (the lowest remaining element first)
        for (uint32_t m = msk[i]; m != 0u;) {
            const int e = __builtin_ctz((m | (m >> 8)) & 0xffu);
            const uint32_t is_gt = (m >> e) & 1u, is_eq = (m >> (8 + e)) & 1u;
            m &= ~((1u << e) | (0x100u << e));
            if (is_gt || eb < wo.take) {
                const uint32_t local = gb + min(eb, wo.take), pos = wo.off + local;
                float rv = r[i][0];
#pragma unroll
                for (int k = 1; k < V; ++k) rv = e == k ? r[i][k] : rv;
                const uint32_t flat = (uint32_t)(ld.rows[i] * g.d + col + e);
                if (staged) {
                    if (local < (uint32_t)kEmitStage) {  // always, when the counts are consistent
                        s_flat[local] = flat;
                        s_rv[local] = __float_as_uint(rv);
                    }
                } else if (pos >= o.cap) {
                    // unreachable when the counts are consistent; never write out of bounds
                } else if (to_list) {
                    o.list_rbits[pos] = __float_as_uint(rv);
                    o.list_idx[pos] = flat;
                } else {
                    write_entry<DT>(o, pos, flat, rv, scale);
                }
            }
            gb += is_gt;
            eb += is_eq;
        }
        before_iter += iter_total;
    }
    if (staged) {
        __syncthreads();
        for (uint32_t t = threadIdx.x; t < n_out; t += kBlock) {
            const uint32_t pos = wo.off + t, flat = s_flat[t];
            const float rv = __uint_as_float(s_rv[t]);
            if (pos >= o.cap) {
                // unreachable when the counts are consistent; never write out of bounds
            } else if (to_list) {
                o.list_rbits[pos] = __float_as_uint(rv);
                o.list_idx[pos] = flat;
            } else {
                write_entry<DT>(o, pos, flat, rv, scale);
            }
        }
    }
}

// ------------------------------------------------------------------ candidate path (bf16, batched)
// The projection pass keeps, per workgroup, its local candidates: the elements in the level-0 bins
// at or above the cut where the workgroup's own count from the top reaches a quota (several times
// its share of the chunk's k), in ascending flat order, with their residuals; the residual is not
// stored.  The chunk's level-0 bin B0 is known after the pass.  A workgroup whose cut is at or
// below B0, and whose candidates fit kCandCap, holds every element of bin B0 and above among its
// candidates, so the level-1 pass and the emission work on those lists; any other workgroup
// recomputes its residuals from X, C and the basis there (the same values, rarely needed).  The
// selection is the same as the full passes'.

__device__ __forceinline__ uint32_t bf16_key(uint32_t bits16)
{
    return __float_as_uint(bf16_bits_to_f(bits16 & 0xffffu)) & 0x7fffffffu;
}

// Two fp32 values rounded to bf16 by one v_cvt_pk_bf16_f32 (the same rounding as two single
// conversions): lo in bits 15..0, hi in bits 31..16.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi)
{
    typedef __attribute__((ext_vector_type(2))) float f2;
    typedef __attribute__((ext_vector_type(2))) __bf16 b2;
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
}

// Level-0 bins (key bits 30..20) of the two bf16 residuals of a packed word: a bf16 value's key is
// its bits 14..0 shifted up by 16, so its bin is bits 14..4 of the value.
__device__ __forceinline__ uint32_t bin_lo(uint32_t w) { return __builtin_amdgcn_ubfe(w, 4, 11); }
__device__ __forceinline__ uint32_t bin_hi(uint32_t w) { return __builtin_amdgcn_ubfe(w, 20, 11); }

// Pass 1: as k_proj_hist_b (coefficients computed or loaded, level-0 histogram with its coarse
// sums, max key), then the workgroup's cut and its candidates.
template <int R>
__global__ __launch_bounds__(kBlock) void k_proj_cand(SaveGeom g, FastGeom fg, const uint16_t *__restrict__ x,
                                                      const float *__restrict__ qp, uint16_t *__restrict__ coeff,
                                                      uint32_t *__restrict__ hist, uint32_t *__restrict__ maxkey,
                                                      const uint16_t *__restrict__ coeff_in,
                                                      uint32_t *__restrict__ coarse, uint32_t quota,
                                                      uint32_t *__restrict__ cand_idx, uint16_t *__restrict__ cand_val,
                                                      CandMeta *__restrict__ meta)
{
    constexpr int DT = STACR_DTYPE_BF16, V = 8, NB = Batch<R>::NB;
    using T = typename Act<DT>::T;
    // the packed residuals wait for the cut in LDS where they fit in 32 KiB (rank 8; registers
    // would cost this kernel its second wave per SIMD), else in registers
    constexpr bool kLdsRes = NB * kBlock * 16 <= 32768;
    __shared__ uint32_t s_hist[kBins];
    __shared__ __align__(16) float s_part[kWaves * 64];
    __shared__ __align__(16) float s_c[kWaves * 64];
    __shared__ uint32_t s_wmax[kWaves];
    __shared__ uint32_t s_wt[kWaves * NB];
    __shared__ uint32_t s_cut;
    __shared__ uint4 s_res[kLdsRes ? NB * kBlock : 1];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    if (row0 >= row_end) return;  // a trailing workgroup with no rows (uniform; later passes skip it)
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t col = (int64_t)u * V, colc = min(col, g.d - V);
    const bool col_ok = col < g.d;
    FastLoads<DT, R, V, false> ld;
    ld.issue(g, slot, row0, row_end, colc, reinterpret_cast<const T *>(x), nullptr, false);
    float q[V][R];
    uint4 qw[R];
    const uint16_t *qph = reinterpret_cast<const uint16_t *>(qp + 2 * g.d * R);
#pragma unroll
    for (int j = 0; j < R; ++j) qw[j] = *reinterpret_cast<const uint4 *>(qph + j * g.d + colc);
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    uint32_t kmax = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const uint32_t w[4] = {qw[j].x, qw[j].y, qw[j].z, qw[j].w};
#pragma unroll
        for (int e = 0; e < V; ++e) q[e][j] = Act<DT>::ld((T)((w[e / 2] >> (16 * (e & 1))) & 0xffffu));
    }
    basis_mask<R, V>(col_ok, q);
    float c[64];
    if (coeff_in) {
        batch_coeff_load<DT, R>(reinterpret_cast<const T *>(coeff_in), g.rank, ld.rows, row_end, fg.c_vec != 0, c);
    } else {
        float acc[64];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const bool live = col_ok && ld.rows[i] < row_end;
            const uint4 xr = live ? ld.raw[i] : make_uint4(0u, 0u, 0u, 0u);
            const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const uint32_t w[4] = {qw[j].x, qw[j].y, qw[j].z, qw[j].w};
                float sum = 0.f;
#pragma unroll
                for (int k = 0; k < 4; ++k) sum = dot2<DT>(xw[k], w[k], sum);
                acc[i * R + j] = sum;
            }
        }
        batch_coeff_from_acc<DT, R>(acc, fg.W, slot, s_part, s_c, row0, g.rpi, row_end, g.rank,
                                    reinterpret_cast<T *>(coeff), c);
    }
    // residuals r = rnd(x - rnd(sum_j c_j q_j)) (the chain of batch_residual), rounded two at a time
    // into the packed bf16 words they are kept as; the histogram bins and the max key come from
    // those words (the max as a packed 16-bit max of |r|'s bits)
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 kmax2 = {0, 0};
    uint4 rp[kLdsRes ? 1 : NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (!(col_ok && ld.rows[i] < row_end)) continue;
        float xv[V];
        ld.x_at(i, true, xv);
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float p0 = 0.f, p1 = 0.f;
#pragma unroll
            for (int j = 0; j < R; ++j) {
                p0 = fmaf(c[i * R + j], q[2 * k][j], p0);
                p1 = fmaf(c[i * R + j], q[2 * k + 1][j], p1);
            }
            const uint32_t pb = bf16_pair(p0, p1);
            w[k] = bf16_pair(xv[2 * k] - __uint_as_float(pb << 16), xv[2 * k + 1] - __uint_as_float(pb & 0xffff0000u));
            atomicAdd(&s_hist[bin_lo(w[k])], 1u);
            atomicAdd(&s_hist[bin_hi(w[k])], 1u);
            kmax2 = __builtin_elementwise_max(kmax2, __builtin_bit_cast(u16x2, w[k] & 0x7fff7fffu));
        }
        const uint4 pr = make_uint4(w[0], w[1], w[2], w[3]);
        if constexpr (kLdsRes) s_res[i * kBlock + threadIdx.x] = pr;
        else rp[i] = pr;
    }
    kmax = (uint32_t)max(kmax2.x, kmax2.y) << 16;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    if (lane == 0) s_wmax[wave] = kmax;
    __syncthreads();
    // the cut: the highest bin where the count from the top reaches the quota (bin 0 when the
    // workgroup has fewer keys), from 64 sums of 32 bins and then the chosen 32 bins
    if (wave == 0) {
        constexpr int FB = kBins / kCoarse;
        uint32_t suf = 0u;
#pragma unroll 8
        for (int b = 0; b < FB; ++b) suf += s_hist[lane * FB + b];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_down(suf, off, 64);
            if (lane + off < 64) suf += y;
        }
        const uint64_t m = __ballot(suf >= quota);
        uint32_t cut = 0u;
        if (m != 0ull) {
            const int cb = 63 - __clzll(m);
            const uint32_t need1 = quota - (cb < 63 ? (uint32_t)__shfl((int)suf, cb + 1, 64) : 0u);
            const int fl = lane & (FB - 1);
            uint32_t sf = s_hist[cb * FB + fl];
#pragma unroll
            for (int off = 1; off < FB; off <<= 1) {
                const uint32_t y = __shfl_down(sf, off, FB);
                if (fl + off < FB) sf += y;
            }
            const uint64_t mf = __ballot(sf >= need1) & ((1ull << FB) - 1);
            cut = (uint32_t)(cb * FB + (mf ? 63 - __clzll(mf) : 0));
        }
        if (lane == 0) s_cut = cut;
    }
    __syncthreads();
    const uint32_t cut = s_cut;
    // the candidates in ascending flat order: (iteration, wave, lane, element)
    uint32_t msk[NB], cnt[NB], incl[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        uint32_t m = 0u;
        if (col_ok && ld.rows[i] < row_end) {
            const uint4 pr = kLdsRes ? s_res[i * kBlock + threadIdx.x] : rp[kLdsRes ? 0 : i];
            const uint32_t w[4] = {pr.x, pr.y, pr.z, pr.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                m |= bin_lo(w[k]) >= cut ? 1u << (2 * k) : 0u;
                m |= bin_hi(w[k]) >= cut ? 2u << (2 * k) : 0u;
            }
        }
        msk[i] = m;
        cnt[i] = (uint32_t)__popc(m);
        incl[i] = wave_inclusive_scan(cnt[i]);
    }
    if (lane == 63)
#pragma unroll
        for (int i = 0; i < NB; ++i) s_wt[wave * NB + i] = incl[i];
    __syncthreads();
    uint32_t before_iter = 0u;
    uint32_t *ci = cand_idx + (int64_t)blockIdx.x * kCandCap;
    uint16_t *cv = cand_val + (int64_t)blockIdx.x * kCandCap;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        uint32_t waves_before = 0u, iter_total = 0u;
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) {
            const uint32_t t = s_wt[wv * NB + i];
            waves_before += wv < wave ? t : 0u;
            iter_total += t;
        }
        uint32_t pos = before_iter + waves_before + incl[i] - cnt[i];
        if (msk[i]) {
            const uint4 pr = kLdsRes ? s_res[i * kBlock + threadIdx.x] : rp[kLdsRes ? 0 : i];
            const uint32_t wd[4] = {pr.x, pr.y, pr.z, pr.w};
            for (uint32_t m = msk[i]; m != 0u; m &= m - 1u, ++pos) {
                const int e = __builtin_ctz(m);
                uint32_t word = wd[0];
#pragma unroll
                for (int k = 1; k < 4; ++k) word = (e >> 1) == k ? wd[k] : word;
                if (pos < (uint32_t)kCandCap) {
                    ci[pos] = (uint32_t)(ld.rows[i] * g.d + col + e);
                    cv[pos] = (uint16_t)((word >> (16 * (e & 1))) & 0xffffu);
                }
            }
        }
        before_iter += iter_total;
    }
    if (threadIdx.x == 0) meta[blockIdx.x] = CandMeta{cut, before_iter};
    // this workgroup's copy of the chunk histogram and of the max key (as k_proj_hist_b)
    const int copy = (int)(blockIdx.x % g.hcopies);
    uint32_t *gh = hist + ((chunk * 3 + 0) * g.hcopies + copy) * kBins;
    for (int b = threadIdx.x; b < kBins; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
    if (threadIdx.x < kCoarse) {
        uint32_t sum = 0u;
#pragma unroll 8
        for (int b = 0; b < kBins / kCoarse; ++b) sum += s_hist[threadIdx.x * (kBins / kCoarse) + b];
        if (sum) atomicAdd(&coarse[(chunk * g.hcopies + copy) * kCoarse + threadIdx.x], sum);
    }
    if (threadIdx.x == 0) {
        uint32_t mx = 0u;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mx = max(mx, s_wmax[w]);
        if (mx) atomicMax(maxkey + copy * kMaxKeyStride, mx);
    }
}

// One vector's residual recomputed from X, C and the basis (the candidate passes' fallback, one
// iteration at a time so that it does not set the kernels' register budget); false outside the
// matrix or the workgroup's rows.
template <int R>
__device__ __forceinline__ bool cand_residual(const SaveGeom &g, const uint16_t *__restrict__ x,
                                              const uint16_t *__restrict__ coeff, const float (&q)[8][R], int64_t row,
                                              int64_t row_end, int64_t col, bool col_ok, float (&r)[8])
{
    constexpr int DT = STACR_DTYPE_BF16;
    const bool live = col_ok && row < row_end;
    float xv[8], c[R];
    unpack_raw<DT, 8>(load_raw<DT, 8>(x + row * g.d + col, live), xv);
    load_coeff<DT, R>(coeff, row, g.rank, live, c);
    batch_residual<DT, R, 8>(xv, c, q, r);
    return live;
}

// A thread's 8 consecutive candidate values (16 bytes), and their flat indices; entries at or past
// `count` are read (inside the workgroup's region) but not used.
struct CandVals {
    uint32_t w[4];
    __device__ __forceinline__ uint32_t bits(int j) const { return (w[j >> 1] >> (16 * (j & 1))) & 0xffffu; }
};

// Level 1 (bf16, batched, candidates): the level-0 selection, then the histogram of key bits
// 19..16 inside B0 and the per-workgroup records of k_refine_hist_b, from the candidates.
template <int R, int HC>
__global__ __launch_bounds__(kBlock) void k_refine_cand(SaveGeom g, FastGeom fg, const uint16_t *__restrict__ x,
                                                        const float *__restrict__ qp, const uint16_t *__restrict__ coeff,
                                                        uint32_t *__restrict__ hist, SelState *__restrict__ state,
                                                        uint32_t k_full, uint32_t k_last, uint32_t *__restrict__ maxkey,
                                                        uint32_t *__restrict__ fold, int64_t fold_stride,
                                                        const uint32_t *__restrict__ coarse,
                                                        const uint16_t *__restrict__ cand_val,
                                                        const CandMeta *__restrict__ meta)
{
    constexpr int NB = Batch<R>::NB;
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_above[kWaves];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const bool has_rows = row0 < row_end;
    const SelState sp = prev_state(0, state, chunk, g.n_chunks, k_full, k_last);
    uint32_t cv[HC];
#pragma unroll
    for (int h = 0; h < HC; ++h) cv[h] = coarse[(chunk * HC + h) * kCoarse + (threadIdx.x & 63)];
    const CandMeta mine = meta[has_rows ? blockIdx.x : 0];
    // the candidate values go out before the selection's histogram words (only the list's used
    // part: the threads past it read nothing)
    CandVals vals;
    {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if ((uint32_t)(kCandPer * threadIdx.x) < min(mine.count, (uint32_t)kCandCap))
            v = *reinterpret_cast<const uint4 *>(cand_val + (int64_t)blockIdx.x * kCandCap + kCandPer * threadIdx.x);
        vals.w[0] = v.x; vals.w[1] = v.y; vals.w[2] = v.z; vals.w[3] = v.w;
    }
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    const SelState sel = select_level0<HC>(cv, hist + chunk * 3 * HC * kBins, sp);
    if (blockIdx.x % g.wgs_per_chunk == 0 && threadIdx.x == 0) state[chunk * 3 + 0] = sel;
    if (HC > 1 && blockIdx.x == 0 && threadIdx.x == 0) {  // fold the max key's copies into the first
        uint32_t m = maxkey[0];
#pragma unroll
        for (int c = 1; c < HC; ++c) m = max(m, maxkey[c * kMaxKeyStride]);
        maxkey[0] = m;
    }
    if (!has_rows) {
        if (threadIdx.x <= 16) fold[threadIdx.x * fold_stride + blockIdx.x] = 0u;
        return;
    }
    const uint32_t prefix = sel.prefix;  // B0
    const bool valid = mine.count <= (uint32_t)kCandCap && mine.cut <= prefix;  // uniform
    __syncthreads();  // s_hist is clear
    uint32_t above = 0u;
    if (valid) {
#pragma unroll
        for (int j = 0; j < kCandPer; ++j) {
            if (kCandPer * threadIdx.x + j >= mine.count) break;
            const uint32_t key = bf16_key(vals.bits(j));
            if ((key >> kDigitShift[0]) == prefix) atomicAdd(&s_hist[(key >> kDigitShift[1]) & (kDigitBins[1] - 1)], 1u);
            above += (key >> kDigitShift[0]) > prefix;
        }
    } else {
        const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
        const int64_t col = (int64_t)u * 8, colc = min(col, g.d - 8);
        const bool col_ok = col < g.d;
        float q[8][R];
        basis_issue<R, 8>(qp + g.d * R, g.d, colc, q);
        basis_mask<R, 8>(col_ok, q);
#pragma unroll 1
        for (int i = 0; i < NB; ++i) {
            float r[8];
            if (!cand_residual<R>(g, x, coeff, q, row0 + (int64_t)i * g.rpi + slot, row_end, col, col_ok, r)) continue;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t key = __float_as_uint(r[e]) & 0x7fffffffu;
                if ((key >> kDigitShift[0]) == prefix) atomicAdd(&s_hist[(key >> kDigitShift[1]) & (kDigitBins[1] - 1)], 1u);
                above += (key >> kDigitShift[0]) > prefix;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) above += (uint32_t)__shfl_xor((int)above, off, 64);
    if ((threadIdx.x & 63) == 0) s_above[threadIdx.x >> 6] = above;
    __syncthreads();
    if (threadIdx.x <= 16) {  // cum[b] for b = threadIdx.x (16: above B0 only), as k_refine_hist_b
        uint32_t c = 0u;
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) c += s_above[wv];
        for (int b = threadIdx.x; b < 16; ++b) c += s_hist[b << 7];
        fold[threadIdx.x * fold_stride + blockIdx.x] = c;
    }
    uint32_t *gh = hist + ((chunk * 3 + 1) * HC + blockIdx.x % HC) * kBins;
    for (int b = threadIdx.x; b < kDigitBins[1]; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
}

// The emission's fallback for a workgroup without a usable candidate list: its residuals
// recomputed (RIN: read from the stored residual) one iteration at a time, survivors compacted in
// the order of k_emit_b and handed to `put` (position, flat index, value).
template <int R, bool RIN, typename Put>
__device__ __forceinline__ void emit_cand_fallback(const SaveGeom &g, const FastGeom &fg, const uint16_t *__restrict__ x,
                                                   const float *__restrict__ qp, const uint16_t *__restrict__ coeff,
                                                   int64_t row0, int64_t row_end, uint32_t T, const WgOffset &wo,
                                                   uint32_t *s_wt, Put &put)
{
    constexpr int NB = Batch<R>::NB;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = threadIdx.x >> g.log2L, u = threadIdx.x & (g.L - 1);
    const int64_t col = (int64_t)u * 8, colc = min(col, g.d - 8);
    const bool col_ok = col < g.d;
    float q[8][RIN ? 1 : R];
    if constexpr (!RIN) {
        basis_issue<R, 8>(qp + g.d * R, g.d, colc, q);
        basis_mask<R, 8>(col_ok, q);
    }
    uint32_t before_iter = 0u;  // survivors of the earlier iterations (all waves)
#pragma unroll 1
    for (int i = 0; i < NB; ++i) {
        const int64_t row = row0 + (int64_t)i * g.rpi + slot;
        float r[8];
        bool live;
        if constexpr (RIN) {
            live = col_ok && row < row_end;
            unpack_raw<STACR_DTYPE_BF16, 8>(load_raw<STACR_DTYPE_BF16, 8>(x + row * g.d + col, live), r);
        } else {
            live = cand_residual<R>(g, x, coeff, q, row, row_end, col, col_ok, r);
        }
        uint32_t m = 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t k = __float_as_uint(r[e]) & 0x7fffffffu;
            m |= (live && k > T) ? 1u << e : 0u;
            m |= (live && k == T) ? 0x100u << e : 0u;
        }
        const uint32_t cnt = (uint32_t)__popc(m & 0xffu) | ((uint32_t)__popc(m >> 8) << 16);
        const uint32_t incl = wave_inclusive_scan(cnt);
        if (lane == 63) s_wt[wave] = incl;
        __syncthreads();
        uint32_t waves_before = 0u, iter_total = 0u;
#pragma unroll
        for (int wv = 0; wv < kWaves; ++wv) {
            const uint32_t t = s_wt[wv];
            waves_before += wv < wave ? t : 0u;
            iter_total += t;
        }
        __syncthreads();  // s_wt is free for the next iteration
        const uint32_t ex = before_iter + waves_before + incl - cnt;
        uint32_t gb = ex & 0xffffu, eb = ex >> 16;
        while (m != 0u) {
            const int e = __builtin_ctz((m | (m >> 8)) & 0xffu);
            const uint32_t is_gt = (m >> e) & 1u, is_eq = (m >> (8 + e)) & 1u;
            m &= ~((1u << e) | (0x100u << e));
            if (is_gt || eb < wo.take) {
                float rv = r[0];
#pragma unroll
                for (int k = 1; k < 8; ++k) rv = e == k ? r[k] : rv;
                put(wo.off + gb + min(eb, wo.take), (uint32_t)(row * g.d + col + e), rv);
            }
            gb += is_gt;
            eb += is_eq;
        }
        before_iter += iter_total;
    }
}

// Emission (bf16, batched, candidates): the final selection and the workgroup's offset and tie
// budget as in k_emit_b, then its survivors from the candidate list (or, for a workgroup without a
// usable list, from recomputed residuals) quantized and written in ascending flat order.
template <int R, int HC, bool RIN = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2))) void k_emit_cand(
    SaveGeom g, FastGeom fg, const uint16_t *__restrict__ x, const float *__restrict__ qp,
    const uint16_t *__restrict__ coeff, SelState *__restrict__ state, uint32_t chunk_k,
    const uint32_t *__restrict__ maxkey, OutSpec o, float *scale_out, int to_list, const uint32_t *__restrict__ hist,
    const uint32_t *__restrict__ fold, int64_t fold_stride, const uint32_t *__restrict__ cand_idx,
    const uint16_t *__restrict__ cand_val, const CandMeta *__restrict__ meta, uint32_t *__restrict__ census,
    uint32_t n_entries, uint32_t census_feats)
{
    constexpr int DT = STACR_DTYPE_BF16;
    __shared__ uint32_t s_off[kWaves];
    __shared__ uint32_t s_wt[kWaves];
    // with a census: this workgroup's entries per feature of the layer, two 16-bit counts a word
    // (features f and f + 2048; a workgroup emits at most kCandCap entries, so no half overflows):
    // census_feats <= 4096
    __shared__ uint32_t s_feat[kBins];
    int64_t chunk, row0, row_end;
    wg_rows(g, blockIdx.x, chunk, row0, row_end);
    const int64_t w = blockIdx.x - chunk * g.wgs_per_chunk;
    const int64_t wg0 = chunk * g.wgs_per_chunk;
    const bool has_rows = row0 < row_end;
    uint32_t hw[HC];
    {
        const uint32_t *h1 = hist + (chunk * 3 + 1) * HC * kBins + ((threadIdx.x & 15) << 7);
#pragma unroll
        for (int c = 0; c < HC; ++c) hw[c] = h1[c * kBins];
    }
    const CandMeta mine = meta[has_rows ? blockIdx.x : 0];
    // the candidates go out before the selection's and the offsets' words (only the list's used
    // part)
    CandVals vals;
    uint32_t flat[kCandPer];
    {
        const int64_t base = (int64_t)blockIdx.x * kCandCap + kCandPer * threadIdx.x;
        const uint32_t n_list = min(mine.count, (uint32_t)kCandCap), t0 = kCandPer * threadIdx.x;
        uint4 v = make_uint4(0u, 0u, 0u, 0u), f0 = v, f1 = v;
        if (t0 < n_list) {
            v = *reinterpret_cast<const uint4 *>(cand_val + base);
            f0 = *reinterpret_cast<const uint4 *>(cand_idx + base);
        }
        if (t0 + 4 < n_list) f1 = *reinterpret_cast<const uint4 *>(cand_idx + base + 4);
        vals.w[0] = v.x; vals.w[1] = v.y; vals.w[2] = v.z; vals.w[3] = v.w;
        flat[0] = f0.x; flat[1] = f0.y; flat[2] = f0.z; flat[3] = f0.w;
        flat[4] = f1.x; flat[5] = f1.y; flat[6] = f1.z; flat[7] = f1.w;
    }
    SelState sel1;
    const SelState st = fold_select<HC>(hw, state[chunk * 3 + 0], &sel1);
    if (w == 0 && threadIdx.x == 0) {
        state[chunk * 3 + 1] = sel1;
        state[chunk * 3 + 2] = st;
    }
    const uint32_t b1 = (st.prefix >> 16) & 15u;
    const uint32_t *fhi = fold + (int64_t)(b1 + 1) * fold_stride + wg0;
    const uint32_t *flo = fold + (int64_t)b1 * fold_stride + wg0;
    const uint32_t mk = *maxkey;
    const uint32_t T = st.prefix;
    const float amax = Act<DT>::rnd(__uint_as_float(mk));
    const float scale = o.bits ? quant_scale(mk, o.bits, amax) : 1.f;
    if (!to_list && blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    if (!has_rows) return;  // uniform: a trailing workgroup with no rows writes nothing
    // the census counts features of the layer's rows (census_feats = segs x g.d when rows are split
    // into segments of g.d features; segment rows run in flat order); power-of-two widths: a mask
    const uint32_t cfeat = census_feats, segs = cfeat / (uint32_t)g.d;
    const uint32_t dmask = (cfeat & (cfeat - 1)) == 0 ? cfeat - 1u : 0u;
    const uint32_t cwords = cfeat < (uint32_t)kBins ? cfeat : (uint32_t)kBins;
    if (census)  // (cleared before the offset sums' barriers)
        for (uint32_t f = threadIdx.x; f < cwords; f += kBlock) s_feat[f] = 0u;
    // the workgroup's output offset and tie budget (the earlier workgroups' records)
    WgOffset wo;
    {
        uint32_t gt = 0u, eq = 0u;
        for (int64_t v = threadIdx.x; v < w; v += kBlock) {
            const uint32_t hi = fhi[v], lo = flo[v];
            gt += hi;
            eq += lo - hi;
        }
        const uint32_t gt_before = block_sum(gt, s_off);
        const uint32_t eq_before = block_sum(eq, s_off);
        const uint32_t my_eq = flo[w] - fhi[w];
        const uint32_t take = eq_before >= st.need ? 0u : min(my_eq, st.need - eq_before);
        wo = WgOffset{(uint32_t)chunk * chunk_k + gt_before + min(st.need, eq_before), take};
    }
    auto put = [&](uint32_t pos, uint32_t fl, float rv) {
        if (pos >= o.cap) {
            // unreachable when the counts are consistent; never write out of bounds
        } else if (to_list) {
            o.list_rbits[pos] = __float_as_uint(rv);
            o.list_idx[pos] = fl;
        } else {
            write_entry<DT>(o, pos, fl, rv, scale);
        }
        if (census) {
            const uint32_t f = dmask ? fl & dmask : fl % cfeat;
            atomicAdd(&s_feat[f & (kBins - 1)], f >= (uint32_t)kBins ? 0x10000u : 1u);
        }
    };
    const bool valid = mine.count <= (uint32_t)kCandCap && mine.cut <= (T >> kDigitShift[0]);  // uniform
    if (valid) {
        uint32_t ngt = 0u, neq = 0u, key[kCandPer];
#pragma unroll
        for (int j = 0; j < kCandPer; ++j) {
            const bool in = kCandPer * threadIdx.x + j < mine.count;
            key[j] = in ? bf16_key(vals.bits(j)) : 0u;
            ngt += in && key[j] > T;
            neq += in && key[j] == T;
        }
        uint32_t tot;
        const uint32_t pre = block_exclusive_scan(ngt | (neq << 16), s_off, &tot);
        uint32_t gb = pre & 0xffffu, eb = pre >> 16;
#pragma unroll
        for (int j = 0; j < kCandPer; ++j) {
            if (kCandPer * threadIdx.x + j >= mine.count) break;
            const bool is_gt = key[j] > T, is_eq = key[j] == T;
            if (is_gt || (is_eq && eb < wo.take)) put(wo.off + gb + min(eb, wo.take), flat[j], bf16_bits_to_f(vals.bits(j)));
            gb += is_gt;
            eb += is_eq;
        }
    } else {
        emit_cand_fallback<R, RIN>(g, fg, x, qp, coeff, row0, row_end, T, wo, s_wt, put);
    }
    if (census) {  // the entries per feature (copy w % 8) and, at a block's first row, its first entry
        __syncthreads();
        uint32_t *counts = census + (int64_t)(blockIdx.x % kCensusCopies) * cfeat;
        for (uint32_t f = threadIdx.x; f < cwords; f += kBlock) {
            const uint32_t v = s_feat[f];
            if (v & 0xffffu) atomicAdd(&counts[f], v & 0xffffu);
            if (v >> 16) atomicAdd(&counts[f + kBins], v >> 16);
        }
        uint32_t *bstart = census + (int64_t)kCensusCopies * cfeat;
        const int64_t seg_rows = (int64_t)kCensusRows * segs;  // a block of the layer's rows in segment rows
        if (threadIdx.x == 0 && row0 % seg_rows == 0) bstart[row0 / seg_rows] = wo.off;
        if (blockIdx.x == 0 && threadIdx.x == 0) bstart[(g.rows / segs + kCensusRows - 1) / kCensusRows] = n_entries;
    }
}

// ------------------------------------------------------------------ trim pass over the list
__global__ __launch_bounds__(kBlock) void k_list_hist(int lvl, const uint32_t *__restrict__ rbits, int64_t n,
                                                      uint32_t *__restrict__ hist, const SelState *__restrict__ state)
{
    __shared__ uint32_t s_hist[kBins];
    for (int b = threadIdx.x; b < kBins; b += kBlock) s_hist[b] = 0u;
    __syncthreads();
    const uint32_t prefix = lvl ? state[lvl - 1].prefix : 0u;
    const int match_shift = lvl ? kDigitShift[lvl - 1] : 31, dshift = kDigitShift[lvl];
    const uint32_t dmask = (uint32_t)kDigitBins[lvl] - 1u;
    const int64_t start = (int64_t)blockIdx.x * kListBlock + threadIdx.x * (kListBlock / kBlock);
    for (int k = 0; k < kListBlock / kBlock; ++k) {
        const int64_t i = start + k;
        if (i >= n) break;
        const uint32_t key = rbits[i] & 0x7fffffffu;
        if ((key >> match_shift) == prefix) atomicAdd(&s_hist[(key >> dshift) & dmask], 1u);
    }
    __syncthreads();
    uint32_t *gh = hist + lvl * kBins;
    for (int b = threadIdx.x; b < kDigitBins[lvl]; b += kBlock)
        if (s_hist[b]) atomicAdd(&gh[b], s_hist[b]);
}

__global__ __launch_bounds__(kBlock) void k_list_count(const uint32_t *__restrict__ rbits, int64_t n,
                                                       const SelState *__restrict__ state, WgCount *__restrict__ counts)
{
    __shared__ uint32_t s_tot[kWaves];
    const uint32_t T = state[2].prefix;
    const int64_t start = (int64_t)blockIdx.x * kListBlock + threadIdx.x * (kListBlock / kBlock);
    uint32_t gt = 0u, eq = 0u;
    for (int k = 0; k < kListBlock / kBlock; ++k) {
        const int64_t i = start + k;
        if (i >= n) break;
        const uint32_t key = rbits[i] & 0x7fffffffu;
        gt += key > T;
        eq += key == T;
    }
    const uint32_t tg = block_sum(gt, s_tot);
    const uint32_t te = block_sum(eq, s_tot);
    if (threadIdx.x == 0) counts[blockIdx.x] = WgCount{tg, te};
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_list_emit(const uint32_t *__restrict__ rbits, const uint32_t *__restrict__ lidx,
                                                      int64_t n, const SelState *__restrict__ state,
                                                      const WgOffset *__restrict__ offs,
                                                      const uint32_t *__restrict__ maxkey, OutSpec o, float *scale_out)
{
    __shared__ uint32_t s_tot[kWaves];
    const uint32_t T = state[2].prefix;
    const WgOffset wo = offs[blockIdx.x];
    const float amax = Act<DT>::rnd(__uint_as_float(*maxkey));
    const float scale = o.bits ? quant_scale(*maxkey, o.bits, amax) : 1.f;
    if (blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    constexpr int per = kListBlock / kBlock;
    const int64_t start = (int64_t)blockIdx.x * kListBlock + threadIdx.x * per;
    uint32_t ngt = 0u, neq = 0u;
    for (int k = 0; k < per; ++k) {
        const int64_t i = start + k;
        if (i >= n) break;
        const uint32_t key = rbits[i] & 0x7fffffffu;
        ngt += key > T;
        neq += key == T;
    }
    uint32_t tot;
    const uint32_t ex = block_exclusive_scan(ngt | (neq << 16), s_tot, &tot);
    uint32_t gb = ex & 0xffffu, eb = ex >> 16;
    for (int k = 0; k < per; ++k) {
        const int64_t i = start + k;
        if (i >= n) break;
        const uint32_t rb = rbits[i];
        const uint32_t key = rb & 0x7fffffffu;
        const bool is_gt = key > T, is_eq = key == T;
        if (is_gt || (is_eq && eb < wo.take)) {
            const uint32_t pos = wo.off + gb + min(eb, wo.take);
            if (pos < o.cap) write_entry<DT>(o, pos, lidx[i], __uint_as_float(rb), scale);
        }
        gb += is_gt;
        eb += is_eq;
    }
}

__global__ void k_pack_int4(const int8_t *__restrict__ q, int64_t n, uint8_t *__restrict__ out)
{
    const int64_t m = (n + 1) / 2;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < m; i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t lo = (uint32_t)q[2 * i] & 0xfu;
        const uint32_t hi = 2 * i + 1 < n ? ((uint32_t)q[2 * i + 1] & 0xfu) : 0u;
        out[i] = (uint8_t)(lo | (hi << 4));
    }
}

// ------------------------------------------------------------------ standalone quantizer
// quantize_values (stacr/quant.py:49-65) on a value vector: max |v| then the symmetric rounding.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_absmax(const typename Act<DT>::T *__restrict__ v, int64_t n,
                                                   uint32_t *__restrict__ maxkey)
{
    uint32_t m = 0u;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        m = max(m, __float_as_uint(Act<DT>::ld(v[i])) & 0x7fffffffu);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
    if ((threadIdx.x & 63) == 0 && m) atomicMax(maxkey, m);
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_quantize(const typename Act<DT>::T *__restrict__ v, int64_t n, int bits,
                                                     const uint32_t *__restrict__ maxkey, void *__restrict__ data,
                                                     float *__restrict__ scale_out)
{
    const float scale = quant_scale(*maxkey, bits, __uint_as_float(*maxkey));
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
    if (bits == 8) {
        for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
            static_cast<int8_t *>(data)[i] = quantize_one(Act<DT>::ld(v[i]), scale, 8);
    } else {
        const int64_t nb = (n + 1) / 2;
        for (int64_t b = (int64_t)blockIdx.x * kBlock + threadIdx.x; b < nb; b += (int64_t)gridDim.x * kBlock) {
            const uint32_t lo = (uint32_t)quantize_one(Act<DT>::ld(v[2 * b]), scale, 4) & 0xfu;
            const uint32_t hi = 2 * b + 1 < n ? ((uint32_t)quantize_one(Act<DT>::ld(v[2 * b + 1]), scale, 4) & 0xfu) : 0u;
            static_cast<uint8_t *>(data)[b] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// ------------------------------------------------------------------ host side
int next_pow2(int64_t v)
{
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

int ilog2(int v)
{
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

int pad_rank(int rank) { return rank <= 4 ? 4 : rank <= 8 ? 8 : rank <= 16 ? 16 : 32; }

int grid_for(int64_t n) { return (int)hmin<int64_t>(4096, hmax<int64_t>(1, (n + kBlock - 1) / kBlock)); }

struct Plan {
    SaveGeom g;
    int V, R;
    bool qreg;
    bool fast;  // the batched kernels (one batch per workgroup)
    bool fold;  // bf16 on the batched path: the emission pass ends the selection (no count pass)
    int64_t n_wgs;
    int Rq;  // the basis copies' padded rank (R, except on the wide path)
    // wide rows (16-bit, see make_plan): g, V, R, fast and n_wgs describe the stored residual as
    // f * rows rows of d / f columns (the later passes); gw, Rq, mvw, ntw and n_wgs_w the
    // projection pass
    bool wide;
    SaveGeom gw;
    int mvw, ntw;
    int64_t n_wgs_w;
    // bf16 on the batched path with a residual and not wide: the candidate passes (k_proj_cand,
    // k_refine_cand, k_emit_cand) with the workgroups' quota
    bool cand;
    uint32_t quota;
    // bf16 on the batched passes over a stored residual (wide rows, or a quota past the list): the
    // level-1 pass writes the candidate lists (bin B0 and above) and k_emit_cand reads them
    bool cand_rin;
    bool trim;
    int64_t n_list_blocks;
    int yc;  // basis columns the projection covers (the rank, or the Y columns the wide pass serves)
};

Plan make_plan_rows(const StacrSaveArgs &a)
{
    Plan p{};
    const int vec = a.dtype == STACR_DTYPE_F32 ? 4 : 8;
    const bool aligned = ((uintptr_t)a.x % 16) == 0;
    p.V = (a.feats % vec == 0 && aligned) ? vec : 1;
    p.R = pad_rank(a.rank);
    p.Rq = p.R;
    SaveGeom &g = p.g;
    g.rows = a.rows;
    g.d = a.feats;
    g.rank = a.rank;
    const int64_t vecs = (a.feats + p.V - 1) / p.V;
    g.L = (int)hmin<int64_t>(kBlock, hmax<int64_t>(16, next_pow2(vecs)));
    g.log2L = ilog2(g.L);
    g.rpi = kBlock / g.L;
    g.mv = (int)((vecs + g.L - 1) / g.L);
    // without a residual there is no selection, and so no chunk: the rows are one span
    g.chunk_rows = a.mode == STACR_MODE_GLOBAL_TOPK || a.k_total == 0 ? a.rows : min(a.chunk_rows, a.rows);
    if (g.chunk_rows < 1) g.chunk_rows = 1;
    g.n_chunks = (a.rows + g.chunk_rows - 1) / g.chunk_rows;
    int64_t target = hmax<int64_t>(1, 16384 / hmax<int64_t>(1, a.feats));
    int64_t rpw = 1;
    while (rpw * 2 <= target) rpw *= 2;
    if (a.mode != STACR_MODE_GLOBAL_TOPK && a.k_total > 0)
        while (rpw > 1 && g.chunk_rows % rpw) rpw >>= 1;
    p.qreg = g.mv == 1 && p.V * p.R <= 128;
    // the batched kernels take exactly one batch (64 / R iterations of the row slots) per workgroup
    const int vec_full = a.dtype == STACR_DTYPE_F32 ? 4 : 8;
    p.fast = p.qreg && p.V == vec_full && p.V * p.R <= 64 && g.mv == 1 && g.L >= 64;
    if (p.fast) rpw = hmin<int64_t>(rpw, (int64_t)(64 / p.R) * g.rpi);
    g.rows_per_wg = rpw;
    g.wgs_per_chunk = (g.chunk_rows + rpw - 1) / rpw;
    g.hcopies = p.fast && g.wgs_per_chunk >= 128 ? kHistCopies : 1;
    p.fold = p.fast && a.dtype == STACR_DTYPE_BF16;
    p.n_wgs = g.n_chunks * g.wgs_per_chunk;
    p.trim = a.k_sum > a.k_total;
    p.n_list_blocks = (a.k_sum + kListBlock - 1) / kListBlock;
    return p;
}

// 16-bit rows the batched kernels do not take: 2048 < d <= 8192 features (d % 8 == 0, aligned,
// rank <= 16), or rank 16 at d <= 2048.  The projection pass (k_proj_hist_w) gives a row to
// ntw threads with mvw vectors each and stores the residual; the later passes run on the batched
// kernels over that residual viewed as f * rows rows of d / f <= 2048 columns (row-major, so the
// flat indices are the same; chunks are f * chunk_rows such rows, so the chunks are the same) at
// rank 8 (they read neither the basis nor C).
Plan make_plan_wide(const StacrSaveArgs &a)
{
    Plan p = make_plan_rows(a);
    if (p.fast || a.dtype == STACR_DTYPE_F32 || p.V != 8 || p.R > 16 || a.feats > 8192) return p;
    int mv, nt;
    if (p.R <= 8) {
        if (a.feats <= 2048) return p;  // (the batched kernels take these when aligned)
        mv = 2;
        nt = a.feats <= 4096 ? 256 : 512;
    } else {
        // (fp16 at rank 16 above 4096 features stays on the per-row kernels: the wide kernel's
        // fp16 conversions push that shape past 256 registers)
        if (a.feats > 4096 && a.dtype == STACR_DTYPE_F16) return p;
        mv = a.feats <= 4096 ? 1 : 2;
        nt = a.feats <= 2048 ? 256 : 512;
    }
    int f = 1;  // virtual rows per row
    while (a.feats / f > 2048 || a.feats % (8 * f) != 0)
        if (++f > 8) return p;
    StacrSaveArgs av = a;
    av.feats = a.feats / f;
    av.rows = a.rows * f;
    av.chunk_rows = a.chunk_rows * f;
    av.rank = a.rank < 8 ? a.rank : 8;
    Plan pv = make_plan_rows(av);
    if (!pv.fast) return p;
    pv.Rq = p.R <= 8 ? 8 : 16;  // (ranks below 8 padded to 8: one kernel shape fewer)
    pv.mvw = mv;
    pv.ntw = nt;
    SaveGeom &gw = pv.gw;
    gw.rows = a.rows;
    gw.d = a.feats;
    gw.rank = a.rank;
    gw.L = nt;
    gw.log2L = ilog2(nt);
    gw.rpi = 1;
    gw.mv = mv;
    gw.chunk_rows = a.mode == STACR_MODE_GLOBAL_TOPK || a.k_total == 0 ? a.rows : min(a.chunk_rows, a.rows);
    if (gw.chunk_rows < 1) gw.chunk_rows = 1;
    gw.n_chunks = (a.rows + gw.chunk_rows - 1) / gw.chunk_rows;
    int64_t rpw = 64 / pv.Rq;  // one batch of rows per workgroup
    if (a.mode != STACR_MODE_GLOBAL_TOPK && a.k_total > 0)
        while (rpw > 1 && gw.chunk_rows % rpw) rpw >>= 1;
    gw.rows_per_wg = rpw;
    gw.wgs_per_chunk = (gw.chunk_rows + rpw - 1) / rpw;
    gw.hcopies = pv.g.hcopies;  // the later passes sum the copies the projection pass fills
    pv.n_wgs_w = gw.n_chunks * gw.wgs_per_chunk;
    pv.wide = gw.n_chunks == pv.g.n_chunks;
    return pv.wide ? pv : p;
}

// The candidate passes take bf16 saves on the batched path (not wide rows) when a workgroup's
// quota, four times its mean share of its chunk's k plus 64, fits half the candidate list: a
// workgroup then needs more than four times its share above the chunk's level-0 bin before it
// falls back to recomputing.
Plan make_plan_base(const StacrSaveArgs &a)
{
    Plan p = make_plan_wide(a);
    if (!p.fold || a.k_total <= 0) return p;
    p.cand_rin = true;  // (unless the projection pass keeps lists itself, below)
    if (p.wide) return p;
    const SaveGeom &g = p.g;
    const double wg_elems = (double)g.rows_per_wg * (double)g.d;
    const int64_t last_rows = g.rows - (g.n_chunks - 1) * g.chunk_rows;
    const double dens = hmax<double>((double)a.k_full / ((double)g.chunk_rows * (double)g.d),
                                     (double)a.k_last / ((double)last_rows * (double)g.d));
    const double quota = 4.0 * dens * wg_elems + 64.0;
    if (quota > kCandCap / 2) return p;
    p.cand = true;
    p.cand_rin = false;
    p.quota = (uint32_t)quota;
    return p;
}

// With y_out asked for y_cols > rank basis columns, the plan is made for a rank of y_cols and kept
// only if it takes the wide projection pass (the one that writes Y), with the coefficients and the
// residual then formed from the first `rank` columns; otherwise the plan is the rank's own.
Plan make_plan(const StacrSaveArgs &a)
{
    if (a.y_out && a.y_cols > a.rank) {
        StacrSaveArgs ay = a;
        ay.rank = a.y_cols;
        Plan p = make_plan_base(ay);
        if (p.wide) {
            p.gw.rank = a.rank;
            p.g.rank = a.rank < 8 ? a.rank : 8;
            p.yc = a.y_cols;
            return p;
        }
    }
    Plan p = make_plan_base(a);
    p.yc = a.rank;
    return p;
}

template <typename T> T *carve(char *base, size_t off) { return reinterpret_cast<T *>(base + off); }

enum { WS_QP, WS_HIST, WS_COARSE, WS_STATE, WS_MAXKEY, WS_COUNTS, WS_OFFS, WS_LRBITS, WS_LIDX, WS_THIST, WS_TSTATE,
       WS_LCOUNTS, WS_LOFFS, WS_Q4, WS_FOLD, WS_R, WS_CIDX, WS_CVAL, WS_CMETA, WS_N };

size_t layout(const StacrSaveArgs &a, const Plan &p, size_t *off)
{
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    // padded basis, then transposed; then transposed in the activation dtype (16-bit types)
    take(WS_QP, 2 * (size_t)a.feats * p.Rq * sizeof(float) + (size_t)a.feats * p.Rq * 2);
    take(WS_HIST, (size_t)p.g.n_chunks * 3 * p.g.hcopies * kBins * sizeof(uint32_t));
    take(WS_COARSE, (size_t)p.g.n_chunks * p.g.hcopies * kCoarse * sizeof(uint32_t));
    take(WS_MAXKEY, (size_t)p.g.hcopies * kMaxKeyStride * sizeof(uint32_t));
    take(WS_STATE, (size_t)p.g.n_chunks * 3 * sizeof(SelState));
    take(WS_COUNTS, (size_t)p.n_wgs * sizeof(WgCount));
    take(WS_OFFS, (size_t)p.n_wgs * sizeof(WgOffset));
    const size_t nl = p.trim ? (size_t)a.k_sum : 0, nb = p.trim ? (size_t)p.n_list_blocks : 0;
    take(WS_LRBITS, nl * sizeof(uint32_t));
    take(WS_LIDX, nl * sizeof(uint32_t));
    take(WS_THIST, p.trim ? 3 * kBins * sizeof(uint32_t) : 0);
    take(WS_TSTATE, p.trim ? 3 * sizeof(SelState) : 0);
    take(WS_LCOUNTS, nb * sizeof(WgCount));
    take(WS_LOFFS, nb * sizeof(WgOffset));
    take(WS_Q4, a.bits == 4 ? (size_t)a.k_total : 0);
    take(WS_FOLD, p.fold ? (size_t)17 * p.n_wgs * sizeof(uint32_t) : 0);  // cum[0..16][workgroup]
    const bool rstore = p.fast && a.dtype != STACR_DTYPE_F32 && a.k_total > 0 && !p.cand;  // (wide rows: p.fast)
    take(WS_R, rstore ? (size_t)a.rows * a.feats * 2 : 0);  // the stored residual (16-bit types)
    const bool lists = p.cand || p.cand_rin;
    const size_t nc = lists ? (size_t)p.n_wgs * kCandCap : 0;  // the candidate lists
    take(WS_CIDX, nc * sizeof(uint32_t));
    take(WS_CVAL, nc * sizeof(uint16_t));
    take(WS_CMETA, lists ? (size_t)p.n_wgs * sizeof(CandMeta) : 0);
    return cur;
}

// The wide projection pass for the plan's (rank, vectors a thread, threads a row).
template <int DT>
int launch_wide_pass1(const StacrSaveArgs &a, const Plan &p, const typename Act<DT>::T *x, const float *qp,
                      typename Act<DT>::T *coeff, uint32_t *hist, uint32_t *maxkey, int do_hist,
                      const typename Act<DT>::T *coeff_in, typename Act<DT>::T *rout, uint32_t *coarse)
{
    // the optional projection outputs (Y only where the pass projects: not on given coefficients)
    float *y_out = a.y_out && !coeff_in ? a.y_out : nullptr;
    float *epart = DT == STACR_DTYPE_BF16 ? a.energy_part : nullptr;
    hipStream_t s = a.stream;
    const unsigned n = (unsigned)p.n_wgs_w;
    const void *cp = coeff_in ? (const void *)coeff_in : (const void *)coeff;
    const int c_vec = a.rank == p.Rq && ((uintptr_t)cp % 16) == 0;
    bool done = false;
    auto go = [&](auto r, auto mv, auto nt) {
        constexpr int R = decltype(r)::value, MV = decltype(mv)::value, NT = decltype(nt)::value;
        if (done || p.Rq != R || p.mvw != MV || p.ntw != NT) return;
        done = true;
        stacr_launch("k_proj_hist_w", s, [&] {
            k_proj_hist_w<DT, R, MV, NT><<<n, NT, 0, s>>>(p.gw, c_vec, x, qp, coeff, hist, maxkey, do_hist, coeff_in, rout, coarse,
                                                          y_out, p.yc, epart);
        });
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using N256 = std::integral_constant<int, 256>;
    using N512 = std::integral_constant<int, 512>;
    go(std::integral_constant<int, 8>{}, I2{}, N256{});
    go(std::integral_constant<int, 8>{}, I2{}, N512{});
    go(std::integral_constant<int, 16>{}, I1{}, N256{});
    go(std::integral_constant<int, 16>{}, I1{}, N512{});
    if constexpr (DT == STACR_DTYPE_BF16) go(std::integral_constant<int, 16>{}, I2{}, N512{});
    if (!done)
        return stacr_fail(STACR_ERR_INVALID, "stacr_save: no wide projection kernel for rank %d, %d x %d", p.Rq, p.mvw, p.ntw);
    if (y_out && a.y_written) *a.y_written = 1;
    if (epart && a.energy_written) *a.energy_written = 1;
    return STACR_OK;
}

template <int DT, int R, int V, bool QREG>
int launch_typed(const StacrSaveArgs &a, const Plan &p, char *ws, const size_t *off)
{
    using T = typename Act<DT>::T;
    hipStream_t s = a.stream;
    const T *x = static_cast<const T *>(a.x);
    T *coeff_out = static_cast<T *>(a.coeff);
    const T *coeff_in = static_cast<const T *>(a.coeff_in);
    const T *coeff = coeff_in ? coeff_in : coeff_out;
    float *qp = carve<float>(ws, off[WS_QP]);
    uint32_t *hist = carve<uint32_t>(ws, off[WS_HIST]);
    uint32_t *maxkey = carve<uint32_t>(ws, off[WS_MAXKEY]);
    SelState *state = carve<SelState>(ws, off[WS_STATE]);
    WgCount *counts = carve<WgCount>(ws, off[WS_COUNTS]);
    const bool resid = a.k_total > 0;
    const int nwg = (int)p.n_wgs;

    // padded basis; histograms and max key (contiguous in the layout) cleared in the same launch
    const int64_t n_zero = resid ? (int64_t)((off[WS_MAXKEY] + (size_t)p.g.hcopies * kMaxKeyStride * sizeof(uint32_t) -
                                              off[WS_HIST]) / sizeof(uint32_t)) : 0;
    // the entry census (bf16 candidate passes without a trim, blocks of whole workgroups): its
    // counts are cleared here and filled by the emission pass.  Lists from X: rows of <= 2048
    // features; lists from the stored residual: also rows split into segments (<= 4096 features)
    const int64_t csegs = p.g.d > 0 && a.feats % p.g.d == 0 ? a.feats / p.g.d : 0;
    const bool census = a.census && (p.cand || p.cand_rin) && !p.trim && csegs >= 1 &&
                        (kCensusRows * csegs) % p.g.rows_per_wg == 0 && p.g.rows % csegs == 0 &&
                        (csegs == 1 ? a.feats <= kBins : p.cand_rin && !p.cand && a.feats <= 2 * kBins);
    const int64_t n_census = census ? (int64_t)kCensusCopies * a.feats : 0;
    stacr_launch("k_prep", s, [&] {
        k_prep<DT><<<grid_for(hmax<int64_t>(hmax<int64_t>(a.feats * p.Rq, n_zero), n_census)), kBlock, 0, s>>>(
            static_cast<const T *>(a.q), a.feats, p.yc, a.q_ld > 0 ? a.q_ld : a.rank, p.Rq, qp, hist, n_zero,
            census ? a.census : nullptr, n_census);
    });
    // batched fast path: one aligned vector per thread per row, basis columns in registers
    constexpr bool kFastOk = QREG && V == Act<DT>::kVec && V * R <= 64;
    const bool fast = kFastOk && p.fast;
    const bool hc8 = p.g.hcopies == kHistCopies;
    uint32_t *fold = carve<uint32_t>(ws, off[WS_FOLD]);
    uint32_t *coarse = carve<uint32_t>(ws, off[WS_COARSE]);
    // 16-bit activations on the batched path: the projection pass stores the residual (exact in
    // the activation dtype) and the later passes read it instead of X, C and the basis
    constexpr bool kRin = sizeof(T) == 2;
    T *rbuf = carve<T>(ws, off[WS_R]);
    const T *xin = kRin ? rbuf : x;
    if (fast != p.fold && DT == STACR_DTYPE_BF16) return stacr_fail(STACR_ERR_INVALID, "stacr_save: bf16 fold outside the batched path");
    if (!fast && p.g.hcopies != 1) return stacr_fail(STACR_ERR_INVALID, "stacr_save: histogram copies outside the batched path");
    FastGeom fg{p.g.L / 64, a.rank == R && ((uintptr_t)coeff % 16) == 0};
    // bf16 candidate passes (the plan takes them only with a residual, so the projection pass
    // always runs them)
    constexpr bool kCandOk = kFastOk && DT == STACR_DTYPE_BF16;
    const bool cand = kCandOk && fast && p.cand && resid;
    const bool cand_rin = kCandOk && fast && p.cand_rin && resid;
    if ((p.cand && !cand) || (p.cand_rin && !cand_rin))
        return stacr_fail(STACR_ERR_INVALID, "stacr_save: candidate passes outside the bf16 batched path");
    uint32_t *cidx = carve<uint32_t>(ws, off[WS_CIDX]);
    uint16_t *cval = carve<uint16_t>(ws, off[WS_CVAL]);
    CandMeta *cmeta = carve<CandMeta>(ws, off[WS_CMETA]);
    if (!coeff_in || resid) {
        if constexpr (kFastOk) {
            if (fast && p.wide) {
                if constexpr (kRin) {
                    const int rc = launch_wide_pass1<DT>(a, p, x, qp, coeff_out, hist, maxkey, resid ? 1 : 0, coeff_in, rbuf, coarse);
                    if (rc) return rc;
                } else {
                    return stacr_fail(STACR_ERR_INVALID, "stacr_save: wide rows outside 16-bit activations");
                }
            } else if (fast && cand) {
                if constexpr (kCandOk)
                    stacr_launch("k_proj_cand", s, [&] { k_proj_cand<R><<<nwg, kBlock, 0, s>>>(p.g, fg, x, qp, coeff_out, hist, maxkey, coeff_in, coarse, p.quota, cidx, cval, cmeta); });
            } else if (fast) {
                stacr_launch("k_proj_hist_b", s, [&] { k_proj_hist_b<DT, R, V, kRin><<<nwg, kBlock, 0, s>>>(p.g, fg, x, qp, coeff_out, hist, maxkey, resid ? 1 : 0, coeff_in, rbuf, coarse); });
            }
        }
        if (!fast)
            stacr_launch("k_proj_hist", s, [&] { k_proj_hist<DT, R, V, QREG><<<nwg, kBlock, 0, s>>>(p.g, x, qp, coeff_out, hist, maxkey, resid ? 1 : 0, coeff_in); });
    }
    if (!resid) return stacr_hip_check(hipGetLastError(), "save kernels");

    const uint32_t kf = (uint32_t)a.k_full, kl = (uint32_t)a.k_last;
    // Each pass first finds the previous radix level's bin for its chunk (every workgroup from the
    // completed histogram; the chunk's first workgroup records it), so no selection launches.
    // (the batched count pass makes the last selection of 16-bit types itself)
    const int n_refine = fast && sizeof(T) == 2 ? 1 : 2;
    for (int lvl = 1; lvl <= n_refine; ++lvl) {
        if constexpr (kFastOk) {
            if (fast) {
                auto refine = [&](auto hc, auto level) {
                    stacr_launch("k_refine_hist_b", s, [&] {
                        k_refine_hist_b<DT, R, V, decltype(hc)::value, kRin, decltype(level)::value><<<nwg, kBlock, 0, s>>>(
                            p.g, fg, xin, qp, coeff, hist, state, kf, kl, maxkey, fold, p.n_wgs, coarse);
                    });
                };
                using L1 = std::integral_constant<int, 1>;
                using L2 = std::integral_constant<int, 2>;
                using H8 = std::integral_constant<int, kHistCopies>;
                using H1 = std::integral_constant<int, 1>;
                auto refine_cand = [&](auto hc) {
                    if constexpr (kCandOk)
                        stacr_launch("k_refine_cand", s, [&] {
                            k_refine_cand<R, decltype(hc)::value><<<nwg, kBlock, 0, s>>>(
                                p.g, fg, x, qp, coeff, hist, state, kf, kl, maxkey, fold, p.n_wgs, coarse, cval, cmeta);
                        });
                };
                auto refine_lists = [&](auto hc) {
                    if constexpr (kCandOk && kRin)
                        stacr_launch("k_refine_hist_b", s, [&] {
                            k_refine_hist_b<DT, R, V, decltype(hc)::value, true, 1, true><<<nwg, kBlock, 0, s>>>(
                                p.g, fg, xin, qp, coeff, hist, state, kf, kl, maxkey, fold, p.n_wgs, coarse, cidx, cval,
                                cmeta);
                        });
                };
                if (lvl == 1 && cand) {
                    if (hc8) refine_cand(H8{});
                    else refine_cand(H1{});
                } else if (lvl == 1 && cand_rin) {
                    if (hc8) refine_lists(H8{});
                    else refine_lists(H1{});
                } else if (lvl == 1) {
                    if (hc8) refine(H8{}, L1{});
                    else refine(H1{}, L1{});
                } else if constexpr (sizeof(T) == 4) {  // only fp32 runs the second refine pass
                    if (hc8) refine(H8{}, L2{});
                    else refine(H1{}, L2{});
                }
            }
        }
        if (!fast) stacr_launch("k_refine_hist", s, [&] { k_refine_hist<DT, R, V, QREG><<<nwg, kBlock, 0, s>>>(p.g, lvl, x, qp, coeff, hist, state, kf, kl); });
    }
    if constexpr (kFastOk) {
        if (fast && hc8 && !p.fold)
            stacr_launch("k_count_b", s, [&] { k_count_b<DT, R, V, kHistCopies, kRin><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, hist, state, counts, kf, kl); });
        if (fast && !hc8 && !p.fold)
            stacr_launch("k_count_b", s, [&] { k_count_b<DT, R, V, 1, kRin><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, hist, state, counts, kf, kl); });
    }
    if (!fast) stacr_launch("k_count", s, [&] { k_count<DT, R, V, QREG><<<nwg, kBlock, 0, s>>>(p.g, x, qp, coeff, hist, state, counts, kf, kl); });

    OutSpec o{};
    o.idx = a.idx;
    o.idx_bytes = a.index_bytes;
    o.bits = a.bits;
    o.data = a.bits == 4 ? (void *)carve<int8_t>(ws, off[WS_Q4]) : a.data;
    uint32_t *lrb = carve<uint32_t>(ws, off[WS_LRBITS]);
    uint32_t *lix = carve<uint32_t>(ws, off[WS_LIDX]);
    o.list_rbits = lrb;
    o.list_idx = lix;
    o.cap = (uint32_t)(p.trim ? a.k_sum : a.k_total);
    if constexpr (kFastOk) {
        // the fold variant (bf16) reads the level-1 histogram copies; other types take the counts
        if constexpr (kCandOk) {
            uint32_t *cen = census ? a.census : nullptr;
            const uint32_t kt = (uint32_t)a.k_sum;  // the entries emitted (no trim: the chunks' k summed)
            if (cand && hc8)
                stacr_launch("k_emit_cand", s, [&] { k_emit_cand<R, kHistCopies><<<nwg, kBlock, 0, s>>>(p.g, fg, x, qp, coeff, state, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs, cidx, cval, cmeta, cen, kt, (uint32_t)a.feats); });
            else if (cand)
                stacr_launch("k_emit_cand", s, [&] { k_emit_cand<R, 1><<<nwg, kBlock, 0, s>>>(p.g, fg, x, qp, coeff, state, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs, cidx, cval, cmeta, cen, kt, (uint32_t)a.feats); });
            if constexpr (kRin) {  // the lists of the level-1 pass; the fallback reads the stored residual
                if (cand_rin && hc8)
                    stacr_launch("k_emit_cand", s, [&] { k_emit_cand<R, kHistCopies, true><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, state, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs, cidx, cval, cmeta, cen, kt, (uint32_t)a.feats); });
                else if (cand_rin)
                    stacr_launch("k_emit_cand", s, [&] { k_emit_cand<R, 1, true><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, state, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs, cidx, cval, cmeta, cen, kt, (uint32_t)a.feats); });
            }
            // (written only by an emission that ran: candidate lists from X, or from the stored
            // residual where this type and rank build that pass)
            if (census && a.census_written && (cand || (kRin && cand_rin))) *a.census_written = 1;
        }
        if (!cand && !cand_rin && fast && hc8 && DT == STACR_DTYPE_BF16)
            stacr_launch("k_emit_b", s, [&] { k_emit_b<DT, R, V, kHistCopies, kRin><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, state, counts, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs); });
        else if (!cand && !cand_rin && fast)
            stacr_launch("k_emit_b", s, [&] { k_emit_b<DT, R, V, 1, kRin><<<nwg, kBlock, 0, s>>>(p.g, fg, xin, qp, coeff, state, counts, kf, maxkey, o, a.scale, p.trim ? 1 : 0, hist, fold, p.n_wgs); });
    }
    if (!fast) stacr_launch("k_emit", s, [&] { k_emit<DT, R, V, QREG><<<nwg, kBlock, 0, s>>>(p.g, x, qp, coeff, state, counts, kf, maxkey, o, a.scale, p.trim ? 1 : 0); });

    if (p.trim) {
        uint32_t *thist = carve<uint32_t>(ws, off[WS_THIST]);
        SelState *tstate = carve<SelState>(ws, off[WS_TSTATE]);
        WgCount *lcounts = carve<WgCount>(ws, off[WS_LCOUNTS]);
        WgOffset *loffs = carve<WgOffset>(ws, off[WS_LOFFS]);
        const int nlb = (int)p.n_list_blocks;
        const uint32_t kt = (uint32_t)a.k_total;
        stacr_launch("k_zero_u32", s, [&] { k_zero_u32<<<grid_for(3 * kBins), kBlock, 0, s>>>(thist, 3 * kBins); });
        for (int lvl = 0; lvl < 3; ++lvl) {
            stacr_launch("k_list_hist", s, [&] { k_list_hist<<<nlb, kBlock, 0, s>>>(lvl, lrb, a.k_sum, thist, tstate); });
            stacr_launch("k_select_step", s, [&] { k_select_step<<<1, kBlock, 0, s>>>(lvl, thist, tstate, 1, kt, kt); });
        }
        stacr_launch("k_list_count", s, [&] { k_list_count<<<nlb, kBlock, 0, s>>>(lrb, a.k_sum, tstate, lcounts); });
        stacr_launch("k_offsets", s, [&] { k_offsets<<<1, kBlock, 0, s>>>(lcounts, loffs, tstate, p.n_list_blocks, kt); });
        o.cap = (uint32_t)a.k_total;
        stacr_launch("k_list_emit", s, [&] { k_list_emit<DT><<<nlb, kBlock, 0, s>>>(lrb, lix, a.k_sum, tstate, loffs, maxkey, o, a.scale); });
    }
    if (a.bits == 4)
        stacr_launch("k_pack_int4", s, [&] { k_pack_int4<<<grid_for((a.k_total + 1) / 2), kBlock, 0, s>>>(carve<int8_t>(ws, off[WS_Q4]), a.k_total,
                                                                   static_cast<uint8_t *>(a.data)); });
    return stacr_hip_check(hipGetLastError(), "save kernels");
}

template <int DT, int R>
int dispatch_vq(const StacrSaveArgs &a, const Plan &p, char *ws, const size_t *off)
{
    constexpr int VEC = Act<DT>::kVec;
    if (p.V == VEC) {
        if (p.qreg) return launch_typed<DT, R, VEC, true>(a, p, ws, off);
        return launch_typed<DT, R, VEC, false>(a, p, ws, off);
    }
    if (p.qreg) return launch_typed<DT, R, 1, true>(a, p, ws, off);
    return launch_typed<DT, R, 1, false>(a, p, ws, off);
}

template <int DT>
int dispatch_r(const StacrSaveArgs &a, const Plan &p, char *ws, const size_t *off)
{
    switch (p.R) {
    case 4: return dispatch_vq<DT, 4>(a, p, ws, off);
    case 8: return dispatch_vq<DT, 8>(a, p, ws, off);
    case 16: return dispatch_vq<DT, 16>(a, p, ws, off);
    default: return dispatch_vq<DT, 32>(a, p, ws, off);
    }
}

}  // namespace

size_t stacr_save_ws_layout(const StacrSaveArgs &a, size_t *offsets)
{
    const Plan p = make_plan(a);
    size_t tmp[WS_N];
    return layout(a, p, offsets ? offsets : tmp);
}

int64_t stacr_save_energy_slots(const StacrSaveArgs &a)
{
    const Plan p = make_plan(a);
    return p.wide && a.dtype == STACR_DTYPE_BF16 ? p.n_wgs_w : 0;
}

int stacr_save_launch(const StacrSaveArgs &a)
{
    const Plan p = make_plan(a);
    size_t off[WS_N];
    const size_t need = layout(a, p, off);
    if (a.workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_save: workspace has %zu bytes, needs %zu", a.workspace_bytes, need);
    if (p.n_wgs > INT32_MAX || p.n_wgs_w > INT32_MAX)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_save: too many workgroups");
    char *ws = static_cast<char *>(a.workspace);
    switch (a.dtype) {
    case STACR_DTYPE_F32: return dispatch_r<STACR_DTYPE_F32>(a, p, ws, off);
    case STACR_DTYPE_BF16: return dispatch_r<STACR_DTYPE_BF16>(a, p, ws, off);
    default: return dispatch_r<STACR_DTYPE_F16>(a, p, ws, off);
    }
}

template <int DT>
static int quantize_typed(const void *v, int64_t n, int bits, void *data, float *scale, uint32_t *maxkey, hipStream_t s)
{
    using T = typename Act<DT>::T;
    stacr_launch("k_zero_u32", s, [&] { k_zero_u32<<<1, kBlock, 0, s>>>(maxkey, 1); });
    stacr_launch("k_absmax", s, [&] { k_absmax<DT><<<grid_for(n), kBlock, 0, s>>>(static_cast<const T *>(v), n, maxkey); });
    stacr_launch("k_quantize", s, [&] { k_quantize<DT><<<grid_for(bits == 4 ? (n + 1) / 2 : n), kBlock, 0, s>>>(static_cast<const T *>(v), n, bits, maxkey,
                                                                          data, scale); });
    return stacr_hip_check(hipGetLastError(), "quantize kernels");
}

int stacr_quantize_launch(const void *v, int dtype, int64_t n, int bits, void *data, float *scale, void *workspace,
                          hipStream_t s)
{
    uint32_t *maxkey = static_cast<uint32_t *>(workspace);
    switch (dtype) {
    case STACR_DTYPE_F32: return quantize_typed<STACR_DTYPE_F32>(v, n, bits, data, scale, maxkey, s);
    case STACR_DTYPE_BF16: return quantize_typed<STACR_DTYPE_BF16>(v, n, bits, data, scale, maxkey, s);
    default: return quantize_typed<STACR_DTYPE_F16>(v, n, bits, data, scale, maxkey, s);
    }
}
