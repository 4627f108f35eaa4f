// The projection engine's other residual selectors (stacr/layers.py:44-101):
//   uniform       k evenly spaced flat positions floor(i * total / k), i = 0..k-1 (:89-98)
//   block_sparse  per chunk, the count = max(1, round(b * blocks)) blocks of `bs` consecutive
//                 elements with the largest energy sum(r^2) in the activation dtype (:81-88)
//   sampled       |r| >= quantile of a seeded sample, first k_total in flat order (:55-66);
//                 the sample positions and the quantile are torch library calls on the host side,
//                 the gather of the sampled magnitudes and the ordered compaction run here.
// and the adaptive engine's block_sparse (stacr/adaptive.py:1788-1938): blocks of `bs` columns of
// one row (the last block of a row padded with zeros), per chunk of rows the top
// ceil(k_blocks * chunk / rows) blocks by energy, then the top k_blocks of all those candidates.
// Every residual is the dtype-native r = rnd(x - rnd(sum_j c_j q_j)) of the save kernels.
// Output indices ascend.  Block ties take the lowest block index (the reference's torch.topk
// leaves that choice unspecified).
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kSegThreads = 1024;  // block_sparse: one workgroup per chunk
constexpr int kThrPer = 16;        // sampled: elements per thread per workgroup tile
constexpr int kThrTile = kBlock * kThrPer;

template <int DT>
__device__ __forceinline__ float resid_at(const typename Act<DT>::T *__restrict__ x,
                                          const typename Act<DT>::T *__restrict__ coeff,
                                          const typename Act<DT>::T *__restrict__ q, int64_t d, int rank,
                                          int64_t row, int64_t col)
{
    using A = Act<DT>;
    float p = 0.f;
    for (int j = 0; j < rank; ++j) p = fmaf(A::ld(coeff[row * rank + j]), A::ld(q[col * rank + j]), p);
    return A::rnd(A::ld(x[row * d + col]) - A::rnd(p));
}

__device__ __forceinline__ void put_index(void *idx, int bytes, int64_t i, int64_t v)
{
    if (bytes == 8) static_cast<int64_t *>(idx)[i] = v;
    else if (bytes == 4) static_cast<int32_t *>(idx)[i] = (int32_t)v;
    else static_cast<int16_t *>(idx)[i] = (int16_t)v;
}

// ------------------------------------------------------------------ uniform
template <int DT>
__global__ __launch_bounds__(kBlock) void k_uniform(const typename Act<DT>::T *__restrict__ x,
                                                    const typename Act<DT>::T *__restrict__ coeff,
                                                    const typename Act<DT>::T *__restrict__ q, int64_t d, int rank,
                                                    uint64_t total, int64_t k, void *idx, int idx_bytes,
                                                    typename Act<DT>::T *__restrict__ values)
{
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= k) return;
    const int64_t pos = (int64_t)((uint64_t)i * total / (uint64_t)k);  // i, total < 2^32: no overflow
    const int64_t row = pos / d, col = pos - row * d;
    put_index(idx, idx_bytes, i, pos);
    values[i] = Act<DT>::st(resid_at<DT>(x, coeff, q, d, rank, row, col));
}

// ------------------------------------------------------------------ block_sparse
// Key of block b: fp32 bits of rnd(sum_o rnd(r_o^2)) (energy >= 0; NaN sorts above +inf).  Block b
// covers columns [(b % bpr) * bs, + bs) of row b / bpr, bpr = ceil(d / bs); columns past d are the
// zero padding and add nothing.  (With d % bs == 0 the blocks are consecutive flat elements.)
__device__ __forceinline__ int64_t block_width(int64_t b, int64_t bpr, int64_t bs, int64_t d)
{
    const int64_t col0 = (b % bpr) * bs;
    return d - col0 < bs ? d - col0 : bs;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_block_keys(const typename Act<DT>::T *__restrict__ x,
                                                       const typename Act<DT>::T *__restrict__ coeff,
                                                       const typename Act<DT>::T *__restrict__ q, int64_t d,
                                                       int rank, int64_t bs, int64_t bpr, int64_t n_blocks,
                                                       uint32_t *__restrict__ keys)
{
    const int64_t b = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (b >= n_blocks) return;
    const int64_t row = b / bpr, col0 = (b - row * bpr) * bs;
    const int64_t width = block_width(b, bpr, bs, d);
    float e = 0.f;
    for (int64_t o = 0; o < width; ++o) {
        const float r = resid_at<DT>(x, coeff, q, d, rank, row, col0 + o);
        e += Act<DT>::rnd(r * r);
    }
    keys[b] = __float_as_uint(Act<DT>::rnd(e)) & 0x7fffffffu;
}

// Per chunk (one workgroup): exact top-`count` keys by a three-digit radix select, ties to the
// lowest block, then the chosen block ids in ascending order to sel[chunk * count_full + ...].
__global__ __launch_bounds__(kSegThreads) void k_block_select(const uint32_t *__restrict__ keys, int64_t n_blocks,
                                                              int64_t seg_blocks, int64_t count_full,
                                                              int64_t count_last, uint32_t *__restrict__ sel)
{
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_tot[kSegThreads / 64];
    __shared__ uint32_t s_pick[2];
    const int tid = threadIdx.x;
    const int64_t seg = blockIdx.x;
    const int64_t base = seg * seg_blocks;
    const int64_t n = (base + seg_blocks <= n_blocks) ? seg_blocks : n_blocks - base;
    const bool last = base + seg_blocks >= n_blocks;
    const uint32_t count = (uint32_t)(last ? count_last : count_full);
    uint32_t prefix = 0, mask = 0, need = count;
    if (tid == 0) { s_pick[0] = 0; s_pick[1] = count; }
    for (int lvl = 0; lvl < 3; ++lvl) {
        const int shift = kDigitShift[lvl], bins = kDigitBins[lvl];
        for (int i = tid; i < bins; i += kSegThreads) s_hist[i] = 0;
        __syncthreads();
        for (int64_t i = tid; i < n; i += kSegThreads) {
            const uint32_t key = keys[base + i];
            if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & (uint32_t)(bins - 1)], 1u);
        }
        __syncthreads();
        // thread t owns the bins_per bins just below bins - t * bins_per (descending key order)
        const int bins_per = bins / kSegThreads > 0 ? bins / kSegThreads : 1;
        const int top = bins - 1 - tid * bins_per;
        uint32_t mine = 0;
        if (top >= 0)
            for (int u = 0; u < bins_per; ++u) mine += s_hist[top - u];
        uint32_t all;
        uint32_t above = block_exclusive_scan<kSegThreads>(mine, s_tot, &all);
        if (top >= 0 && above < need && need <= above + mine) {
            for (int u = 0; u < bins_per; ++u) {
                const uint32_t h = s_hist[top - u];
                if (above + h >= need) {
                    s_pick[0] = prefix | ((uint32_t)(top - u) << shift);
                    s_pick[1] = need - above;
                    break;
                }
                above += h;
            }
        }
        __syncthreads();
        prefix = s_pick[0];
        need = s_pick[1];
        mask |= (uint32_t)(bins - 1) << shift;
        __syncthreads();
    }
    // ordered compaction: keys above the threshold, plus the first `need` equal to it
    uint32_t out = 0, ties = 0;
    uint32_t *dst = sel + seg * count_full;
    for (int64_t t0 = 0; t0 < n; t0 += kSegThreads) {
        const int64_t i = t0 + tid;
        const uint32_t key = i < n ? keys[base + i] : 0u;
        const bool gt = i < n && key > prefix;
        const bool eq = i < n && key == prefix;
        uint32_t n_eq, n_keep;
        const uint32_t eq_rank = ties + block_exclusive_scan<kSegThreads>(eq ? 1u : 0u, s_tot, &n_eq);
        const bool keep = gt || (eq && eq_rank < need);
        const uint32_t pos = out + block_exclusive_scan<kSegThreads>(keep ? 1u : 0u, s_tot, &n_keep);
        if (keep && pos < count) dst[pos] = (uint32_t)(base + i);
        ties += n_eq;
        out += n_keep;
    }
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_block_emit(const typename Act<DT>::T *__restrict__ x,
                                                       const typename Act<DT>::T *__restrict__ coeff,
                                                       const typename Act<DT>::T *__restrict__ q, int64_t d,
                                                       int rank, int64_t bs, int64_t n_blocks,
                                                       const uint32_t *__restrict__ sel, int64_t n_out, void *idx,
                                                       int idx_bytes, typename Act<DT>::T *__restrict__ values)
{
    const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (e >= n_out) return;
    const int64_t b = sel[e / bs];
    const int64_t blk = b < n_blocks ? b : n_blocks - 1;  // reads stay inside X whatever sel holds
    const int64_t pos = blk * bs + e % bs;
    const int64_t row = pos / d, col = pos - row * d;
    put_index(idx, idx_bytes, e, pos);
    values[e] = Act<DT>::st(resid_at<DT>(x, coeff, q, d, rank, row, col));
}

// Keys of the candidate blocks, in candidate order (ascending block ids), for the global trim.
__global__ __launch_bounds__(kBlock) void k_block_gather_keys(const uint32_t *__restrict__ keys,
                                                              const uint32_t *__restrict__ cand, int64_t n_cand,
                                                              uint32_t *__restrict__ ckeys)
{
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n_cand) ckeys[i] = keys[cand[i]];
}

// One workgroup: the final block list (candidates, or the candidates at the trim's positions),
// each block's first output slot (exclusive scan of the block widths) and the entry count.
__global__ __launch_bounds__(kSegThreads) void k_block_offsets(const uint32_t *__restrict__ cand,
                                                               const uint32_t *__restrict__ pick, int64_t n_final,
                                                               int64_t bpr, int64_t bs, int64_t d,
                                                               uint32_t *__restrict__ final_blocks,
                                                               int64_t *__restrict__ offsets,
                                                               int64_t *__restrict__ count)
{
    __shared__ uint32_t s_tot[kSegThreads / 64];
    int64_t run = 0;
    for (int64_t t0 = 0; t0 < n_final; t0 += kSegThreads) {
        const int64_t i = t0 + threadIdx.x;
        uint32_t width = 0;
        if (i < n_final) {
            const uint32_t b = pick ? cand[pick[i]] : cand[i];
            final_blocks[i] = b;
            width = (uint32_t)block_width(b, bpr, bs, d);
        }
        uint32_t all;
        const uint32_t before = block_exclusive_scan<kSegThreads>(width, s_tot, &all);
        if (i < n_final) offsets[i] = run + before;
        run += all;
    }
    if (threadIdx.x == 0) *count = run;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_block_emit_rows(const typename Act<DT>::T *__restrict__ x,
                                                            const typename Act<DT>::T *__restrict__ coeff,
                                                            const typename Act<DT>::T *__restrict__ q, int64_t d,
                                                            int rank, int64_t bs, int64_t bpr, int64_t n_blocks,
                                                            const uint32_t *__restrict__ final_blocks,
                                                            const int64_t *__restrict__ offsets, int64_t n_final,
                                                            void *idx, int idx_bytes,
                                                            typename Act<DT>::T *__restrict__ values)
{
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t i = t / bs, o = t - (t / bs) * bs;
    if (i >= n_final) return;
    const int64_t b0 = final_blocks[i];
    const int64_t b = b0 < n_blocks ? b0 : n_blocks - 1;  // reads stay inside X whatever the list holds
    if (o >= block_width(b, bpr, bs, d)) return;  // zero padding past the row's end is not stored
    const int64_t row = b / bpr, col = (b - row * bpr) * bs + o;
    const int64_t e = offsets[i] + o;
    put_index(idx, idx_bytes, e, row * d + col);
    values[e] = Act<DT>::st(resid_at<DT>(x, coeff, q, d, rank, row, col));
}

// ------------------------------------------------------------------ sampled
template <int DT>
__global__ __launch_bounds__(kBlock) void k_sample_abs(const typename Act<DT>::T *__restrict__ x,
                                                       const typename Act<DT>::T *__restrict__ coeff,
                                                       const typename Act<DT>::T *__restrict__ q, int64_t d,
                                                       int rank, int64_t total, const int64_t *__restrict__ pos,
                                                       int64_t n, typename Act<DT>::T *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const int64_t p = pos[i];
    if (p < 0 || p >= total) {  // outside X: NaN, which no threshold passes
        out[i] = Act<DT>::st(__builtin_nanf(""));
        return;
    }
    const int64_t row = p / d, col = p - row * d;
    out[i] = Act<DT>::st(fabsf(resid_at<DT>(x, coeff, q, d, rank, row, col)));
}

// |r| >= threshold, compared in the activation dtype: torch promotes the fp32 0-dim quantile to
// the magnitude tensor's dtype for the comparison.  NaN on either side does not pass.
template <int DT>
__device__ __forceinline__ bool passes(float r, float thr_d) { return fabsf(r) >= thr_d; }

template <int DT>
__global__ __launch_bounds__(kBlock) void k_thr_count(const typename Act<DT>::T *__restrict__ x,
                                                      const typename Act<DT>::T *__restrict__ coeff,
                                                      const typename Act<DT>::T *__restrict__ q, int64_t d,
                                                      int rank, int64_t total, const float *__restrict__ thr,
                                                      uint32_t *__restrict__ wg_count)
{
    __shared__ uint32_t s_tot[kWaves];
    const float t = Act<DT>::rnd(*thr);
    const int64_t t0 = (int64_t)blockIdx.x * kThrTile;
    uint32_t c = 0;
    for (int s = 0; s < kThrPer; ++s) {
        const int64_t p = t0 + (int64_t)s * kBlock + threadIdx.x;
        if (p < total) {
            const int64_t row = p / d, col = p - row * d;
            c += passes<DT>(resid_at<DT>(x, coeff, q, d, rank, row, col), t) ? 1u : 0u;
        }
    }
    const uint32_t sum = block_sum(c, s_tot);
    if (threadIdx.x == 0) wg_count[blockIdx.x] = sum;
}

// Exclusive offsets of the per-workgroup counts; count_out = min(cap, passing entries), or every
// passing entry when cap is 0 (a count-only call).
__global__ __launch_bounds__(kSegThreads) void k_thr_offsets(const uint32_t *__restrict__ wg_count, int64_t n_wg,
                                                             int64_t cap, uint32_t *__restrict__ wg_off,
                                                             int64_t *__restrict__ count_out)
{
    __shared__ uint32_t s_tot[kSegThreads / 64];
    uint64_t run = 0;
    for (int64_t b = 0; b < n_wg; b += kSegThreads) {
        const int64_t i = b + threadIdx.x;
        const uint32_t v = i < n_wg ? wg_count[i] : 0u;
        uint32_t tile;
        const uint32_t ex = block_exclusive_scan<kSegThreads>(v, s_tot, &tile);
        if (i < n_wg) wg_off[i] = (uint32_t)(run + ex);  // total < 2^32
        run += tile;
    }
    if (threadIdx.x == 0) *count_out = cap == 0 || (int64_t)run < cap ? (int64_t)run : cap;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_thr_emit(const typename Act<DT>::T *__restrict__ x,
                                                     const typename Act<DT>::T *__restrict__ coeff,
                                                     const typename Act<DT>::T *__restrict__ q, int64_t d, int rank,
                                                     int64_t total, const float *__restrict__ thr,
                                                     const uint32_t *__restrict__ wg_off, int64_t cap, void *idx,
                                                     int idx_bytes, typename Act<DT>::T *__restrict__ values)
{
    __shared__ uint32_t s_tot[kWaves];
    const uint32_t base = wg_off[blockIdx.x];
    if ((int64_t)base >= cap) return;  // uniform per workgroup: the whole tile lies past the cap
    const float t = Act<DT>::rnd(*thr);
    const int64_t t0 = (int64_t)blockIdx.x * kThrTile;
    uint32_t run = base;
    for (int s = 0; s < kThrPer; ++s) {
        const int64_t p = t0 + (int64_t)s * kBlock + threadIdx.x;
        float r = 0.f;
        bool keep = false;
        if (p < total) {
            const int64_t row = p / d, col = p - row * d;
            r = resid_at<DT>(x, coeff, q, d, rank, row, col);
            keep = passes<DT>(r, t);
        }
        uint32_t n_keep;
        const uint32_t pos = run + block_exclusive_scan<kBlock>(keep ? 1u : 0u, s_tot, &n_keep);
        if (keep && (int64_t)pos < cap) {
            put_index(idx, idx_bytes, pos, p);
            values[pos] = Act<DT>::st(r);
        }
        run += n_keep;
    }
}

unsigned blocks_of(int64_t n) { return (unsigned)((n + kBlock - 1) / kBlock); }

template <int DT>
using TP = const typename Act<DT>::T *;

template <int DT>
int uniform_typed(const void *x, const void *coeff, const void *q, int64_t rows, int64_t d, int rank, int64_t k,
                  void *idx, int idx_bytes, void *values, hipStream_t s)
{
    using T = typename Act<DT>::T;
    if (k > 0)
        stacr_launch("k_uniform", s, [&] {
            k_uniform<DT><<<blocks_of(k), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank,
                                                          (uint64_t)(rows * d), k, idx, idx_bytes, (T *)values);
        });
    return stacr_hip_check(hipGetLastError(), "uniform selector");
}

template <int DT>
int block_typed(const void *x, const void *coeff, const void *q, int64_t rows, int64_t d, int rank, int64_t bs,
                int64_t seg_blocks, int64_t n_seg, int64_t count_full, int64_t count_last, void *idx, int idx_bytes,
                void *values, uint32_t *keys, uint32_t *sel, hipStream_t s)
{
    using T = typename Act<DT>::T;
    const int64_t n_blocks = rows * d / bs;
    const int64_t n_out = ((n_seg - 1) * count_full + count_last) * bs;
    stacr_launch("k_block_keys", s, [&] {
        k_block_keys<DT><<<blocks_of(n_blocks), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, bs,
                                                               d / bs, n_blocks, keys);
    });
    stacr_launch("k_block_select", s, [&] {
        k_block_select<<<(unsigned)n_seg, kSegThreads, 0, s>>>(keys, n_blocks, seg_blocks, count_full, count_last,
                                                                sel);
    });
    stacr_launch("k_block_emit", s, [&] {
        k_block_emit<DT><<<blocks_of(n_out), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, bs,
                                                            n_blocks, sel, n_out, idx, idx_bytes, (T *)values);
    });
    return stacr_hip_check(hipGetLastError(), "block_sparse selector");
}

// Workspace of the adaptive block_sparse selector, carved from one caller-supplied buffer.
struct AdaptiveBlockWs {
    uint32_t *keys;          // energy key per block (rows * bpr)
    uint32_t *cand;          // per-chunk picks, chunk c at c * count_full (n_cand in total)
    uint32_t *ckeys;         // keys of the candidates (global trim)
    uint32_t *pick;          // positions in `cand` the global trim keeps (k_blocks)
    uint32_t *final_blocks;  // the kept blocks, ascending
    int64_t *offsets;        // first output slot of each kept block
};

AdaptiveBlockWs adaptive_block_layout(void *ws, int64_t n_blocks, int64_t n_cand, int64_t k_blocks, size_t *total)
{
    char *p = static_cast<char *>(ws);
    size_t at = 0;
    auto take = [&](size_t bytes) {
        char *here = p ? p + at : nullptr;
        at += (bytes + 255) & ~size_t(255);
        return here;
    };
    AdaptiveBlockWs w;
    w.keys = reinterpret_cast<uint32_t *>(take((size_t)n_blocks * 4));
    w.cand = reinterpret_cast<uint32_t *>(take((size_t)n_cand * 4));
    w.ckeys = reinterpret_cast<uint32_t *>(take((size_t)n_cand * 4));
    w.pick = reinterpret_cast<uint32_t *>(take((size_t)k_blocks * 4));
    w.final_blocks = reinterpret_cast<uint32_t *>(take((size_t)n_cand * 4));
    w.offsets = reinterpret_cast<int64_t *>(take((size_t)n_cand * 8));
    if (total) *total = at;
    return w;
}

template <int DT>
int adaptive_block_typed(const void *x, const void *coeff, const void *q, int64_t rows, int64_t d, int rank,
                         int64_t bs, int64_t chunk_rows, int64_t n_seg, int64_t count_full, int64_t count_last,
                         int64_t k_blocks, void *idx, int idx_bytes, void *values, int64_t *count,
                         const AdaptiveBlockWs &w, hipStream_t s)
{
    using T = typename Act<DT>::T;
    const int64_t bpr = (d + bs - 1) / bs;
    const int64_t n_blocks = rows * bpr;
    const int64_t n_cand = (n_seg - 1) * count_full + count_last;
    const bool trim = n_cand > k_blocks;
    const int64_t n_final = trim ? k_blocks : n_cand;
    stacr_launch("k_block_keys", s, [&] {
        k_block_keys<DT><<<blocks_of(n_blocks), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, bs,
                                                               bpr, n_blocks, w.keys);
    });
    stacr_launch("k_block_select", s, [&] {
        k_block_select<<<(unsigned)n_seg, kSegThreads, 0, s>>>(w.keys, n_blocks, chunk_rows * bpr, count_full,
                                                                count_last, w.cand);
    });
    if (trim) {
        stacr_launch("k_block_gather_keys", s, [&] {
            k_block_gather_keys<<<blocks_of(n_cand), kBlock, 0, s>>>(w.keys, w.cand, n_cand, w.ckeys);
        });
        stacr_launch("k_block_select", s, [&] {
            k_block_select<<<1, kSegThreads, 0, s>>>(w.ckeys, n_cand, n_cand, k_blocks, k_blocks, w.pick);
        });
    }
    stacr_launch("k_block_offsets", s, [&] {
        k_block_offsets<<<1, kSegThreads, 0, s>>>(w.cand, trim ? w.pick : nullptr, n_final, bpr, bs, d, w.final_blocks,
                                                  w.offsets, count);
    });
    stacr_launch("k_block_emit", s, [&] {
        k_block_emit_rows<DT><<<blocks_of(n_final * bs), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank,
                                                                        bs, bpr, n_blocks, w.final_blocks, w.offsets,
                                                                        n_final, idx, idx_bytes, (T *)values);
    });
    return stacr_hip_check(hipGetLastError(), "adaptive block_sparse selector");
}

template <int DT>
int sample_typed(const void *x, const void *coeff, const void *q, int64_t total, int64_t d, int rank,
                 const int64_t *pos, int64_t n, void *out, hipStream_t s)
{
    using T = typename Act<DT>::T;
    if (n > 0)
        stacr_launch("k_sample_abs", s, [&] {
            k_sample_abs<DT><<<blocks_of(n), kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, total,
                                                            pos, n, (T *)out);
        });
    return stacr_hip_check(hipGetLastError(), "sampled magnitudes");
}

template <int DT>
int threshold_typed(const void *x, const void *coeff, const void *q, int64_t rows, int64_t d, int rank,
                    const float *thr, int64_t cap, void *idx, int idx_bytes, void *values, int64_t *count,
                    uint32_t *wg_count, uint32_t *wg_off, hipStream_t s)
{
    using T = typename Act<DT>::T;
    const int64_t total = rows * d;
    const int64_t n_wg = (total + kThrTile - 1) / kThrTile;
    if (n_wg > 0)
        stacr_launch("k_thr_count", s, [&] {
            k_thr_count<DT><<<(unsigned)n_wg, kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, total,
                                                             thr, wg_count);
        });
    stacr_launch("k_thr_offsets", s, [&] {
        k_thr_offsets<<<1, kSegThreads, 0, s>>>(wg_count, n_wg, cap, wg_off, count);
    });
    if (n_wg > 0 && cap > 0)
        stacr_launch("k_thr_emit", s, [&] {
            k_thr_emit<DT><<<(unsigned)n_wg, kBlock, 0, s>>>((TP<DT>)x, (TP<DT>)coeff, (TP<DT>)q, d, rank, total,
                                                            thr, wg_off, cap, idx, idx_bytes, (T *)values);
        });
    return stacr_hip_check(hipGetLastError(), "threshold selector");
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

#define STACR_DT_SWITCH(dt, call)                                            \
    switch (dt) {                                                            \
    case STACR_DTYPE_F32: { constexpr int DT = STACR_DTYPE_F32; return call; } \
    case STACR_DTYPE_BF16: { constexpr int DT = STACR_DTYPE_BF16; return call; } \
    default: { constexpr int DT = STACR_DTYPE_F16; return call; }             \
    }

int stacr_uniform_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                         int rank, int64_t k, void *idx, int idx_bytes, void *values, hipStream_t s)
{
    STACR_DT_SWITCH(dtype, uniform_typed<DT>(x, coeff, q, rows, d, rank, k, idx, idx_bytes, values, s))
}

size_t stacr_block_ws(int64_t rows, int64_t d, int64_t bs, int64_t n_seg, int64_t count_full)
{
    return align256((size_t)(rows * d / bs) * 4) + align256((size_t)(n_seg * count_full) * 4);
}

int stacr_block_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d, int rank,
                       int64_t bs, int64_t seg_rows, int64_t count_full, int64_t count_last, void *idx,
                       int idx_bytes, void *values, void *ws, hipStream_t s)
{
    const int64_t n_seg = (rows + seg_rows - 1) / seg_rows;
    uint32_t *keys = static_cast<uint32_t *>(ws);
    uint32_t *sel = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + align256((size_t)(rows * d / bs) * 4));
    const int64_t seg_blocks = seg_rows * d / bs;
    STACR_DT_SWITCH(dtype, block_typed<DT>(x, coeff, q, rows, d, rank, bs, seg_blocks, n_seg, count_full, count_last,
                                           idx, idx_bytes, values, keys, sel, s))
}

size_t stacr_adaptive_block_ws(int64_t rows, int64_t d, int64_t bs, int64_t n_cand, int64_t k_blocks)
{
    size_t total = 0;
    adaptive_block_layout(nullptr, rows * ((d + bs - 1) / bs), n_cand, k_blocks, &total);
    return total;
}

int stacr_adaptive_block_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                                int rank, int64_t bs, int64_t chunk_rows, int64_t count_full, int64_t count_last,
                                int64_t k_blocks, void *idx, int idx_bytes, void *values, int64_t *count, void *ws,
                                hipStream_t s)
{
    const int64_t n_seg = (rows + chunk_rows - 1) / chunk_rows;
    const int64_t n_cand = (n_seg - 1) * count_full + count_last;
    const AdaptiveBlockWs w = adaptive_block_layout(ws, rows * ((d + bs - 1) / bs), n_cand, k_blocks, nullptr);
    STACR_DT_SWITCH(dtype, adaptive_block_typed<DT>(x, coeff, q, rows, d, rank, bs, chunk_rows, n_seg, count_full,
                                                    count_last, k_blocks, idx, idx_bytes, values, count, w, s))
}

int stacr_sample_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                        int rank, const int64_t *pos, int64_t n, void *out, hipStream_t s)
{
    STACR_DT_SWITCH(dtype, sample_typed<DT>(x, coeff, q, rows * d, d, rank, pos, n, out, s))
}

size_t stacr_threshold_ws(int64_t rows, int64_t d)
{
    const int64_t n_wg = (rows * d + kThrTile - 1) / kThrTile;
    return 2 * align256((size_t)hmax<int64_t>(1, n_wg) * 4);
}

int stacr_threshold_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                           int rank, const float *thr, int64_t cap, void *idx, int idx_bytes, void *values,
                           int64_t *count, void *ws, hipStream_t s)
{
    const int64_t n_wg = (rows * d + kThrTile - 1) / kThrTile;
    uint32_t *wg_count = static_cast<uint32_t *>(ws);
    uint32_t *wg_off = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + align256((size_t)hmax<int64_t>(1, n_wg) * 4));
    STACR_DT_SWITCH(dtype, threshold_typed<DT>(x, coeff, q, rows, d, rank, thr, cap, idx, idx_bytes, values, count,
                                               wg_count, wg_off, s))
}
