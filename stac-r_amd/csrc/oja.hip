// One Oja subspace step of the basis refresh (stacr/layers.py:346-353, stacr/oja.py:64-81):
//   Y = X Q,  U = X^T Y / N - Q (Y^T Y / N),  M = Q + lr U          (all fp32, X read in its dtype)
// The caller re-orthonormalizes M (reduced QR stays a library call).  Every sum has a fixed
// order, so results are deterministic run to run.
//
// 16-bit X with d in {512, 1024, 2048} and rank <= 8 (the projection engine's layers) takes one
// pass over X, three launches:
//   k_oja_pass    a workgroup owns a range of rows; a thread owns 8 columns of a row slot (d / 8
//                 threads per slot, 1, 2 or 4 slots) with those columns' basis rows and X^T Y
//                 accumulators in registers.  Per batch of 8 rows per slot: the 64 partial dots
//                 (8 rows x 8 basis columns) are reduce-scattered across the wave (lane l gets value
//                 l), summed over the slot's waves, and shared through LDS as Y; every thread then
//                 adds x Y to its X^T Y and the slot's first wave adds Y^T Y.  The workgroup's
//                 partial X^T Y and Y^T Y are its output.
//   k_oja_yty_sum one workgroup: Y^T Y = the partials summed in workgroup order (4 stripes, then
//                 the stripes in order)
//   k_oja_finish  8 threads per (feature, basis column) each sum a stripe of the partial X^T Y, the
//                 stripes are added in order, then U and M
// Otherwise four launches:
//   k_oja_y       one wave per row: y = x . Q (lane-strided dot, butterfly), plus the workgroup's
//                 partial Y^T Y over its 16 rows
//   k_oja_yty     one workgroup: Y^T Y = sum of the partials in workgroup order
//   k_oja_xty     (row split, 64-column group): each lane owns one column and R accumulators,
//                 the 4 waves take interleaved rows and are added in LDS in wave order
//   k_oja_update  one thread per (feature, basis column): X^T Y = sum over splits, then U and M
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kOjaRowsPerWg = 16;  // k_oja_y: 4 waves x 4 rows
constexpr int kOjaCols = 64;       // k_oja_xty: columns per workgroup (one per lane)
constexpr int kOjaTargetWg = 1024; // k_oja_xty: workgroups to aim for (4 per CU)
constexpr int kOjaMaxSplit = 256;

struct OjaGeom {
    int R;            // register rank (4, 8, 16 or 32)
    int64_t n_wg;     // k_oja_y workgroups
    int64_t n_cg;     // k_oja_xty column groups
    int64_t n_split;  // k_oja_xty row splits
    size_t off_y, off_ytyp, off_yty, off_part, total;
};

int pad_r(int rank) { return rank <= 4 ? 4 : rank <= 8 ? 8 : rank <= 16 ? 16 : 32; }

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

OjaGeom oja_geom(int64_t rows, int64_t d, int rank)
{
    OjaGeom g{};
    g.R = pad_r(rank);
    g.n_wg = (rows + kOjaRowsPerWg - 1) / kOjaRowsPerWg;
    g.n_cg = (d + kOjaCols - 1) / kOjaCols;
    const int64_t want = (kOjaTargetWg + g.n_cg - 1) / hmax<int64_t>(1, g.n_cg);
    g.n_split = hmax<int64_t>(1, hmin<int64_t>(hmin<int64_t>(want, kOjaMaxSplit), (rows + 3) / 4));
    size_t o = 0;
    g.off_y = o;
    o = align256(o + (size_t)rows * rank * sizeof(float));
    g.off_ytyp = o;
    o = align256(o + (size_t)g.n_wg * g.R * g.R * sizeof(float));
    g.off_yty = o;
    o = align256(o + (size_t)g.R * g.R * sizeof(float));
    g.off_part = o;
    o = align256(o + (size_t)g.n_split * rank * d * sizeof(float));
    g.total = o;
    return g;
}

template <int R>
__global__ __launch_bounds__(kBlock) void k_oja_y(const void *__restrict__ x, int dt, int64_t rows, int64_t d,
                                                  const float *__restrict__ q, int rank, float *__restrict__ y,
                                                  float *__restrict__ yty_part)
{
    __shared__ float s_y[kOjaRowsPerWg][R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * kOjaRowsPerWg;
    for (int k = 0; k < kOjaRowsPerWg / kWaves; ++k) {
        const int lr = wave * (kOjaRowsPerWg / kWaves) + k;
        const int64_t row = r0 + lr;
        float acc[R];
#pragma unroll
        for (int j = 0; j < R; ++j) acc[j] = 0.f;
        if (row < rows) {
            for (int64_t e = lane; e < d; e += 64) {
                const float xv = load_any(x, dt, row * d + e);
                const float *qe = q + e * rank;
#pragma unroll
                for (int j = 0; j < R; ++j)
                    if (j < rank) acc[j] = fmaf(xv, qe[j], acc[j]);
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
#pragma unroll
            for (int j = 0; j < R; ++j) acc[j] += __shfl_xor(acc[j], off, 64);
        // every lane holds all R sums now; lane j keeps column j
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < R; ++j) v = lane == j ? acc[j] : v;
        const bool live = row < rows && lane < rank;
        if (lane < R) s_y[lr][lane] = live ? v : 0.f;
        if (live) y[row * rank + lane] = v;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < R * R; p += kBlock) {
        const int j = p / R, k = p % R;
        float s = 0.f;
        for (int lr = 0; lr < kOjaRowsPerWg; ++lr) s = fmaf(s_y[lr][j], s_y[lr][k], s);
        yty_part[(int64_t)blockIdx.x * R * R + p] = s;
    }
}

template <int R>
__global__ __launch_bounds__(kBlock) void k_oja_yty(const float *__restrict__ yty_part, int64_t n_wg,
                                                    float *__restrict__ yty)
{
    for (int p = threadIdx.x; p < R * R; p += kBlock) {
        float s = 0.f;
        for (int64_t w = 0; w < n_wg; ++w) s += yty_part[w * R * R + p];
        yty[p] = s;
    }
}

template <int R>
__global__ __launch_bounds__(kBlock) void k_oja_xty(const void *__restrict__ x, int dt, int64_t rows, int64_t d,
                                                    const float *__restrict__ y, int rank, int64_t n_split,
                                                    float *__restrict__ part)
{
    __shared__ float s_acc[kWaves - 1][R][kOjaCols];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t split = blockIdx.x;
    const int64_t per = (rows + n_split - 1) / n_split;
    const int64_t t0 = split * per, t1 = t0 + per < rows ? t0 + per : rows;
    const int64_t col = (int64_t)blockIdx.y * kOjaCols + lane;
    const bool live = col < d;
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = 0.f;
    for (int64_t t = t0 + wave; t < t1; t += kWaves) {
        const float xv = live ? load_any(x, dt, t * d + col) : 0.f;
        const float *yt = y + t * rank;
#pragma unroll
        for (int j = 0; j < R; ++j)
            if (j < rank) acc[j] = fmaf(xv, yt[j], acc[j]);
    }
    if (wave > 0)
#pragma unroll
        for (int j = 0; j < R; ++j) s_acc[wave - 1][j][lane] = acc[j];
    __syncthreads();
    if (wave == 0 && live) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            if (j < rank) {
                float s = acc[j];
#pragma unroll
                for (int w = 0; w < kWaves - 1; ++w) s += s_acc[w][j][lane];
                part[(split * rank + j) * d + col] = s;
            }
        }
    }
}

// part is [split][j][feature]; q, update and out are [feature][j].
template <int R>
__global__ __launch_bounds__(kBlock) void k_oja_update(const float *__restrict__ part, int64_t n_split, int64_t d,
                                                       int rank, const float *__restrict__ yty,
                                                       const float *__restrict__ q, float n, float lr,
                                                       float *__restrict__ update, float *__restrict__ out)
{
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= d * rank) return;
    const int64_t i = t % d;
    const int j = (int)(t / d);
    float xs = 0.f;
    for (int64_t s = 0; s < n_split; ++s) xs += part[(s * rank + j) * d + i];
    float qy = 0.f;
    for (int k = 0; k < rank; ++k) qy = fmaf(q[i * rank + k], yty[k * R + j] / n, qy);
    const float u = xs / n - qy;
    update[i * rank + j] = u;
    out[i * rank + j] = fmaf(lr, u, q[i * rank + j]);
}

// ------------------------------------------------------------------ one-pass path
constexpr int kFastR = 8;           // basis columns held per thread (rank <= 8, zero-padded)
constexpr int kFastBatch = 8;       // rows per slot per batch: 8 rows x 8 columns = 64 partials
constexpr int kFastWgs = 256;       // workgroups of the pass (at most)
constexpr int kFastStripes = 8;     // threads summing one output's partials in k_oja_finish

bool oja_fast(int dtype, int64_t rows, int64_t d, int rank)
{
    return (dtype == STACR_DTYPE_BF16 || dtype == STACR_DTYPE_F16) && rows > 0 && rank >= 1 && rank <= kFastR &&
           (d == 512 || d == 1024 || d == 2048);
}

struct OjaFast {
    int W, slots;          // waves per row slot, row slots per workgroup
    int64_t n_wg, rows_per_wg;
    size_t off_xty, off_yty, off_ytysum, total;
};

OjaFast oja_fast_geom(int64_t rows, int64_t d)
{
    OjaFast f{};
    f.W = (int)(d / 512);
    f.slots = kWaves / f.W;
    const int64_t batch_rows = (int64_t)f.slots * kFastBatch;
    // whole batches per workgroup, as many workgroups as give each at least one batch
    const int64_t batches = (rows + batch_rows - 1) / batch_rows;
    f.n_wg = hmin<int64_t>(kFastWgs, batches);
    f.rows_per_wg = ((batches + f.n_wg - 1) / f.n_wg) * batch_rows;
    f.n_wg = (rows + f.rows_per_wg - 1) / f.rows_per_wg;
    size_t o = 0;
    f.off_xty = o;
    o = align256(o + (size_t)f.n_wg * d * kFastR * sizeof(float));
    f.off_yty = o;
    o = align256(o + (size_t)f.n_wg * kFastR * kFastR * sizeof(float));
    f.off_ytysum = o;
    o = align256(o + (size_t)kFastR * kFastR * sizeof(float));
    f.total = o;
    return f;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_oja_pass(const uint16_t *__restrict__ x, int64_t rows, int d,
                                                     const float *__restrict__ q, int rank, int W,
                                                     int64_t rows_per_wg, float *__restrict__ xty_part,
                                                     float *__restrict__ yty_part)
{
    __shared__ float s_part[kWaves * 64];          // per-wave reduce-scatter results
    __shared__ float s_y[kWaves][64];              // Y of the batch, per slot: [row i][column j]
    __shared__ float s_acc[3 * 2048 * kFastR / 4]; // X^T Y of slots 1.. (at the end)
    __shared__ float s_yty[kWaves][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per_slot = 64 * W, slots = kWaves / W;
    const int slot = tid / per_slot, v = tid - slot * per_slot;  // v: this thread's 8 columns 8v ..
    const int w0 = slot * W;                                     // the slot's first wave
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t r1 = r0 + rows_per_wg < rows ? r0 + rows_per_wg : rows;

    // this thread's basis rows (columns 8v .. 8v + 7), zero past the rank
    float qr[8][kFastR];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < kFastR; ++j) qr[e][j] = j < rank ? q[(int64_t)(8 * v + e) * rank + j] : 0.f;
    float acc[8][kFastR];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int j = 0; j < kFastR; ++j) acc[e][j] = 0.f;
    float yty = 0.f;  // the slot's first wave: Y^T Y[lane / 8][lane % 8]

    for (int64_t base = r0; base < r1; base += (int64_t)slots * kFastBatch) {
        // the slot's 8 rows: loads issued together (rows past the range read as zero); the raw
        // 16-bit values stay in registers and are converted where used
        uint4 raw[kFastBatch];
        auto xval = [&](int i, int e) {
            const uint32_t w = e < 2 ? raw[i].x : e < 4 ? raw[i].y : e < 6 ? raw[i].z : raw[i].w;
            return Act<DT>::ld((typename Act<DT>::T)((w >> (16 * (e & 1))) & 0xffffu));
        };
#pragma unroll
        for (int i = 0; i < kFastBatch; ++i) {
            const int64_t row = base + (int64_t)slot * kFastBatch + i;
            raw[i] = row < r1 ? *reinterpret_cast<const uint4 *>(x + row * d + 8 * v) : make_uint4(0u, 0u, 0u, 0u);
        }
        float p[64];
#pragma unroll
        for (int i = 0; i < kFastBatch; ++i) {
#pragma unroll
            for (int j = 0; j < kFastR; ++j) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) t = fmaf(xval(i, e), qr[e][j], t);
                p[i * kFastR + j] = t;
            }
        }
        const float part = wave_reduce_scatter64(p);  // lane l: this wave's sum of value l
        if (W > 1) s_part[wave * 64 + lane] = part;
        __syncthreads();
        if (wave == w0) {
            float y = part;
            for (int w = 1; w < W; ++w) y += s_part[(w0 + w) * 64 + lane];
            s_y[slot][lane] = y;
        }
        __syncthreads();
        if (wave == w0) {  // Y^T Y over the batch's rows, in row order
            const int j = lane >> 3, k = lane & 7;
#pragma unroll
            for (int i = 0; i < kFastBatch; ++i) yty = fmaf(s_y[slot][i * 8 + j], s_y[slot][i * 8 + k], yty);
        }
        // X^T Y: acc[e][j] += x[i][e] Y[i][j], rows in order
#pragma unroll
        for (int i = 0; i < kFastBatch; ++i) {
            float yi[kFastR];
#pragma unroll
            for (int j = 0; j < kFastR; ++j) yi[j] = s_y[slot][i * 8 + j];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xe = xval(i, e);
#pragma unroll
                for (int j = 0; j < kFastR; ++j) acc[e][j] = fmaf(xe, yi[j], acc[e][j]);
            }
        }
        __syncthreads();  // s_y and s_part are rewritten by the next batch
    }

    // the slots' X^T Y added in slot order, then written: [wg][feature][8]
    for (int sl = 1; sl < slots; ++sl) {
        if (slot == sl) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int j = 0; j < kFastR; ++j) s_acc[((sl - 1) * per_slot + v) * 64 + e * 8 + j] = acc[e][j];
        }
    }
    if (wave == w0) s_yty[slot][lane] = yty;
    __syncthreads();
    if (slot == 0) {
        for (int sl = 1; sl < slots; ++sl)
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int j = 0; j < kFastR; ++j) acc[e][j] += s_acc[((sl - 1) * per_slot + v) * 64 + e * 8 + j];
        float4 *dst = reinterpret_cast<float4 *>(xty_part + ((int64_t)blockIdx.x * d + 8 * v) * kFastR);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            dst[2 * e] = make_float4(acc[e][0], acc[e][1], acc[e][2], acc[e][3]);
            dst[2 * e + 1] = make_float4(acc[e][4], acc[e][5], acc[e][6], acc[e][7]);
        }
        if (tid < 64) {
            float t = s_yty[0][tid];
            for (int sl = 1; sl < slots; ++sl) t += s_yty[sl][tid];
            yty_part[(int64_t)blockIdx.x * 64 + tid] = t;
        }
    }
}

// Sum of a[first + k * stride], k = 0 .. n - 1, in order, with the loads issued 16 at a time.
__device__ __forceinline__ float strided_sum(const float *__restrict__ a, int64_t first, int64_t stride, int64_t n)
{
    float t = 0.f;
    for (int64_t k0 = 0; k0 < n; k0 += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = k0 + k < n ? a[first + (k0 + k) * stride] : 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) t += v[k];
    }
    return t;
}

// Y^T Y: thread (stripe s, value p) sums workgroups s, s + 4, ... in order; then the 4 stripes in order
__global__ __launch_bounds__(kBlock) void k_oja_yty_sum(const float *__restrict__ yty_part, int64_t n_wg,
                                                        float *__restrict__ yty)
{
    __shared__ float s_t[4][64];
    const int p = threadIdx.x & 63, st = threadIdx.x >> 6;
    const float t = strided_sum(yty_part, (int64_t)st * 64 + p, 4 * 64, (n_wg - st + 3) / 4);
    s_t[st][p] = t;
    __syncthreads();
    if (threadIdx.x < 64) yty[p] = ((s_t[0][p] + s_t[1][p]) + s_t[2][p]) + s_t[3][p];
}

// kFastStripes threads per output (feature i, column j): stripe s sums workgroups s, s + 8, ...;
// the stripes are then added in order; U = X^T Y / n - (Q Y^T Y / n), M = Q + lr U.
__global__ __launch_bounds__(kBlock) void k_oja_finish(const float *__restrict__ xty_part, int64_t n_wg, int d,
                                                       int rank, const float *__restrict__ yty,
                                                       const float *__restrict__ q, float n, float lr,
                                                       float *__restrict__ update, float *__restrict__ out)
{
    __shared__ float s_t[kBlock];
    const int st = threadIdx.x % kFastStripes;
    const int64_t o = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / kFastStripes;  // output index i * 8 + j
    const int64_t total = (int64_t)d * kFastR;
    const float t = o < total ? strided_sum(xty_part, st * total + o, kFastStripes * total,
                                            (n_wg - st + kFastStripes - 1) / kFastStripes)
                              : 0.f;
    s_t[threadIdx.x] = t;
    __syncthreads();
    if (st != 0 || o >= total) return;
    float xs = 0.f;
    for (int k = 0; k < kFastStripes; ++k) xs += s_t[threadIdx.x + k];
    const int64_t i = o / kFastR;
    const int j = (int)(o % kFastR);
    if (j >= rank) return;
    float qy = 0.f;
    for (int k = 0; k < rank; ++k) qy = fmaf(q[i * rank + k], yty[k * kFastR + j] / n, qy);
    const float u = xs / n - qy;
    update[i * rank + j] = u;
    out[i * rank + j] = fmaf(lr, u, q[i * rank + j]);
}

int launch_oja_fast(const void *x, int dt, int64_t rows, int64_t d, const float *q, int rank, float lr,
                    float *update, float *out, char *ws, hipStream_t s)
{
    const OjaFast f = oja_fast_geom(rows, d);
    float *xty = reinterpret_cast<float *>(ws + f.off_xty);
    float *ytyp = reinterpret_cast<float *>(ws + f.off_yty);
    float *yty = reinterpret_cast<float *>(ws + f.off_ytysum);
    const uint16_t *xs = static_cast<const uint16_t *>(x);
    if (dt == STACR_DTYPE_BF16)
        stacr_launch("k_oja_pass", s, [&] {
            k_oja_pass<STACR_DTYPE_BF16><<<(unsigned)f.n_wg, kBlock, 0, s>>>(xs, rows, (int)d, q, rank, f.W,
                                                                              f.rows_per_wg, xty, ytyp);
        });
    else
        stacr_launch("k_oja_pass", s, [&] {
            k_oja_pass<STACR_DTYPE_F16><<<(unsigned)f.n_wg, kBlock, 0, s>>>(xs, rows, (int)d, q, rank, f.W,
                                                                             f.rows_per_wg, xty, ytyp);
        });
    stacr_launch("k_oja_yty_sum", s, [&] { k_oja_yty_sum<<<1, kBlock, 0, s>>>(ytyp, f.n_wg, yty); });
    const int64_t threads = d * kFastR * kFastStripes;
    const float n_rows = (float)hmax<int64_t>(1, rows);
    stacr_launch("k_oja_finish", s, [&] {
        k_oja_finish<<<(unsigned)((threads + kBlock - 1) / kBlock), kBlock, 0, s>>>(xty, f.n_wg, (int)d, rank, yty, q,
                                                                                   n_rows, lr, update, out);
    });
    return stacr_hip_check(hipGetLastError(), "oja step");
}

template <int R>
int launch_oja(const OjaGeom &g, const void *x, int dt, int64_t rows, int64_t d, const float *q, int rank, float lr,
               float *update, float *out, char *ws, hipStream_t s)
{
    float *y = reinterpret_cast<float *>(ws + g.off_y);
    float *ytyp = reinterpret_cast<float *>(ws + g.off_ytyp);
    float *yty = reinterpret_cast<float *>(ws + g.off_yty);
    float *part = reinterpret_cast<float *>(ws + g.off_part);
    if (g.n_wg > 0)
        stacr_launch("k_oja_y", s,
                     [&] { k_oja_y<R><<<(unsigned)g.n_wg, kBlock, 0, s>>>(x, dt, rows, d, q, rank, y, ytyp); });
    stacr_launch("k_oja_yty", s, [&] { k_oja_yty<R><<<1, kBlock, 0, s>>>(ytyp, g.n_wg, yty); });
    const dim3 grid((unsigned)g.n_split, (unsigned)g.n_cg);
    stacr_launch("k_oja_xty", s,
                 [&] { k_oja_xty<R><<<grid, kBlock, 0, s>>>(x, dt, rows, d, y, rank, g.n_split, part); });
    const int64_t n = d * rank;
    const float n_rows = (float)hmax<int64_t>(1, rows);
    stacr_launch("k_oja_update", s, [&] {
        k_oja_update<R><<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, s>>>(part, g.n_split, d, rank, yty, q,
                                                                                 n_rows, lr, update, out);
    });
    return stacr_hip_check(hipGetLastError(), "oja step");
}

}  // namespace

size_t stacr_oja_ws_bytes(int64_t rows, int64_t d, int rank)
{
    // the larger of the two layouts, so that a workspace sized for one shape serves either path
    const size_t general = oja_geom(rows, d, rank).total;
    return rows > 0 && (d == 512 || d == 1024 || d == 2048) ? hmax(general, oja_fast_geom(rows, d).total) : general;
}

int stacr_oja_launch(const void *x, int dtype, int64_t rows, int64_t d, const float *q, int rank, float lr,
                     float *update, float *out, void *ws, hipStream_t s)
{
    char *w = static_cast<char *>(ws);
    if (oja_fast(dtype, rows, d, rank) && (uintptr_t)x % 16 == 0) return launch_oja_fast(x, dtype, rows, d, q, rank, lr, update, out, w, s);
    const OjaGeom g = oja_geom(rows, d, rank);
    switch (g.R) {
    case 4: return launch_oja<4>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 8: return launch_oja<8>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 16: return launch_oja<16>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    default: return launch_oja<32>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    }
}
