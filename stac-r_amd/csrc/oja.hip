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

// ------------------------------------------------------------------ matrix-core path (bf16 X)
// Y = X Q and X^T Y on v_mfma_f32_16x16x32_bf16 at fp32 accuracy: X is exact in bf16, and each
// fp32 operand on the other side (Q, Y) is split into three bf16 terms h + m + l (h = rnd(v),
// m = rnd(v - h), l = rnd(v - h - m); both differences are exact by Sterbenz's lemma), so every
// product is exact, the three terms carry 24 bits of v, and the sums are fp32.  Launches:
//   k_oja_ymf     (row block, group of <= 2048 features): a wave owns 256 features (8 steps of 32)
//                 with their basis operands in registers (its basis rows copied through LDS); per
//                 pair of 16-row tiles 48 products give the wave's partial Y, and the workgroup adds
//                 its waves' partials in wave order.  Output:
//                 the group's Y (fp32); with several groups k_oja_ysum adds them in group order.  Not
//                 launched when the caller supplies Y (the save's own projection, for the adaptive
//                 engine's post-forward refresh).
//   k_oja_xtymf   (256-feature group, row split): 32-row tiles of X copied straight into LDS three
//                 deep (buffer_load ... lds), Y loaded a tile ahead into registers; Y^T is the
//                 products' A operand (three bf16 terms),
//                 X read transposed (ds_read_b64_tr_b16) the B operand, four 16-feature tiles a
//                 wave.  Output: the split's partial X^T Y and (feature group 0) its partial Y^T Y
//                 (on the matrix cores too).
//   k_oja_finish_mf: the partials added in split order (Y^T Y by every workgroup), then U and M.
// X is read once when Y is given, twice otherwise.
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfK = 256;           // features a wave of the Y pass owns
constexpr int kMfSteps = kMfK / 32; // its 32-feature product steps
constexpr int kMfGroup = 2048;      // features of one Y-pass feature group (8 waves)
constexpr int kMfYRows = 16;        // rows per Y-pass tile
constexpr int kMfFg = 256;          // features of one X^T Y workgroup
constexpr int kMfRows = 32;         // rows per X^T Y tile
constexpr int kMfMaxRank = 16;

__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c)
{
    typedef __attribute__((ext_vector_type(8))) __bf16 v8;
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
}

// eight fp32 values -> three bf16 operands (h, m, l), value i in element i of each
__device__ __forceinline__ void split3x8(const float (&v)[8], uint4 (&o)[3])
{
    uint32_t h[8], m[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h[i] = f_to_bf16_bits(v[i]);
        const float r1 = v[i] - bf16_bits_to_f(h[i]);
        m[i] = f_to_bf16_bits(r1);
        l[i] = f_to_bf16_bits(r1 - bf16_bits_to_f(m[i]));
    }
    o[0] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
    o[1] = make_uint4(m[0] | m[1] << 16, m[2] | m[3] << 16, m[4] | m[5] << 16, m[6] | m[7] << 16);
    o[2] = make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
}

// A raw buffer resource over `bytes` bytes at p (clamped to 4 GiB - 1): loads past the end read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t oja_rsrc(const void *p, uint64_t bytes)
{
    const int n = bytes < 0xffffffffull ? (int)(uint32_t)bytes : (int)0xffffffffu;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n, 0x00020000);
}

// 16 bytes per lane at byte voffset of the resource into LDS at wave_dst + 16 * lane
__device__ __forceinline__ void oja_copy16(__amdgpu_buffer_rsrc_t r, void *wave_dst, uint32_t voffset)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)wave_dst, 16, (int)voffset,
                                             0, 0, 0);
}

// ds_read_b64_tr_b16: in a 16-lane group lane m addresses 8 bytes (row r0 + m / 4, columns
// 4 (m % 4) .. + 3 of a 16-column block) and lane n receives the block's column n, rows r0 .. r0 + 3
__device__ __forceinline__ uint2 oja_tr16(const uint16_t *p)
{
    typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
    bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4 *)(p));
    return __builtin_bit_cast(uint2, v);
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void k_oja_ymf(const uint16_t *__restrict__ x, int64_t rows, int64_t d,
                                                      const float *__restrict__ q, int rank, int64_t rows_per_wg,
                                                      int64_t y_stride, float *__restrict__ y)
{
    __shared__ __attribute__((aligned(1024))) float s_q[NW][kMfK * kMfMaxRank];  // each wave's basis rows
    __shared__ float s_p[NW][2 * kMfYRows * 16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, g = lane >> 4;
    const int64_t kg = blockIdx.y;
    const int64_t kw0 = kg * kMfGroup + (int64_t)wave * kMfK;
    // the wave's basis rows kw0 .. kw0 + 255 (contiguous: 256 * rank floats) copied into its own LDS
    // region, 1 KiB a copy (past the basis the loads read 0); the first X tiles' loads are issued
    // behind them, so both latencies overlap
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t r1 = r0 + rows_per_wg < rows ? r0 + rows_per_wg : rows;
    {
        const __amdgpu_buffer_rsrc_t rq = oja_rsrc(q, (uint64_t)d * rank * 4);
        const int copies = (kMfK * rank * 4 + 1023) / 1024;
        for (int c = 0; c < copies; ++c)
            oja_copy16(rq, &s_q[wave][c * 256], (uint32_t)((kw0 * rank) * 4 + c * 1024 + lane * 16));
    }
    // A operands of two 16-row tiles: X[t0 + 16 h + n][kw0 + 32 s + 8 g .. + 7] (rows past the block
    // repeat its last row, columns past d the row's last vector: their basis operands are zero, and
    // their outputs are not written)
    uint4 xa[2][kMfSteps];
    auto load_x = [&](int64_t t0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t row = t0 + 16 * h + n < r1 ? t0 + 16 * h + n : r1 - 1;
#pragma unroll
            for (int s = 0; s < kMfSteps; ++s) {
                const int64_t f = kw0 + 32 * s + 8 * g;
                xa[h][s] = *reinterpret_cast<const uint4 *>(x + row * d + (f < d ? f : d - 8));
            }
        }
    };
    load_x(r0);
    asm volatile("" ::: "memory");  // (keeps the X loads ahead of the basis reads below)
    // basis operands: B[k][n] = Q[kw0 + 32 s + 8 g + k % 8][n], zero past the rank (and past d: the
    // copy read 0 there); a step's eight reads are issued together
    uint4 bq[kMfSteps][3];
    const int ncl = n < rank ? n : rank - 1;
    const float nmask = n < rank ? 1.f : 0.f;
#pragma unroll
    for (int s = 0; s < kMfSteps; ++s) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = s_q[wave][(32 * s + 8 * g + i) * rank + ncl];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= nmask;  // (basis values are finite)
        split3x8(v, bq[s]);
    }
    float *yg = y + kg * y_stride;
    for (int64_t t0 = r0; t0 < r1; t0 += 2 * kMfYRows) {
        f32x4 acc[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            acc[h] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < kMfSteps; ++s)
#pragma unroll
                for (int p = 0; p < 3; ++p) acc[h] = mfma_bf16(xa[h][s], bq[s][p], acc[h]);
        }
        if (t0 + 2 * kMfYRows < r1) load_x(t0 + 2 * kMfYRows);  // the next step's tiles, in flight meanwhile
        // D: lane (n, g) holds rows 4 g .. + 3 of column n
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) s_p[wave][(16 * h + 4 * g + i) * 16 + n] = acc[h][i];
        __syncthreads();
        for (int e = tid; e < 2 * kMfYRows * 16; e += NW * 64) {
            const int i = e >> 4, j = e & 15;
            float v = s_p[0][e];
            for (int w = 1; w < NW; ++w) v += s_p[w][e];
            if (j < rank && t0 + i < r1) yg[(t0 + i) * rank + j] = v;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_oja_xtymf(const uint16_t *__restrict__ x, int64_t rows, int64_t d,
                                                    const float *__restrict__ y, int64_t y_stride, int rank,
                                                    int64_t rows_per_split, float *__restrict__ xty_part,
                                                    float *__restrict__ yty_part)
{
    constexpr int kXElems = kMfRows * kMfFg;  // 16 KiB of bf16 a tile
    __shared__ __attribute__((aligned(1024))) uint16_t s_x0[kXElems];
    __shared__ __attribute__((aligned(1024))) uint16_t s_x1[kXElems];
    __shared__ __attribute__((aligned(1024))) uint16_t s_x2[kXElems];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, g = lane >> 4, m = lane & 15;
    const int64_t f0 = (int64_t)blockIdx.x * kMfFg;
    const int64_t split = blockIdx.y;
    const int64_t t_begin = split * rows_per_split;
    const int64_t t_end = t_begin + rows_per_split < rows ? t_begin + rows_per_split : rows;
    const int nt = (int)((t_end - t_begin + kMfRows - 1) / kMfRows);  // >= 1 (every split has rows)
    const bool do_yty = blockIdx.x == 0;
    (void)y_stride;

    const __amdgpu_buffer_rsrc_t rx = oja_rsrc(x, (uint64_t)rows * d * 2);
    // X tile copies: rows t0 .. t0 + 31, features f0 .. f0 + 255 (row r of the tile holds its 16-byte
    // chunk c at position c ^ (r % 32), so the transposed reads of four rows hit different banks; past
    // the matrix the loads read 0).  Four copies a wave, every step (the tile index clamped: a copy
    // past the last tile refills a buffer nothing reads again), so each step's memory instructions
    // are the same and one wait count serves every step.
    auto issue_x = [&](int b, uint16_t *bx) {
        const int64_t t0 = t_begin + (int64_t)(b < nt ? b : nt - 1) * kMfRows;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = 2 * (4 * wave + k) + (lane >> 5);
            const int c = (lane & 31) ^ (r & 31);
            const uint32_t voff = (uint32_t)(((t0 + r) * d + f0 + 8 * c) * 2);
            oja_copy16(rx, bx + (4 * wave + k) * 512, voff);
        }
    };
    // Y^T operand values of a tile: lane (n, g) takes Y[t0 + 8 g + i][n], i = 0..7 (plain loads, a tile
    // ahead; rows clamped into the split, masked where used)
    const int nc = n < rank ? n : rank - 1;
    auto load_y = [&](int b, float (&v)[8]) {
        const int64_t t0 = t_begin + (int64_t)b * kMfRows;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + 8 * g + i < t_end ? t0 + 8 * g + i : t_end - 1;
            v[i] = y[t * rank + nc];
        }
    };

    f32x4 acc[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) acc[qt] = {0.f, 0.f, 0.f, 0.f};
    // feature group 0, wave 0: Y^T Y on the matrix cores (A = Y^T, B = Y hold the same values per
    // lane); the terms h h, h m, m h, m m, h l, l h (the rest are below fp32 rounding)
    f32x4 yty = {0.f, 0.f, 0.f, 0.f};
    const bool yty_wave = do_yty && wave == 0;

    auto compute = [&](int b, const uint16_t *__restrict__ bx, const float (&yv)[8]) {
        const int64_t t0 = t_begin + (int64_t)b * kMfRows;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = n < rank && t0 + 8 * g + i < t_end ? yv[i] : 0.f;
        uint4 a[3];
        split3x8(v, a);
        const int r_lo = 8 * g + (m >> 2), r_hi = r_lo + 4;
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            const int c = 2 * (4 * wave + qt) + ((m & 3) >> 1);  // chunk of features 16 (4 w + qt) + 4 (m % 4)
            const int eo = (m & 1) * 4;                           // elements into the chunk
            const uint2 lo = oja_tr16(bx + r_lo * kMfFg + ((c ^ (r_lo & 31)) << 3) + eo);
            const uint2 hi = oja_tr16(bx + r_hi * kMfFg + ((c ^ (r_hi & 31)) << 3) + eo);
            const uint4 bop = make_uint4(lo.x, lo.y, hi.x, hi.y);
            acc[qt] = mfma_bf16(a[0], bop, acc[qt]);
            acc[qt] = mfma_bf16(a[1], bop, acc[qt]);
            acc[qt] = mfma_bf16(a[2], bop, acc[qt]);
        }
        if (yty_wave) {
            yty = mfma_bf16(a[0], a[0], yty);
            yty = mfma_bf16(a[0], a[1], yty);
            yty = mfma_bf16(a[1], a[0], yty);
            yty = mfma_bf16(a[1], a[1], yty);
            yty = mfma_bf16(a[0], a[2], yty);
            yty = mfma_bf16(a[2], a[0], yty);
        }
    };

    // Memory order: X(0), X(1), Y(0) ahead; step c issues Y(c + 1), then X(c + 2).  When step c waits,
    // X(c) (two steps back) and Y(c) (one step back) must have landed; the four copies of X(c + 1),
    // issued last, may still fly.  Step 0 waits for everything.
    float ycur[8], ynext[8];
    issue_x(0, s_x0);
    issue_x(1, s_x1);
    load_y(0, ycur);
    auto step = [&](int c, const uint16_t *__restrict__ bx, uint16_t *__restrict__ bx2) {
        if (c == 0) __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
        else __builtin_amdgcn_s_waitcnt(0x0074);         // vmcnt(4) lgkmcnt(0): X(c + 1) may fly
        asm volatile("s_barrier" ::: "memory");
        load_y(c + 1, ynext);
        issue_x(c + 2, bx2);
        compute(c, bx, ycur);
#pragma unroll
        for (int i = 0; i < 8; ++i) ycur[i] = ynext[i];
    };
    int c = 0;
    while (true) {  // every tile but the last, three per round (the buffers known at compile time)
        if (c + 1 >= nt) break;
        step(c++, s_x0, s_x2);
        if (c + 1 >= nt) break;
        step(c++, s_x1, s_x0);
        if (c + 1 >= nt) break;
        step(c++, s_x2, s_x1);
    }
    // the last tile: its copies and Y were issued a step earlier, ahead of one refill of X
    if (c == 0) __builtin_amdgcn_s_waitcnt(0x0070);
    else __builtin_amdgcn_s_waitcnt(0x0074);
    asm volatile("s_barrier" ::: "memory");
    if (c % 3 == 0) compute(c, s_x0, ycur);
    else if (c % 3 == 1) compute(c, s_x1, ycur);
    else compute(c, s_x2, ycur);

    // D: lane (n, g) of tile qt holds (X^T Y)[f0 + 16 (4 w + qt) + n][4 g + i], i = 0..3
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
        const int64_t f = f0 + 16 * (4 * wave + qt) + n;
        if (f >= d) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * g + i;
            if (j < rank) xty_part[(split * d + f) * rank + j] = acc[qt][i];
        }
    }
    if (yty_wave)
#pragma unroll
        for (int i = 0; i < 4; ++i) yty_part[split * 256 + (4 * g + i) * 16 + n] = yty[i];
}

// Y[t][j] = sum over the feature groups of their partial Y, in group order
__global__ __launch_bounds__(256) void k_oja_ysum(const float *__restrict__ yp, int64_t y_stride, int nkg, int64_t n,
                                                 float *__restrict__ y)
{
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    float v = yp[e];
    for (int k = 1; k < nkg; ++k) v += yp[k * y_stride + e];
    y[e] = v;
}

// U = X^T Y / n - Q (Y^T Y / n), M = Q + lr U, 256 outputs a workgroup of 1024 threads.  Sums in a
// fixed order, split st of stripe k = st % 4 taken by the stripe's thread in split order, then the
// four stripes added in order: Y^T Y ([split][j * 16 + k], only the rank x rank values) by every
// workgroup, and X^T Y ([split][feature][rank]) per output; loads issued 16 at a time.
constexpr int kFinStripes = 4;
constexpr int kFinOuts = 256;
__global__ __launch_bounds__(1024) void k_oja_finish_mf(const float *__restrict__ xty_part, int64_t n_split, int64_t d,
                                                       int rank, const float *__restrict__ yty_part,
                                                       const float *__restrict__ q, float n, float lr,
                                                       float *__restrict__ update, float *__restrict__ out)
{
    __shared__ float s_y[kFinStripes][256];
    __shared__ float s_x[kFinStripes][kFinOuts];
    const int tid = threadIdx.x, ol = tid & 255, st = tid >> 8;
    const int64_t o = (int64_t)blockIdx.x * kFinOuts + ol;
    const bool live = o < d * rank;
    const int yj = ol >> 4, yk = ol & 15;
    const bool ylive = yj < rank && yk < rank;
    float xs = 0.f, ys = 0.f;
    for (int64_t s0 = st; s0 < n_split; s0 += 16 * kFinStripes) {
        float vx[16], vy[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const int64_t sp = s0 + (int64_t)c * kFinStripes;
            vx[c] = live && sp < n_split ? xty_part[sp * d * rank + o] : 0.f;
            vy[c] = ylive && sp < n_split ? yty_part[sp * 256 + ol] : 0.f;
        }
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            xs += vx[c];
            ys += vy[c];
        }
    }
    s_x[st][ol] = xs;
    s_y[st][ol] = ys;
    __syncthreads();
    if (st != 0 || !live) return;
    float xt = s_x[0][ol];
#pragma unroll
    for (int k = 1; k < kFinStripes; ++k) xt += s_x[k][ol];
    const int64_t i = o / rank;
    const int j = (int)(o - i * rank);
    float qy = 0.f;
    for (int k = 0; k < rank; ++k) {
        const int yo = k * 16 + j;
        const float yt = ((s_y[0][yo] + s_y[1][yo]) + s_y[2][yo]) + s_y[3][yo];
        qy = fmaf(q[i * rank + k], yt / n, qy);
    }
    const float u = xt / n - qy;
    update[o] = u;
    out[o] = fmaf(lr, u, q[o]);
}

struct OjaMf {
    int nw, nkg;             // Y pass: waves per workgroup, feature groups
    int64_t n_rb, rows_per_wg, y_stride;
    int64_t n_fg, n_split, rows_per_split;
    size_t off_yp, off_y, off_xty, off_ytyp, off_yty, total;
};

bool oja_mf_ok(int dtype, int64_t rows, int64_t d, int rank, const void *x)
{
    return dtype == STACR_DTYPE_BF16 && rows > 0 && rank >= 1 && rank <= kMfMaxRank && d >= 8 && d % 8 == 0 &&
           d <= 4 * kMfGroup && (uintptr_t)x % 16 == 0 && (uint64_t)(rows + kMfRows) * d * 2 < (1ull << 32);
}

OjaMf oja_mf_geom(int64_t rows, int64_t d, int rank)
{
    OjaMf f{};
    f.nkg = (int)((d + kMfGroup - 1) / kMfGroup);
    f.nw = d <= 1024 ? 4 : 8;
    const int64_t ytiles = (rows + 2 * kMfYRows - 1) / (2 * kMfYRows);  // 32-row steps
    f.n_rb = hmax<int64_t>(1, hmin<int64_t>(ytiles, (256 + f.nkg - 1) / f.nkg));
    f.rows_per_wg = ((ytiles + f.n_rb - 1) / f.n_rb) * 2 * kMfYRows;
    f.n_rb = (rows + f.rows_per_wg - 1) / f.rows_per_wg;
    f.y_stride = ((rows + kMfRows - 1) / kMfRows) * kMfRows * rank;  // a group's Y, 16-byte aligned
    f.n_fg = (d + kMfFg - 1) / kMfFg;
    // splits: about 1024 workgroups, each with at least 16 rows per basis column (its partial X^T Y
    // is then at most an eighth of the X it reads)
    const int64_t min_rows = 16 * (rank <= 8 ? 8 : 16);
    const int64_t tiles = (rows + kMfRows - 1) / kMfRows;
    int64_t want = (1024 + f.n_fg - 1) / f.n_fg;
    want = hmin<int64_t>(want, hmax<int64_t>(1, rows / min_rows));
    want = hmax<int64_t>(1, hmin<int64_t>(want, tiles));
    f.rows_per_split = ((tiles + want - 1) / want) * kMfRows;
    f.n_split = (rows + f.rows_per_split - 1) / f.rows_per_split;
    size_t o = 0;
    f.off_yp = o;  // the groups' partial Y (several groups only)
    o = align256(o + (f.nkg > 1 ? (size_t)f.nkg * f.y_stride * sizeof(float) : 0));
    f.off_y = o;
    o = align256(o + (size_t)f.y_stride * sizeof(float));
    f.off_xty = o;
    o = align256(o + (size_t)f.n_split * d * rank * sizeof(float));
    f.off_ytyp = o;
    o = align256(o + (size_t)f.n_split * 256 * sizeof(float));
    f.off_yty = o;
    o = align256(o + 256 * sizeof(float));
    f.total = o;
    return f;
}

// y_given: rows x rank fp32 (X Q computed elsewhere, 16-byte aligned) or NULL
int launch_oja_mf(const void *x, int64_t rows, int64_t d, const float *q, int rank, const float *y_given, float lr,
                  float *update, float *out, char *ws, hipStream_t s)
{
    const OjaMf f = oja_mf_geom(rows, d, rank);
    const uint16_t *xs = static_cast<const uint16_t *>(x);
    float *ybuf = reinterpret_cast<float *>(ws + f.off_y);
    float *xty = reinterpret_cast<float *>(ws + f.off_xty);
    float *ytyp = reinterpret_cast<float *>(ws + f.off_ytyp);
    const float *ysrc = y_given;
    int64_t y_stride = (int64_t)rows * rank;
    if (!y_given) {
        // several groups write partial Y side by side, then k_oja_ysum adds them into ybuf
        float *ygroups = f.nkg > 1 ? reinterpret_cast<float *>(ws + f.off_yp) : ybuf;
        const dim3 grid((unsigned)f.n_rb, (unsigned)f.nkg);
        auto ypass = [&](auto nw) {
            constexpr int NW = decltype(nw)::value;
            stacr_launch("k_oja_ymf", s, [&] {
                k_oja_ymf<NW><<<grid, NW * 64, 0, s>>>(xs, rows, d, q, rank, f.rows_per_wg, f.y_stride, ygroups);
            });
        };
        if (f.nw == 4) ypass(std::integral_constant<int, 4>{});
        else ypass(std::integral_constant<int, 8>{});
        if (f.nkg > 1) {
            const int64_t ny = rows * rank;
            stacr_launch("k_oja_ysum", s, [&] {
                k_oja_ysum<<<(unsigned)((ny + 255) / 256), 256, 0, s>>>(ygroups, f.y_stride, f.nkg, ny, ybuf);
            });
        }
        ysrc = ybuf;
        y_stride = f.y_stride;
    }
    const dim3 grid((unsigned)f.n_fg, (unsigned)f.n_split);
    stacr_launch("k_oja_xtymf", s, [&] {
        k_oja_xtymf<<<grid, 256, 0, s>>>(xs, rows, d, ysrc, y_stride, rank, f.rows_per_split, xty, ytyp);
    });
    const int64_t outs = d * rank;
    const float n_rows = (float)rows;
    stacr_launch("k_oja_finish_mf", s, [&] {
        k_oja_finish_mf<<<(unsigned)((outs + kFinOuts - 1) / kFinOuts), 1024, 0, s>>>(xty, f.n_split, d, rank, ytyp, q,
                                                                                     n_rows, lr, update, out);
    });
    return stacr_hip_check(hipGetLastError(), "oja step (matrix cores)");
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
    // the largest of the layouts, so that a workspace sized for one shape serves every path
    size_t need = oja_geom(rows, d, rank).total;
    if (rows > 0 && (d == 512 || d == 1024 || d == 2048)) need = hmax(need, oja_fast_geom(rows, d).total);
    if (rows > 0 && rank >= 1 && rank <= kMfMaxRank && d >= 8) need = hmax(need, oja_mf_geom(rows, d, rank).total);
    return need;
}

bool stacr_oja_given_y_ok(int dtype, int64_t rows, int64_t d, int rank, const void *x, const void *y)
{
    return oja_mf_ok(dtype, rows, d, rank, x) && y && (uintptr_t)y % 16 == 0 && (rows * rank) % 4 == 0;
}

int stacr_oja_given_y_launch(const void *x, int64_t rows, int64_t d, const float *q, int rank, const float *y,
                             float lr, float *update, float *out, void *ws, hipStream_t s)
{
    return launch_oja_mf(x, rows, d, q, rank, y, lr, update, out, static_cast<char *>(ws), s);
}

int stacr_oja_launch(const void *x, int dtype, int64_t rows, int64_t d, const float *q, int rank, float lr,
                     float *update, float *out, void *ws, hipStream_t s)
{
    char *w = static_cast<char *>(ws);
    if (oja_mf_ok(dtype, rows, d, rank, x)) return launch_oja_mf(x, rows, d, q, rank, nullptr, lr, update, out, w, s);
    if (oja_fast(dtype, rows, d, rank) && (uintptr_t)x % 16 == 0) return launch_oja_fast(x, dtype, rows, d, q, rank, lr, update, out, w, s);
    const OjaGeom g = oja_geom(rows, d, rank);
    switch (g.R) {
    case 4: return launch_oja<4>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 8: return launch_oja<8>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 16: return launch_oja<16>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    default: return launch_oja<32>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    }
}
