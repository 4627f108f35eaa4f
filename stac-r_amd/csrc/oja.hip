// One Oja subspace step of the basis refresh (stacr/layers.py:346-353, stacr/oja.py:64-81):
//   Y = X Q,  U = X^T Y / N - Q (Y^T Y / N),  M = Q + lr U          (all fp32, X read in its dtype)
// The caller re-orthonormalizes M (reduced QR stays a library call).
// Four launches; every sum has a fixed order, so results are deterministic run to run:
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

size_t stacr_oja_ws_bytes(int64_t rows, int64_t d, int rank) { return oja_geom(rows, d, rank).total; }

int stacr_oja_launch(const void *x, int dtype, int64_t rows, int64_t d, const float *q, int rank, float lr,
                     float *update, float *out, void *ws, hipStream_t s)
{
    const OjaGeom g = oja_geom(rows, d, rank);
    char *w = static_cast<char *>(ws);
    switch (g.R) {
    case 4: return launch_oja<4>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 8: return launch_oja<8>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    case 16: return launch_oja<16>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    default: return launch_oja<32>(g, x, dtype, rows, d, q, rank, lr, update, out, w, s);
    }
}
