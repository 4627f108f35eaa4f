// Reduced QR of a tall fp32 matrix past the one-workgroup kernel's size (cols <= 16, any number of
// rows): the basis re-orthonormalization of wide layers (stacr/oja.py:8-11, stacr/adaptive.py:3368,
// where the reference runs torch.linalg.qr), e.g. cfg 4's 8192 x 16 basis.
//
// CholeskyQR in fp64, with LAPACK's signs.  For A = Q+ R+ (R+ with a positive diagonal), LAPACK's
// Householder QR (sgeqr2: R[j][j] = -sign(alpha_j) * norm, tau = 0 where the column below the
// diagonal is zero) gives R = S R+ and Q = Q+ S for a diagonal S of signs, and its reflectors are the
// same for A and for Q+ (the columns of A are positive combinations of those of Q+ along R+'s
// diagonal).  The Householder QR of an orthonormal Q+ has R = S, and S comes out of an LU of Q+'s
// top n x n block without pivoting in which every pivot first picks s_j = -sign(d_j) for the
// current diagonal entry d_j (the alpha of step j) and then eliminates with d_j - s_j (Ballard,
// Demmel, Grigori, Jacquelin, Nguyen and Solomonik, "Reconstructing Householder vectors from
// tall-skinny QR", 2014); |d_j| = 1 is LAPACK's tau = 0 case, where the sign is kept.
//
//   k_qrt_gram    P workgroups: the partial Gram matrices A_p^T A_p of their row slices in fp64 on
//                 v_mfma_f64_16x16x4f64 (each lane's element is both operands), into the workspace.
//   k_qrt_factor  one workgroup: the partials summed in slice order, G = R+^T R+ (Cholesky), X = R+^-1,
//                 the top block of Q+ = A X and its sign-choosing LU: M = X S into the workspace,
//                 R = S R+ into r.  Where the fp64 route is not exact enough (a Cholesky pivot below
//                 1e-10 of its column's squared norm, i.e. a column within 1e-5 of the span of the
//                 earlier ones, a zero column among them; or a condition estimate above 1e5), the same
//                 workgroup runs LAPACK's Householder QR itself with the matrix streamed through q
//                 (sgeqr2, then sorg2r forming Q in place), and flags it.  (A sign decision with |d_j|
//                 near zero stays on the fp64 route: there LAPACK's fp32 alpha has no reliable sign
//                 either, and a Householder QR summing in another order would not reproduce it.)
//   k_qrt_apply   P workgroups: Q = A M (fp64 products, rounded once to fp32), unless flagged.
// Every sum has a fixed order, so the result is the same on every run.
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kQtCols = 16;
constexpr int kQtGramThreads = 256;  // 4 waves
constexpr int kQtFactorThreads = 512;
constexpr int kQtBatch = 8;        // rows a thread loads together in the Householder route's passes
constexpr int kQtMaxSlices = 32;  // the factor sums the slices' partials: few of them
typedef double d4 __attribute__((ext_vector_type(4)));

struct QtGeom {
    int64_t rows;
    int cols;
    int64_t rows_per_slice;  // a multiple of 16
    int slices;
};

// workspace (doubles): [slices][256] partial Gram matrices, then M [256], then the flag
__host__ __device__ inline size_t qt_m_offset(int slices) { return (size_t)slices * 256; }
__host__ __device__ inline size_t qt_flag_offset(int slices) { return (size_t)slices * 256 + 256; }

// ---- the partial Gram matrices
__global__ __launch_bounds__(kQtGramThreads) void k_qrt_gram(const float *__restrict__ a, QtGeom g,
                                                             double *__restrict__ ws)
{
    __shared__ double s_acc[4][256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * g.rows_per_slice;
    const int64_t r1 = r0 + g.rows_per_slice < g.rows ? r0 + g.rows_per_slice : g.rows;
    const int col = lane & 15;
    d4 acc = {0.0, 0.0, 0.0, 0.0};
    // groups of 4 rows; lane l holds A[row + l / 16][l % 16], both the A (i = col, k = row) and the
    // B (k = row, j = col) operand of G += A_g^T A_g
    for (int64_t row = r0 + 4 * wave; row < r1; row += 16) {
        const int64_t rr = row + (lane >> 4);
        const double v = rr < r1 && col < g.cols ? (double)a[rr * g.cols + col] : 0.0;
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(v, v, acc, 0, 0, 0);
    }
    // D layout: lane l, slot k holds G[l / 16 + 4 k][l % 16]
#pragma unroll
    for (int k = 0; k < 4; ++k) s_acc[wave][((lane >> 4) + 4 * k) * 16 + col] = acc[k];
    __syncthreads();
    const int e = threadIdx.x;  // 256 entries, the waves in order
    ws[(size_t)blockIdx.x * 256 + e] = ((s_acc[0][e] + s_acc[1][e]) + s_acc[2][e]) + s_acc[3][e];
}

// One value a thread summed over the threads of the same column (lanes c, c + 16, c + 32, c + 48 of
// every wave: an xor tree over the wave's four row groups, then the waves in order), in one exchange
// (two barriers).  Every thread receives its column's total and, in *pivot, column j's.  s_part holds
// 16 values a wave.
__device__ __forceinline__ float qt_column_sum(float v, int j, float *pivot, float *s_part)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c = lane & 15;
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lane < 16) s_part[wave * 16 + lane] = v;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);
    float t = s_part[c], tj = s_part[j];
    for (int w = 1; w < nw; ++w) {
        t += s_part[w * 16 + c];
        tj += s_part[w * 16 + j];
    }
    __syncthreads();
    *pivot = tj;
    return t;
}

// LAPACK's sgeqr2 + sorg2r on A (rows x n, row-major in q, fp32), streamed by the workgroup: thread t
// takes column t % 16 of rows t / 16, t / 16 + blockDim / 16, ... in every pass, kQtBatch of them
// loaded together (sixteen consecutive threads read one row's consecutive words), a row's column-j
// entry passed along its sixteen lanes;
// each column's sums over its threads' rows in that order, then over the workgroup.  R into r (n x n,
// may be NULL), Q left in q.  (LAPACK's rescaling of a reflector whose beta is below the safe minimum
// is not made: inputs that small fall outside fp32's normal range.)
__device__ void qt_householder(const float *__restrict__ a, int64_t m, int n, float *__restrict__ q,
                               float *__restrict__ r, float *s_part, float *s_tau)
{
    const int lane = threadIdx.x & 63, c = lane & 15, base = lane & 48;
    const int64_t g0 = threadIdx.x >> 4, gstep = blockDim.x >> 4;
    const bool col = c < n;
    for (int64_t i = threadIdx.x; i < m * n; i += blockDim.x) q[i] = a[i];
    __syncthreads();
    for (int j = 0; j < n; ++j) {
        // the squared norm of x = A[j+1:, j] (column j's threads) and the dots of x with the columns
        // k > j (column k's threads)
        float part = 0.f;
        for (int64_t i0 = g0; i0 < m; i0 += kQtBatch * gstep) {
            float e[kQtBatch];
#pragma unroll
            for (int u = 0; u < kQtBatch; ++u) {
                const int64_t i = i0 + u * gstep;
                e[u] = col && i < m ? q[i * n + c] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < kQtBatch; ++u) {
                const int64_t i = i0 + u * gstep;
                const float x = __shfl(e[u], base + j, 64);
                if (i > j && i < m) part = fmaf(x, e[u], part);
            }
        }
        float norm2;
        const float dot = qt_column_sum(part, j, &norm2, s_part);
        const float alpha = q[(int64_t)j * n + j];
        const float xnorm = sqrtf(norm2);
        float tau = 0.f, beta = alpha, scale = 0.f;
        if (xnorm != 0.f) {  // slarfg: beta = -sign(alpha) * hypot(alpha, xnorm)
            const float h = hypotf(alpha, xnorm);
            beta = alpha >= 0.f ? -h : h;
            tau = (beta - alpha) / beta;
            scale = 1.f / (alpha - beta);
        }
        // w_c = v^T A[:, c] for c > j (v_j = 1, v_i = scale x_i)
        const float wc = col && c > j ? q[(int64_t)j * n + c] + scale * dot : 0.f;
        if (threadIdx.x == 0) s_tau[j] = tau;
        __syncthreads();  // (row j is read above and written below)
        for (int64_t i0 = g0; i0 < m; i0 += kQtBatch * gstep) {
            float e[kQtBatch];
#pragma unroll
            for (int u = 0; u < kQtBatch; ++u) {
                const int64_t i = i0 + u * gstep;
                e[u] = col && i < m ? q[i * n + c] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < kQtBatch; ++u) {
                const int64_t i = i0 + u * gstep;
                const float x = __shfl(e[u], base + j, 64);
                if (i < j || i >= m || !col) continue;
                const float v = i == j ? 1.f : x * scale;
                if (c > j && tau != 0.f) q[i * n + c] = fmaf(-tau * wc, v, e[u]);
                if (c == j) q[i * n + c] = i == j ? beta : v;  // R[j][j], then the reflector below
            }
        }
        __syncthreads();
    }
    if (r)
        for (int e = threadIdx.x; e < n * n; e += blockDim.x) {
            const int i = e / n, k = e % n;
            r[e] = k >= i ? q[(int64_t)i * n + k] : 0.f;
        }
    __syncthreads();
    // sorg2r: from the last reflector to the first
    for (int j = n - 1; j >= 0; --j) {
        const float tau = s_tau[j];
        if (tau != 0.f && j + 1 < n) {  // (uniform) H_j on the columns already formed
            float part = 0.f;
            for (int64_t i0 = g0; i0 < m; i0 += kQtBatch * gstep) {
                float e[kQtBatch];
#pragma unroll
                for (int u = 0; u < kQtBatch; ++u) {
                    const int64_t i = i0 + u * gstep;
                    e[u] = col && i < m ? q[i * n + c] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < kQtBatch; ++u) {
                    const int64_t i = i0 + u * gstep;
                    const float x = __shfl(e[u], base + j, 64);
                    if (i >= j && i < m) part = fmaf(i == j ? 1.f : x, e[u], part);
                }
            }
            float unused;
            const float dot = qt_column_sum(part, j, &unused, s_part);
            const float wc = c > j ? dot : 0.f;
            for (int64_t i0 = g0; i0 < m; i0 += kQtBatch * gstep) {
                float e[kQtBatch];
#pragma unroll
                for (int u = 0; u < kQtBatch; ++u) {
                    const int64_t i = i0 + u * gstep;
                    e[u] = col && i < m ? q[i * n + c] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < kQtBatch; ++u) {
                    const int64_t i = i0 + u * gstep;
                    const float x = __shfl(e[u], base + j, 64);
                    if (i >= j && i < m && col && c > j) q[i * n + c] = fmaf(-tau * wc, i == j ? 1.f : x, e[u]);
                }
            }
            __syncthreads();
        }
        for (int64_t i = g0; i < m; i += gstep) {  // column j itself
            if (c != j) continue;
            const float v = q[i * n + j];
            q[i * n + j] = i < j ? 0.f : i == j ? 1.f - tau : -tau * v;
        }
        __syncthreads();
    }
}

// x in lane l (l wave-uniform), to every lane
__device__ __forceinline__ double qt_lane(double x, int l)
{
    const uint64_t b = (uint64_t)__double_as_longlong(x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// ---- the factorization
__global__ __launch_bounds__(kQtFactorThreads) void k_qrt_factor(const float *__restrict__ a, QtGeom g,
                                                                 double *__restrict__ ws, float *__restrict__ q,
                                                                 float *__restrict__ r)
{
    __shared__ double s_red[2][256];
    __shared__ double s_g[256], s_a[256];
    __shared__ float s_partf[kQtFactorThreads / 64 * 16], s_tau[kQtCols];
    __shared__ int s_ok;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = g.cols;
    {   // G: the slices' partials summed in slice order (two interleaved runs, then in order), eight
        // loads in flight at a time
        const int e = tid & 255, run = tid >> 8;
        double s = 0.0;
        int p = run;
        for (; p + 14 < g.slices; p += 16) {
            double v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = ws[(size_t)(p + 2 * k) * 256 + e];
#pragma unroll
            for (int k = 0; k < 8; ++k) s += v[k];
        }
        for (; p < g.slices; p += 2) s += ws[(size_t)p * 256 + e];
        s_red[run][e] = s;
    }
    // A's top n x n block (for the sign-choosing LU)
    if (tid < n * n) s_a[tid] = (double)a[tid];
    __syncthreads();
    if (tid < 256) s_g[tid] = s_red[0][tid] + s_red[1][tid];
    __syncthreads();
    if (wave == 0) {
        // lane c (< n) holds column c of each matrix in registers; row entries of other columns
        // come by readlane (all loops unrolled: indices are compile-time constants)
        const int c = lane;
        const bool mine = c < n;
        double w[kQtCols];  // G's column c, then R's (right-looking Cholesky, in place)
#pragma unroll
        for (int i = 0; i < kQtCols; ++i) w[i] = mine ? s_g[i * 16 + c] : 0.0;
        bool ok = true;
        double idg[kQtCols];  // 1 / R[j][j] (the same in every lane)
        // (every loop runs its full constant count, the steps past n skipped by uniform branches, so
        // that it unrolls and every register and lane index is a constant)
#pragma unroll
        for (int j = 0; j < kQtCols; ++j) {
            if (j < n) {
                const double wjj = qt_lane(w[j], j);
                ok = ok && wjj > 1e-10 * s_g[j * 16 + j];
                const double rjj = sqrt(wjj > 0.0 ? wjj : 1e-300), inv = 1.0 / rjj;
                idg[j] = inv;
                // row j of R: R[j][c] = W[j][c] / R[j][j] (c > j), R[j][j]; zero left of the diagonal
                w[j] = c > j ? w[j] * inv : c == j ? rjj : 0.0;
                // the trailing rows: W[i][c] -= R[j][i] R[j][c] for j < i <= c
#pragma unroll
                for (int i = j + 1; i < kQtCols; ++i) {
                    if (i < n) {
                        const double rji = qt_lane(w[j], i);
                        if (c >= i) w[i] -= rji * w[j];
                    }
                }
            }
        }
        // X = R^-1, column c, rows from the bottom: X[i][c] = (delta_ic - sum_{p>i} R[i][p] X[p][c]) / R[i][i]
        // (times the reciprocal from the Cholesky step)
        double x[kQtCols];
#pragma unroll
        for (int i = kQtCols - 1; i >= 0; --i) {
            x[i] = 0.0;
            if (i < n) {
                double v = c == i ? 1.0 : 0.0;
#pragma unroll
                for (int p = i + 1; p < kQtCols; ++p)
                    if (p < n) v -= qt_lane(w[i], p) * x[p];
                x[i] = mine ? v * idg[i] : 0.0;
            }
        }
        // condition estimate ||R||_F ||X||_F
        double fr = 0.0, fx = 0.0;
#pragma unroll
        for (int i = 0; i < kQtCols; ++i) {
            fr += mine && i <= c ? w[i] * w[i] : 0.0;
            fx += x[i] * x[i];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            fr += __shfl_xor(fr, off, 64);
            fx += __shfl_xor(fx, off, 64);
        }
        ok = ok && sqrt(fr) * sqrt(fx) <= 1e5;
        // T = A[0:n] X, column c
        double t[kQtCols];
#pragma unroll
        for (int i = 0; i < kQtCols; ++i) {
            double v = 0.0;
            if (i < n)
#pragma unroll
                for (int p = 0; p < kQtCols; ++p)
                    if (p < n) v += s_a[i * n + p] * x[p];
            t[i] = v;
        }
        // the sign-choosing LU of T: s_j = -sign(d_j) (kept where |d_j| = 1), then eliminate with d_j - s_j
        double sg[kQtCols], my_s = 1.0;
#pragma unroll
        for (int j = 0; j < kQtCols; ++j) {
            sg[j] = 1.0;
            if (j < n) {
                const double d = qt_lane(t[j], j), ad = fabs(d);
                if (ad >= 1.0 - 1e-12) {
                    sg[j] = d >= 0.0 ? 1.0 : -1.0;
                } else {
                    sg[j] = d >= 0.0 ? -1.0 : 1.0;
                    const double inv_u = 1.0 / (d - sg[j]);
#pragma unroll
                    for (int i = j + 1; i < kQtCols; ++i)
                        if (i < n) {
                            const double l = qt_lane(t[i], j) * inv_u;
                            if (c > j) t[i] -= l * t[j];
                        }
                }
                if (c == j) my_s = sg[j];
            }
        }
        // M = X S into the workspace, R = S R+ into r
        double *wm = ws + qt_m_offset(g.slices);
        if (c < 16)
#pragma unroll
            for (int i = 0; i < kQtCols; ++i) wm[i * 16 + c] = mine ? x[i] * my_s : 0.0;
        if (r && mine)
#pragma unroll
            for (int i = 0; i < kQtCols; ++i)
                if (i < n) r[i * n + c] = c >= i ? (float)(sg[i] * w[i]) : 0.f;
        if (c == 0) s_ok = ok ? 1 : 0;
    }
    __syncthreads();
    if (tid == 0) ws[qt_flag_offset(g.slices)] = s_ok ? 1.0 : 0.0;
    if (!s_ok) qt_householder(a, g.rows, n, q, r, s_partf, s_tau);  // (uniform)
}

// ---- Q = A M
__global__ __launch_bounds__(kQtGramThreads) void k_qrt_apply(const float *__restrict__ a, QtGeom g,
                                                              const double *__restrict__ ws, float *__restrict__ q)
{
    if (ws[qt_flag_offset(g.slices)] == 0.0) return;  // (uniform) the Householder route wrote q
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, kk = lane >> 4;
    const double *wm = ws + qt_m_offset(g.slices);
    double mb[4];  // B operand of k-chunk c: M[4 c + kk][col]
#pragma unroll
    for (int c = 0; c < 4; ++c) mb[c] = wm[(4 * c + kk) * 16 + col];
    const int64_t r0 = (int64_t)blockIdx.x * g.rows_per_slice;
    const int64_t r1 = r0 + g.rows_per_slice < g.rows ? r0 + g.rows_per_slice : g.rows;
    for (int64_t row0 = r0 + 16 * wave; row0 < r1; row0 += 64) {
        // A operand of chunk c: lane l holds A[row0 + l % 16][4 c + l / 16]
        const int64_t ra = row0 + col;
        d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = 4 * c + kk;
            const double v = ra < r1 && k < g.cols ? (double)a[ra * g.cols + k] : 0.0;
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(v, mb[c], acc, 0, 0, 0);
        }
        // D: lane l, slot s holds row row0 + l / 16 + 4 s, column l % 16
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t row = row0 + kk + 4 * s;
            if (row < r1 && col < g.cols) q[row * g.cols + col] = (float)acc[s];
        }
    }
}

QtGeom qt_geom(int64_t rows, int cols)
{
    QtGeom g;
    g.rows = rows;
    g.cols = cols;
    int64_t per = (rows + kQtMaxSlices - 1) / kQtMaxSlices;
    per = per < 64 ? 64 : per;
    per = (per + 15) / 16 * 16;
    g.rows_per_slice = per;
    g.slices = (int)((rows + per - 1) / per);
    return g;
}

}  // namespace

extern "C" int stacr_qr_tall_workspace_bytes(int64_t rows, int cols, size_t *bytes)
{
    if (!bytes) return stacr_fail(STACR_ERR_INVALID, "stacr_qr_tall_workspace_bytes: NULL output");
    if (rows < 1 || cols < 1 || cols > kQtCols || cols > rows)
        return stacr_fail(STACR_ERR_INVALID, "stacr_qr_tall: bad shape %lld x %d", (long long)rows, cols);
    const QtGeom g = qt_geom(rows, cols);
    *bytes = (qt_flag_offset(g.slices) + 1) * sizeof(double);
    return STACR_OK;
}

extern "C" int stacr_qr_tall(const float *a, int64_t rows, int cols, float *q, float *r, void *workspace,
                             size_t workspace_bytes, void *stream)
{
    size_t need = 0;
    const int rc = stacr_qr_tall_workspace_bytes(rows, cols, &need);
    if (rc) return rc;
    if (!a || !q || !workspace) return stacr_fail(STACR_ERR_INVALID, "stacr_qr_tall: NULL pointer argument");
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_qr_tall: workspace has %zu bytes, needs %zu", workspace_bytes, need);
    if ((uintptr_t)workspace % 8) return stacr_fail(STACR_ERR_INVALID, "stacr_qr_tall: workspace not 8-byte aligned");
    const QtGeom g = qt_geom(rows, cols);
    hipStream_t s = static_cast<hipStream_t>(stream);
    double *ws = static_cast<double *>(workspace);
    stacr_launch("k_qrt_gram", s, [&] { k_qrt_gram<<<g.slices, kQtGramThreads, 0, s>>>(a, g, ws); });
    stacr_launch("k_qrt_factor", s, [&] { k_qrt_factor<<<1, kQtFactorThreads, 0, s>>>(a, g, ws, q, r); });
    stacr_launch("k_qrt_apply", s, [&] { k_qrt_apply<<<g.slices, kQtGramThreads, 0, s>>>(a, g, ws, q); });
    return stacr_hip_check(hipGetLastError(), "stacr_qr_tall");
}
