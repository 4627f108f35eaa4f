// Reduced QR of a tall fp32 matrix A (rows x cols, cols <= 16, rows * cols <= 32768) in one
// workgroup: the basis re-orthonormalization after every Oja step (stacr/oja.py:8-11,
// stacr/adaptive.py:3368), which the reference runs as torch.linalg.qr.
//
// The factorization follows LAPACK's unblocked Householder QR (sgeqr2 with slarfg's reflector,
// then sorg2r forming Q in place), so Q and R carry LAPACK's signs: R[j][j] = -sign(alpha_j)
// ||(alpha_j, x_j)|| for the j-th partially reduced column (alpha_j its diagonal entry, x_j the
// entries below), a reflector with tau = 0 where x_j = 0.  The matrix is held in registers (up to
// 64 values a thread of 512); norms and dot products accumulate in fp32, as LAPACK's sgeqr2, in a
// fixed order (each thread's rows in order, DPP rotations within 16 lanes, the rows and waves in
// order), so the result is the same on every run.  One launch replaces the chain of small library
// launches a QR costs otherwise.
#include <utility>

#include "internal.h"

using namespace stacr;

namespace {

// f(std::integral_constant<int, J>) for J = 0 .. N - 1, in order: the column steps unrolled with
// the column index a compile-time constant (the matrix is held in registers)
template <typename F, int... Js>
__device__ __forceinline__ void qr_static_for(F &&f, std::integer_sequence<int, Js...>)
{
    (f(std::integral_constant<int, Js>{}), ...);
}

constexpr int kQrThreads = 512;
constexpr int kQrWaves = kQrThreads / 64;
constexpr int kQrMaxCols = 16;
constexpr int kQrMaxElems = 32768;  // rows * cols: 64 values a thread

// x shifted by a DPP row rotation (CTRL)
template <int CTRL>
__device__ __forceinline__ float qr_dpp(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float qr_lane(float x, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// x from this lane's partner within its 16-lane row for exchange distance D, by one DPP move that
// every lane executes alike (a per-lane choice between two moves is compiled into branches, and a
// DPP move then reads lanes the branch has switched off): D = 8, row_ror:8 (lane l ^ 8); D = 4,
// row_half_mirror (lane l ^ 7); D = 2, 1, quad_perm [2 3 0 1] and [1 0 3 2] (lanes l ^ 2, l ^ 1)
template <int D>
__device__ __forceinline__ float qr_xor(float x)
{
    if constexpr (D == 8) return qr_dpp<0x128>(x);       // row_ror:8
    else if constexpr (D == 4) return qr_dpp<0x141>(x);  // row_half_mirror
    else if constexpr (D == 2) return qr_dpp<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    else return qr_dpp<0xB1>(x);                         // quad_perm [1, 0, 3, 2]
}

// P values a[0..P-1] (P = 4, 8, 16) summed over the wave's 64 lanes: lane l ends with the total of
// value l % P.  Within each 16-lane row a butterfly over the partners of distances 8, 4, 2, 1 (lane
// l ^ 8, l ^ 7, l ^ 2, l ^ 1, which between them reach all 16 lanes once): halving exchanges (a
// lane keeps the half of the values its lane bit names and adds its partner's share of it) for
// the bits that index the values, plain sums for the others, ordered so that partners always
// hold the same values (the sum over the l ^ 7 partner comes before any exchange, or is an
// exchange itself).  Then rows 0 + 1 and 2 + 3, and the two halves, by v_permlane16_swap /
// v_permlane32_swap, whose pairs add the lower lane's value to the upper's in every lane; plain
// sums likewise add lower + upper in both lanes, so every lane holding value c has the same bits.
template <int P>
__device__ __forceinline__ float qr_wave_scatter(float (&a)[P])
{
    const int lane = threadIdx.x & 63;
    auto scatter = [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        const bool upper = (lane & D) != 0;
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const float send = upper ? a[k] : a[k + D], keep = upper ? a[k + D] : a[k];
            a[k] = keep + qr_xor<D>(send);
        }
    };
    auto fold = [&](auto dc, auto nc) {  // a[k] += the partner's a[k], k < N (lower + upper in both lanes)
        constexpr int D = decltype(dc)::value, N = decltype(nc)::value;
        const bool upper = (lane & D) != 0;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const float other = qr_xor<D>(a[k]);
            a[k] = upper ? other + a[k] : a[k] + other;
        }
    };
    using I8 = std::integral_constant<int, 8>;
    using I4 = std::integral_constant<int, 4>;
    using I2 = std::integral_constant<int, 2>;
    using I1 = std::integral_constant<int, 1>;
    if constexpr (P == 16) {
        scatter(I8{});
        scatter(I4{});
    } else if constexpr (P == 8) {
        scatter(I4{});
    } else {
        fold(I4{}, I4{});
    }
    scatter(I2{});
    scatter(I1{});
    if constexpr (P <= 8) fold(I8{}, I1{});
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[0]), __float_as_uint(a[0]), false, false);
    float x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sums of C per-thread values over the workgroup, in a fixed order, the same bits in every
// thread: the wave's totals (C >= 4: the reduce-scatter above, lane c holding value c; fewer: each
// 16-lane row by DPP rotations (1, 2, 4, 8) and the four row sums (lanes 0, 16, 32, 48) in order),
// then the waves' sums in order through LDS (two slots, alternated by the caller, so one barrier
// suffices; lane c of each wave reads value c's).
template <int C>
__device__ __forceinline__ void qr_sums(float *v, float (*s_part)[kQrMaxCols + 1])
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if constexpr (C >= 4) {
        constexpr int P = C <= 4 ? 4 : C <= 8 ? 8 : 16;
        static_assert(C <= 16, "at most 16 values a sum");
        float a[P];
#pragma unroll
        for (int c = 0; c < P; ++c) a[c] = c < C ? v[c] : 0.f;
        const float t = qr_wave_scatter<P>(a);
        if (lane < C) s_part[wave][lane] = t;
    } else {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            float x = v[c];
            x += qr_dpp<0x121>(x);  // row_ror:1
            x += qr_dpp<0x122>(x);  // row_ror:2
            x += qr_dpp<0x124>(x);  // row_ror:4
            x += qr_dpp<0x128>(x);  // row_ror:8
            const float t = ((qr_lane(x, 0) + qr_lane(x, 16)) + qr_lane(x, 32)) + qr_lane(x, 48);
            if (lane == 0) s_part[wave][c] = t;
        }
    }
    __syncthreads();
    // lane c of every wave adds value c over the waves, in order; the wave then shares the C
    // totals through scalar registers
    float t = 0.f;
    if (lane < C) {
#pragma unroll
        for (int w = 0; w < kQrWaves; ++w) t += s_part[w][lane];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = qr_lane(t, c);
}

// The matrix lives in registers: thread t holds rows t + p * 512 (p < RPT) of all K columns, so
// every step below is unrolled over the columns (indices known at compile time); columns at or past
// n are zero and take no part.
template <int RPT, int K>
__global__ __launch_bounds__(kQrThreads) void k_qr_house(const float *__restrict__ a, int64_t m, int n,
                                                         float *__restrict__ q, float *__restrict__ r)
{
    __shared__ float s_part[2][kQrWaves][kQrMaxCols + 1];  // alternated by the reductions
    __shared__ float s_alpha[kQrMaxCols];
    int slot = 0;
    auto sums = [&](auto cc, float *v) {
        qr_sums<decltype(cc)::value>(v, s_part[slot]);
        slot ^= 1;
    };
    const int tid = threadIdx.x;
    float x[RPT][K];
#pragma unroll
    for (int p = 0; p < RPT; ++p) {
        const int64_t row = tid + (int64_t)p * kQrThreads;
#pragma unroll
        for (int k = 0; k < K; ++k) x[p][k] = row < m && k < n ? a[row * n + k] : 0.f;
    }
    float tau[K];

    // ---- dgeqr2: for each column, dlarfg's reflector, then the trailing columns
    qr_static_for([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (j >= n) return;  // (uniform)
        // alpha = A[j][j] (thread j holds row j, j < 512), the squares below it
        if (tid == j) s_alpha[j] = x[0][j];
        float ss = 0.f;
#pragma unroll
        for (int p = 0; p < RPT; ++p) {
            const int64_t row = tid + (int64_t)p * kQrThreads;
            if (row > j && row < m) ss = fmaf(x[p][j], x[p][j], ss);
        }
        sums(std::integral_constant<int, 1>{}, &ss);
        const float alpha = s_alpha[j];
        tau[j] = 0.f;
        float beta = alpha;
        if (ss > 0.f) {  // (uniform)
            beta = -copysignf(sqrtf(fmaf(alpha, alpha, ss)), alpha);
            tau[j] = (beta - alpha) / beta;
            const float scale = 1.f / (alpha - beta);
#pragma unroll
            for (int p = 0; p < RPT; ++p) {
                const int64_t row = tid + (int64_t)p * kQrThreads;
                if (row > j) x[p][j] *= scale;  // v below the diagonal (v_j = 1)
            }
            if constexpr (j + 1 < K) {
                // w_k = sum_{i >= j} v_i A[k][i] for k > j, then A[k][i] -= tau w_k v_i
                float w[K - j - 1];
#pragma unroll
                for (int k = j + 1; k < K; ++k) {
                    float t = 0.f;
#pragma unroll
                    for (int p = 0; p < RPT; ++p) {
                        const int64_t row = tid + (int64_t)p * kQrThreads;
                        const float vi = row == j ? 1.f : row > j ? x[p][j] : 0.f;
                        t = fmaf(vi, x[p][k], t);
                    }
                    w[k - j - 1] = t;
                }
                sums(std::integral_constant<int, K - j - 1>{}, w);
#pragma unroll
                for (int p = 0; p < RPT; ++p) {
                    const int64_t row = tid + (int64_t)p * kQrThreads;
                    if (row < j) continue;
                    const float vi = row == j ? 1.f : x[p][j];
#pragma unroll
                    for (int k = j + 1; k < K; ++k) x[p][k] = fmaf(-tau[j] * w[k - j - 1], vi, x[p][k]);
                }
            }
        }
        if (tid == j) x[0][j] = beta;  // R[j][j]
    }, std::make_integer_sequence<int, K>{});
    // R: row j is thread j's (p = 0) entries at columns >= j
    if (r && tid < n) {
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (k < n) r[tid * n + k] = k >= tid ? x[0][k] : 0.f;
    }

    // ---- dorg2r: Q in place, from the last reflector to the first
    qr_static_for([&](auto jc) {
        constexpr int j = K - 1 - decltype(jc)::value;
        if (j >= n) return;  // (uniform)
        if constexpr (j + 1 < K) {
            if (tau[j] != 0.f && j + 1 < n) {  // (uniform) apply H_j to the columns already formed
                float w[K - j - 1];
#pragma unroll
                for (int k = j + 1; k < K; ++k) {
                    float t = 0.f;
#pragma unroll
                    for (int p = 0; p < RPT; ++p) {
                        const int64_t row = tid + (int64_t)p * kQrThreads;
                        const float vi = row == j ? 1.f : row > j ? x[p][j] : 0.f;
                        t = fmaf(vi, x[p][k], t);
                    }
                    w[k - j - 1] = t;
                }
                sums(std::integral_constant<int, K - j - 1>{}, w);
#pragma unroll
                for (int p = 0; p < RPT; ++p) {
                    const int64_t row = tid + (int64_t)p * kQrThreads;
                    if (row < j) continue;
                    const float vi = row == j ? 1.f : x[p][j];
#pragma unroll
                    for (int k = j + 1; k < K; ++k) x[p][k] = fmaf(-tau[j] * w[k - j - 1], vi, x[p][k]);
                }
            }
        }
#pragma unroll
        for (int p = 0; p < RPT; ++p) {
            const int64_t row = tid + (int64_t)p * kQrThreads;
            x[p][j] = row < j ? 0.f : row == j ? 1.f - tau[j] : -tau[j] * x[p][j];
        }
    }, std::make_integer_sequence<int, K>{});
#pragma unroll
    for (int p = 0; p < RPT; ++p) {
        const int64_t row = tid + (int64_t)p * kQrThreads;
        if (row >= m) continue;
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (k < n) q[row * n + k] = x[p][k];
    }
}

}  // namespace

extern "C" int stacr_qr(const float *a, int64_t rows, int cols, float *q, float *r, void *stream)
{
    if (rows < 1 || cols < 1 || cols > rows) return stacr_fail(STACR_ERR_INVALID, "stacr_qr: bad shape %lld x %d",
                                                             (long long)rows, cols);
    if (!a || !q) return stacr_fail(STACR_ERR_INVALID, "stacr_qr: NULL pointer argument");
    if (cols > kQrMaxCols || rows * (int64_t)cols > kQrMaxElems)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_qr: needs cols <= %d and rows * cols <= %d", kQrMaxCols,
                          kQrMaxElems);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // (rows a thread holds, and the columns rounded up: RPT * K <= 64)
    const int rpt = (int)((rows + kQrThreads - 1) / kQrThreads);
    auto go = [&](auto kernel) { stacr_launch("k_qr_house", s, [&] { kernel<<<1, kQrThreads, 0, s>>>(a, rows, cols, q, r); }); };
    if (rpt <= 2 && cols <= 8) go(k_qr_house<2, 8>);
    else if (rpt <= 2 && cols <= 16) go(k_qr_house<2, 16>);
    else if (rpt <= 4 && cols <= 8) go(k_qr_house<4, 8>);
    else if (rpt <= 4) go(k_qr_house<4, 16>);
    else if (rpt <= 8) go(k_qr_house<8, 8>);
    else go(k_qr_house<16, 4>);
    return stacr_hip_check(hipGetLastError(), "stacr_qr");
}
