// The C1 checkpoint-boundary codec's device work (stacr/protocols/checkpointing.py:411-545):
// everything pack_tensor reads from a boundary activation X (rows x hidden) once its fp32
// coefficients C = X Q are formed (a library GEMM, as the reference's `flat_fp32 @ basis_fp32`),
// the stored coefficients, and unpack_record's reconstruction.
//
//   k_c1_observe   one pass over X: thread = one feature, its basis row in registers; for each row
//                  (the workgroup's coefficient rows staged in LDS) the reconstruction
//                  p = sum_j c_j q_j (fp32 chain, j ascending), the residual e = x - p, and per
//                  workgroup fp64 sums of e^2 and x^2 (each square rounded to fp32 first, as
//                  `pow(2)` does), NaN flags and NaN-ignoring max |.| of X, the
//                  reconstruction and the residual; the first feature block also reduces the
//                  coefficients (per-component max |c| propagating NaN, flags) and the basis
//   k_c1_finish    one workgroup: the partials in a fixed order (the same result on every run),
//                  the energy error / max(denom, 1e-12), and the per-component scales
//                  s_j = (m_j finite and > 0 ? m_j : 1) / 127 (_quantize_coefficients, :374-393)
//   k_c1_store     the record's coefficients: int8 clamp(round_half_even(c / s_j), -127, 127), or
//                  C rounded once to the basis dtype
//   k_c1_restore   out = sum_j c'_j q_j in fp32 (c' = code * s_j for int8 coefficients), rounded
//                  once to the boundary's dtype (_dequantize_coefficients and unpack_record,
//                  :395-400,531-545)
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kC1Threads = 256;  // features per workgroup of the observe / restore passes
constexpr int kC1Stage = 16;     // coefficient rows staged in LDS at a time
constexpr int kC1Rows = 64;      // rows per workgroup

struct C1Part {
    double err, x2;
    float xmax, rmax, emax, pad;
    uint32_t flags, pad2[3];
};

__device__ __forceinline__ float ld_any(const void *p, int dt, int64_t i) { return load_any(p, dt, i); }

// NaN-ignoring max of |v| (inf included) and the flags it raises (bits: a NaN, a value not NaN)
__device__ __forceinline__ void observe(float v, float &m, uint32_t &flags, uint32_t nan_bit, uint32_t valid_bit)
{
    const float a = fabsf(v);
    if (a != a) {
        flags |= nan_bit;
        return;
    }
    flags |= valid_bit;
    m = fmaxf(m, a);
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_or(uint32_t v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v |= (uint32_t)__shfl_xor((int)v, off, 64);
    return v;
}
__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int R>
__global__ __launch_bounds__(kC1Threads) void k_c1_observe(const void *__restrict__ x, int x_dt, int64_t rows,
                                                           int64_t hidden, const float *__restrict__ coeff,
                                                           const void *__restrict__ basis, int b_dt, int rank,
                                                           C1Part *__restrict__ parts, float *__restrict__ camax,
                                                           float *__restrict__ maxes)
{
    __shared__ __align__(16) float s_c[kC1Stage * R];
    __shared__ double s_d[2][kC1Threads / 64];
    __shared__ float s_f[3][kC1Threads / 64];
    __shared__ uint32_t s_u[kC1Threads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t col = (int64_t)blockIdx.x * kC1Threads + tid;
    const bool col_ok = col < hidden;
    const bool coeff_block = blockIdx.x == 0;  // also reduces the coefficients of its rows
    uint32_t flags = 0u;
    float q[R];
    float bmax = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        q[j] = (col_ok && j < rank) ? ld_any(basis, b_dt, col * rank + j) : 0.f;
        if (blockIdx.y == 0 && col_ok && j < rank) observe(q[j], bmax, flags, STACR_C1_BASIS_NAN, STACR_C1_BASIS_VALID);
    }
    float xmax = 0.f, rmax = 0.f, emax = 0.f, cmax = 0.f, cam = 0.f;
    double err = 0.0, x2 = 0.0;
    const int64_t row0 = (int64_t)blockIdx.y * kC1Rows;
    const int64_t row1 = row0 + kC1Rows < rows ? row0 + kC1Rows : rows;
    for (int64_t rb = row0; rb < row1; rb += kC1Stage) {
        const int n = (int)(row1 - rb < kC1Stage ? row1 - rb : kC1Stage);
        __syncthreads();  // the previous stage's reads are done
        for (int i = tid; i < n * R; i += kC1Threads) {
            const int r = i / R, j = i - (i / R) * R;
            s_c[i] = j < rank ? coeff[(rb + r) * rank + j] : 0.f;
        }
        __syncthreads();
        if (coeff_block && tid < rank) {
            for (int r = 0; r < n; ++r) {
                const float c = s_c[r * R + tid];
                observe(c, cmax, flags, STACR_C1_COEFF_NAN, STACR_C1_COEFF_VALID);
                const float a = fabsf(c);
                cam = (a != a || cam != cam) ? __builtin_nanf("") : fmaxf(cam, a);
            }
        }
        if (col_ok) {
            for (int r = 0; r < n; ++r) {
                const float *c = s_c + r * R;
                float p = 0.f;
#pragma unroll
                for (int j = 0; j < R; ++j)
                    if (j < rank) p = fmaf(c[j], q[j], p);
                const float xv = ld_any(x, x_dt, (rb + r) * hidden + col);
                const float e = xv - p;
                observe(xv, xmax, flags, STACR_C1_INPUT_NAN, STACR_C1_INPUT_VALID);
                observe(p, rmax, flags, STACR_C1_RECON_NAN, STACR_C1_RECON_VALID);
                observe(e, emax, flags, STACR_C1_RESIDUAL_NAN, STACR_C1_RESIDUAL_VALID);
                err += (double)(e * e);
                x2 += (double)(xv * xv);
            }
        }
    }
    if (coeff_block && tid < rank) camax[blockIdx.y * rank + tid] = cam;
    // the workgroup's partials (wave order, then waves in order)
    err = wave_sum(err);
    x2 = wave_sum(x2);
    xmax = wave_max(xmax);
    rmax = wave_max(rmax);
    emax = wave_max(fmaxf(emax, 0.f));
    bmax = wave_max(bmax);
    cmax = wave_max(cmax);
    flags = wave_or(flags);
    if (lane == 0) {
        s_d[0][wave] = err;
        s_d[1][wave] = x2;
        s_f[0][wave] = xmax;
        s_f[1][wave] = rmax;
        s_f[2][wave] = emax;
        s_u[wave] = flags;
    }
    __syncthreads();
    if (tid == 0) {
        C1Part pt{};
        for (int w = 0; w < kC1Threads / 64; ++w) {
            pt.err += s_d[0][w];
            pt.x2 += s_d[1][w];
            pt.xmax = fmaxf(pt.xmax, s_f[0][w]);
            pt.rmax = fmaxf(pt.rmax, s_f[1][w]);
            pt.emax = fmaxf(pt.emax, s_f[2][w]);
            pt.flags |= s_u[w];
        }
        parts[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = pt;
    }
    // the coefficient maxima of the first feature block (per row group) and the basis maxima of
    // the first row group (per feature block): maxes[g] and maxes[groups + b]
    __syncthreads();
    if (lane == 0) {
        s_f[0][wave] = cmax;
        s_f[1][wave] = bmax;
    }
    __syncthreads();
    if (tid == 0) {
        float cm = 0.f, bm = 0.f;
        for (int w = 0; w < kC1Threads / 64; ++w) {
            cm = fmaxf(cm, s_f[0][w]);
            bm = fmaxf(bm, s_f[1][w]);
        }
        if (coeff_block) maxes[blockIdx.y] = cm;
        if (blockIdx.y == 0) maxes[gridDim.y + blockIdx.x] = bm;
    }
}

// One workgroup: partials in a fixed order, the stats record and the per-component scales.
__global__ __launch_bounds__(kC1Threads) void k_c1_finish(const C1Part *__restrict__ parts, int64_t n_parts,
                                                          const float *__restrict__ camax, const float *__restrict__ maxes,
                                                          int64_t groups, int64_t col_blocks, int rank,
                                                          StacrC1Stats *__restrict__ stats, float *__restrict__ scales)
{
    __shared__ double s_d[2][kC1Threads];
    __shared__ float s_f[5][kC1Threads];
    __shared__ uint32_t s_u[kC1Threads];
    const int tid = threadIdx.x;
    double err = 0.0, x2 = 0.0;
    float xmax = 0.f, rmax = 0.f, emax = 0.f, cmax = 0.f, bmax = 0.f;
    uint32_t flags = 0u;
    for (int64_t i = tid; i < n_parts; i += kC1Threads) {
        const C1Part p = parts[i];
        err += p.err;
        x2 += p.x2;
        xmax = fmaxf(xmax, p.xmax);
        rmax = fmaxf(rmax, p.rmax);
        emax = fmaxf(emax, p.emax);
        flags |= p.flags;
    }
    for (int64_t g = tid; g < groups; g += kC1Threads) cmax = fmaxf(cmax, maxes[g]);
    for (int64_t b = tid; b < col_blocks; b += kC1Threads) bmax = fmaxf(bmax, maxes[groups + b]);
    s_d[0][tid] = err;
    s_d[1][tid] = x2;
    s_f[0][tid] = xmax;
    s_f[1][tid] = rmax;
    s_f[2][tid] = emax;
    s_f[3][tid] = cmax;
    s_f[4][tid] = bmax;
    s_u[tid] = flags;
    __syncthreads();
    for (int half = kC1Threads / 2; half > 0; half >>= 1) {  // a fixed tree
        if (tid < half) {
            s_d[0][tid] += s_d[0][tid + half];
            s_d[1][tid] += s_d[1][tid + half];
#pragma unroll
            for (int k = 0; k < 5; ++k) s_f[k][tid] = fmaxf(s_f[k][tid], s_f[k][tid + half]);
            s_u[tid] |= s_u[tid + half];
        }
        __syncthreads();
    }
    if (tid < rank) {
        float m = 0.f;
        for (int64_t g = 0; g < groups; ++g) {
            const float a = camax[g * rank + tid];
            m = (a != a || m != m) ? __builtin_nanf("") : fmaxf(m, a);
        }
        const bool ok = m == m && m > 0.f && m <= 3.402823466e38f;
        scales[tid] = (ok ? m : 1.f) / 127.f;
    }
    if (tid == 0) {
        StacrC1Stats st{};
        st.error = s_d[0][0];
        st.denom = s_d[1][0];
        const float e32 = (float)st.error, d32 = fmaxf((float)st.denom, 1e-12f);
        st.energy = e32 / d32;
        st.input_max_abs = s_f[0][0];
        st.reconstruction_max_abs = s_f[1][0];
        st.residual_max_abs = s_f[2][0];
        st.coeff_max_abs = s_f[3][0];
        st.basis_max_abs = s_f[4][0];
        st.flags = s_u[0];
        *stats = st;
    }
}

template <int OUT>
__global__ __launch_bounds__(kC1Threads) void k_c1_store(const float *__restrict__ coeff, int64_t n, int rank,
                                                         const float *__restrict__ scales, int quantize,
                                                         void *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * kC1Threads + threadIdx.x;
    if (i >= n) return;
    const float c = coeff[i];
    if (quantize) {
        const float qv = rintf(c / scales[i % rank]);
        const float cl = qv != qv ? 0.f : fminf(fmaxf(qv, -127.f), 127.f);
        static_cast<int8_t *>(out)[i] = (int8_t)(int)cl;
    } else {
        static_cast<typename Act<OUT>::T *>(out)[i] = Act<OUT>::st(c);
    }
}

template <int R, int OUT>
__global__ __launch_bounds__(kC1Threads) void k_c1_restore(const void *__restrict__ coeff, int c_dt,
                                                           const float *__restrict__ scales,
                                                           const void *__restrict__ basis, int b_dt, int64_t rows,
                                                           int64_t hidden, int rank,
                                                           typename Act<OUT>::T *__restrict__ out)
{
    __shared__ __align__(16) float s_c[kC1Stage * R];
    const int tid = threadIdx.x;
    const int64_t col = (int64_t)blockIdx.x * kC1Threads + tid;
    const bool col_ok = col < hidden;
    float q[R];
#pragma unroll
    for (int j = 0; j < R; ++j) q[j] = (col_ok && j < rank) ? ld_any(basis, b_dt, col * rank + j) : 0.f;
    const int64_t row0 = (int64_t)blockIdx.y * kC1Rows;
    const int64_t row1 = row0 + kC1Rows < rows ? row0 + kC1Rows : rows;
    for (int64_t rb = row0; rb < row1; rb += kC1Stage) {
        const int n = (int)(row1 - rb < kC1Stage ? row1 - rb : kC1Stage);
        __syncthreads();
        for (int i = tid; i < n * R; i += kC1Threads) {
            const int r = i / R, j = i - (i / R) * R;
            float v = 0.f;
            if (j < rank) {
                const int64_t e = (rb + r) * rank + j;
                v = c_dt == STACR_DTYPE_I8 ? (float)static_cast<const int8_t *>(coeff)[e] * scales[j]
                                           : ld_any(coeff, c_dt, e);
            }
            s_c[i] = v;
        }
        __syncthreads();
        if (col_ok) {
            for (int r = 0; r < n; ++r) {
                const float *c = s_c + r * R;
                float p = 0.f;
#pragma unroll
                for (int j = 0; j < R; ++j)
                    if (j < rank) p = fmaf(c[j], q[j], p);
                out[(rb + r) * hidden + col] = Act<OUT>::st(p);
            }
        }
    }
}

int pad_c1_rank(int rank) { return rank <= 8 ? 8 : rank <= 16 ? 16 : rank <= 32 ? 32 : rank <= 64 ? 64 : 128; }

bool float_dt(int dt) { return dt == STACR_DTYPE_F32 || dt == STACR_DTYPE_BF16 || dt == STACR_DTYPE_F16; }

int64_t c1_groups(int64_t rows) { return (rows + kC1Rows - 1) / kC1Rows; }
int64_t c1_col_blocks(int64_t hidden) { return (hidden + kC1Threads - 1) / kC1Threads; }

size_t c1_ws(int64_t rows, int64_t hidden, int rank)
{
    const int64_t g = c1_groups(rows), b = c1_col_blocks(hidden);
    const size_t parts = (size_t)(g * b) * sizeof(C1Part);
    const size_t cam = (size_t)(g * rank) * sizeof(float);
    const size_t fl = (size_t)(g + b) * sizeof(float);
    return ((parts + 255) & ~(size_t)255) + ((cam + 255) & ~(size_t)255) + fl;
}

}  // namespace

extern "C" int stacr_c1_workspace_bytes(int64_t rows, int64_t hidden, int rank, size_t *bytes)
{
    if (rows < 0 || hidden < 0 || rank < 1 || rank > STACR_C1_MAX_RANK || !bytes)
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_workspace_bytes: bad shape (rank 1..%d)", STACR_C1_MAX_RANK);
    *bytes = c1_ws(rows, hidden, rank);
    return STACR_OK;
}

extern "C" int stacr_c1_observe(const void *x, int dtype, int64_t rows, int64_t hidden, const float *coeff,
                                const void *basis, int basis_dtype, int rank, void *stats, float *scales,
                                void *workspace, size_t workspace_bytes, void *stream)
{
    if (!float_dt(dtype) || !float_dt(basis_dtype)) return stacr_fail(STACR_ERR_INVALID, "stacr_c1_observe: unsupported dtype");
    if (rows < 1 || hidden < 1 || rank < 1 || rank > STACR_C1_MAX_RANK)
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_observe: bad shape (rank 1..%d)", STACR_C1_MAX_RANK);
    if (c1_groups(rows) > 65535) return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_c1_observe: more than %d rows", 65535 * kC1Rows);
    if (!x || !coeff || !basis || !stats || !scales || !workspace) return stacr_fail(STACR_ERR_INVALID, "stacr_c1_observe: NULL pointer argument");
    if (workspace_bytes < c1_ws(rows, hidden, rank))
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_c1_observe: workspace has %zu bytes, needs %zu", workspace_bytes,
                          c1_ws(rows, hidden, rank));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t g = c1_groups(rows), b = c1_col_blocks(hidden);
    char *ws = static_cast<char *>(workspace);
    C1Part *parts = reinterpret_cast<C1Part *>(ws);
    const size_t parts_b = ((size_t)(g * b) * sizeof(C1Part) + 255) & ~(size_t)255;
    float *camax = reinterpret_cast<float *>(ws + parts_b);
    float *maxes = reinterpret_cast<float *>(ws + parts_b + (((size_t)(g * rank) * sizeof(float) + 255) & ~(size_t)255));
    const dim3 grid((unsigned)b, (unsigned)g);
    auto go = [&](auto r) {
        constexpr int R = decltype(r)::value;
        stacr_launch("k_c1_observe", s, [&] {
            k_c1_observe<R><<<grid, kC1Threads, 0, s>>>(x, dtype, rows, hidden, coeff, basis, basis_dtype, rank, parts,
                                                        camax, maxes);
        });
    };
    switch (pad_c1_rank(rank)) {
    case 8: go(std::integral_constant<int, 8>{}); break;
    case 16: go(std::integral_constant<int, 16>{}); break;
    case 32: go(std::integral_constant<int, 32>{}); break;
    case 64: go(std::integral_constant<int, 64>{}); break;
    default: go(std::integral_constant<int, 128>{}); break;
    }
    stacr_launch("k_c1_finish", s, [&] {
        k_c1_finish<<<1, kC1Threads, 0, s>>>(parts, g * b, camax, maxes, g, b, rank, static_cast<StacrC1Stats *>(stats), scales);
    });
    return stacr_hip_check(hipGetLastError(), "c1 observe");
}

extern "C" int stacr_c1_store(const float *coeff, int64_t rows, int rank, const float *scales, int quantize, void *out,
                              int out_dtype, void *stream)
{
    if (rows < 0 || rank < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_c1_store: bad shape");
    if (quantize ? out_dtype != STACR_DTYPE_I8 : !float_dt(out_dtype))
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_store: output dtype must be int8 when quantizing, else a float type");
    if (rows == 0) return STACR_OK;
    if (!coeff || !out || (quantize && !scales)) return stacr_fail(STACR_ERR_INVALID, "stacr_c1_store: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t n = rows * rank;
    const unsigned grid = (unsigned)((n + kC1Threads - 1) / kC1Threads);
    stacr_launch("k_c1_store", s, [&] {
        if (quantize || out_dtype == STACR_DTYPE_F32)
            k_c1_store<STACR_DTYPE_F32><<<grid, kC1Threads, 0, s>>>(coeff, n, rank, scales, quantize, out);
        else if (out_dtype == STACR_DTYPE_BF16)
            k_c1_store<STACR_DTYPE_BF16><<<grid, kC1Threads, 0, s>>>(coeff, n, rank, scales, 0, out);
        else
            k_c1_store<STACR_DTYPE_F16><<<grid, kC1Threads, 0, s>>>(coeff, n, rank, scales, 0, out);
    });
    return stacr_hip_check(hipGetLastError(), "c1 store");
}

extern "C" int stacr_c1_restore(const void *coeff, int coeff_dtype, const float *scales, const void *basis,
                                int basis_dtype, int64_t rows, int64_t hidden, int rank, void *out, int out_dtype,
                                void *stream)
{
    if (!(float_dt(coeff_dtype) || coeff_dtype == STACR_DTYPE_I8) || !float_dt(basis_dtype) || !float_dt(out_dtype))
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_restore: unsupported dtype");
    if (rows < 0 || hidden < 0 || rank < 1 || rank > STACR_C1_MAX_RANK)
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_restore: bad shape (rank 1..%d)", STACR_C1_MAX_RANK);
    if (rows == 0 || hidden == 0) return STACR_OK;
    if (c1_groups(rows) > 65535) return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_c1_restore: more than %d rows", 65535 * kC1Rows);
    if (!coeff || !basis || !out || (coeff_dtype == STACR_DTYPE_I8 && !scales))
        return stacr_fail(STACR_ERR_INVALID, "stacr_c1_restore: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)c1_col_blocks(hidden), (unsigned)c1_groups(rows));
    auto go = [&](auto r, auto o) {
        constexpr int R = decltype(r)::value, OUT = decltype(o)::value;
        stacr_launch("k_c1_restore", s, [&] {
            k_c1_restore<R, OUT><<<grid, kC1Threads, 0, s>>>(coeff, coeff_dtype, scales, basis, basis_dtype, rows, hidden,
                                                             rank, static_cast<typename Act<OUT>::T *>(out));
        });
    };
    auto by_out = [&](auto r) {
        if (out_dtype == STACR_DTYPE_F32) go(r, std::integral_constant<int, STACR_DTYPE_F32>{});
        else if (out_dtype == STACR_DTYPE_BF16) go(r, std::integral_constant<int, STACR_DTYPE_BF16>{});
        else go(r, std::integral_constant<int, STACR_DTYPE_F16>{});
    };
    switch (pad_c1_rank(rank)) {
    case 8: by_out(std::integral_constant<int, 8>{}); break;
    case 16: by_out(std::integral_constant<int, 16>{}); break;
    case 32: by_out(std::integral_constant<int, 32>{}); break;
    case 64: by_out(std::integral_constant<int, 64>{}); break;
    default: by_out(std::integral_constant<int, 128>{}); break;
    }
    return stacr_hip_check(hipGetLastError(), "c1 restore");
}
