// Dense reconstruction of a saved activation: the saved-tensor hooks' unpack
// (stacr/compressor.py:127-133 with stacr/residual.py:13-20).
//
//   out = rnd(C Q^T)                       C: rows x rank, Q: feats x rank, in the activation dtype
//   out = rnd(out + dense(idx, values))    when a residual was saved (the dense tensor is zero
//                                          away from the entries, so elsewhere this only turns
//                                          -0 into +0, as the reference's addition does)
//
// Each element of C Q^T is an fp32 fused-multiply-add chain over the rank, rounded once to the
// activation dtype (the rounding of a 16-bit matrix product accumulated in fp32).  Two launches:
//   k_recon_dense    a thread owns 4 consecutive columns, keeps their basis rows in registers and
//                    walks a range of rows; the row's coefficients are wave-uniform loads
//   k_recon_scatter  one thread per residual entry: the element's low-rank value again (the same
//                    chain), plus the entry's value, rounded once (the indices are unique, so no two
//                    threads touch one element; recomputing keeps the sign of a -0 low-rank value,
//                    which the dense pass has turned into +0, exactly as the reference adds it)
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kCols = 4;           // columns per thread
constexpr int kRowsPerWg = 32;     // rows a workgroup walks

template <int DT, int R>
__global__ __launch_bounds__(kBlock) void k_recon_dense(const typename Act<DT>::T *__restrict__ coeff,
                                                        const typename Act<DT>::T *__restrict__ q, int64_t rows,
                                                        int64_t feats, int rank, int add_zero,
                                                        typename Act<DT>::T *__restrict__ out)
{
    using T = typename Act<DT>::T;
    const int64_t col0 = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * kCols;
    const int64_t r0 = (int64_t)blockIdx.y * kRowsPerWg;
    if (col0 >= feats || r0 >= rows) return;
    const int nc = feats - col0 < kCols ? (int)(feats - col0) : kCols;
    float qv[kCols][R];
#pragma unroll
    for (int c = 0; c < kCols; ++c)
#pragma unroll
        for (int j = 0; j < R; ++j) qv[c][j] = (c < nc && j < rank) ? Act<DT>::ld(q[(col0 + c) * rank + j]) : 0.f;
    const int64_t r1 = r0 + kRowsPerWg < rows ? r0 + kRowsPerWg : rows;
    for (int64_t r = r0; r < r1; ++r) {
        float cj[R];
#pragma unroll
        for (int j = 0; j < R; ++j) cj[j] = j < rank ? Act<DT>::ld(coeff[r * rank + j]) : 0.f;
        T v[kCols];
#pragma unroll
        for (int c = 0; c < kCols; ++c) {
            float p = 0.f;
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (j < rank) p = fmaf(cj[j], qv[c][j], p);
            float o = Act<DT>::rnd(p);
            if (add_zero) o = o + 0.f;
            v[c] = Act<DT>::st(o);
        }
        T *dst = out + r * feats + col0;
        if (nc == kCols && ((uintptr_t)dst % (kCols * sizeof(T))) == 0) {
            if constexpr (sizeof(T) == 2) {
                uint2 w;
                w.x = (uint32_t)(uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16);
                w.y = (uint32_t)(uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16);
                *reinterpret_cast<uint2 *>(dst) = w;
            } else {
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            }
        } else {
            for (int c = 0; c < nc; ++c) dst[c] = v[c];
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kBlock) void k_recon_scatter(const typename Act<DT>::T *__restrict__ coeff,
                                                          const typename Act<DT>::T *__restrict__ q, int64_t feats,
                                                          int rank, const void *__restrict__ idx, int idx64,
                                                          const typename Act<DT>::T *__restrict__ values, int64_t nnz,
                                                          int64_t total, typename Act<DT>::T *__restrict__ out)
{
    const int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (k >= nnz) return;
    const int64_t flat = idx64 ? static_cast<const int64_t *>(idx)[k] : (int64_t) static_cast<const int32_t *>(idx)[k];
    if (flat < 0 || flat >= total) return;  // an entry outside the tensor (invalid input) is skipped
    const int64_t row = flat / feats, col = flat - row * feats;
    float p = 0.f;
    for (int j = 0; j < rank; ++j) p = fmaf(Act<DT>::ld(coeff[row * rank + j]), Act<DT>::ld(q[col * rank + j]), p);
    out[flat] = Act<DT>::st(Act<DT>::rnd(p) + Act<DT>::ld(values[k]));
}

template <int DT, int R>
void launch_dense(const void *coeff, const void *q, int64_t rows, int64_t feats, int rank, int add_zero, void *out,
                  hipStream_t s)
{
    using T = typename Act<DT>::T;
    const dim3 grid((unsigned)((feats + (int64_t)kBlock * kCols - 1) / ((int64_t)kBlock * kCols)),
                    (unsigned)((rows + kRowsPerWg - 1) / kRowsPerWg));
    stacr_launch("k_recon_dense", s, [&] {
        k_recon_dense<DT, R><<<grid, kBlock, 0, s>>>(static_cast<const T *>(coeff), static_cast<const T *>(q), rows,
                                                     feats, rank, add_zero, static_cast<T *>(out));
    });
}

template <int DT>
int launch_typed(const void *coeff, const void *q, int64_t rows, int64_t feats, int rank, const void *idx,
                 int index_bytes, const void *values, int64_t nnz, int has_residual, void *out, hipStream_t s)
{
    using T = typename Act<DT>::T;
    const int add = has_residual ? 1 : 0;
    if (rank <= 4) launch_dense<DT, 4>(coeff, q, rows, feats, rank, add, out, s);
    else if (rank <= 8) launch_dense<DT, 8>(coeff, q, rows, feats, rank, add, out, s);
    else if (rank <= 16) launch_dense<DT, 16>(coeff, q, rows, feats, rank, add, out, s);
    else launch_dense<DT, 32>(coeff, q, rows, feats, rank, add, out, s);
    if (nnz > 0) {
        stacr_launch("k_recon_scatter", s, [&] {
            k_recon_scatter<DT><<<(unsigned)((nnz + kBlock - 1) / kBlock), kBlock, 0, s>>>(
                static_cast<const T *>(coeff), static_cast<const T *>(q), feats, rank, idx, index_bytes == 8,
                static_cast<const T *>(values), nnz, rows * feats, static_cast<T *>(out));
        });
    }
    return stacr_hip_check(hipGetLastError(), "reconstruct kernels");
}

}  // namespace

extern "C" int stacr_reconstruct(const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats, int rank,
                                 const void *idx, int index_bytes, const void *values, int64_t nnz, int has_residual,
                                 void *out, void *stream)
{
    if (rows < 0 || feats < 0) return stacr_fail(STACR_ERR_INVALID, "stacr_reconstruct: negative shape");
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_reconstruct: rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (dtype != STACR_DTYPE_F32 && dtype != STACR_DTYPE_BF16 && dtype != STACR_DTYPE_F16)
        return stacr_fail(STACR_ERR_INVALID, "stacr_reconstruct: unsupported dtype code %d", dtype);
    if (nnz < 0 || (nnz > 0 && index_bytes != 4 && index_bytes != 8))
        return stacr_fail(STACR_ERR_INVALID, "stacr_reconstruct: nnz must be >= 0 and index_bytes 4 or 8");
    if (rows * feats == 0) return STACR_OK;
    if (!coeff || !q || !out || (nnz > 0 && (!idx || !values)))
        return stacr_fail(STACR_ERR_INVALID, "stacr_reconstruct: NULL pointer argument");
    if ((rows + kRowsPerWg - 1) / kRowsPerWg > 65535)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_reconstruct: more than %d rows", 65535 * kRowsPerWg);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
    case STACR_DTYPE_F32:
        return launch_typed<STACR_DTYPE_F32>(coeff, q, rows, feats, rank, idx, index_bytes, values, nnz, has_residual, out, s);
    case STACR_DTYPE_BF16:
        return launch_typed<STACR_DTYPE_BF16>(coeff, q, rows, feats, rank, idx, index_bytes, values, nnz, has_residual, out, s);
    default:
        return launch_typed<STACR_DTYPE_F16>(coeff, q, rows, feats, rank, idx, index_bytes, values, nnz, has_residual, out, s);
    }
}
