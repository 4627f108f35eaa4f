// Weight gradient from the saved factors: dW = (G^T C) Q^T + G^T R_s, dbias = sum_t G.
//
// Restates stacr/layers.py:172-198.  All accumulation is fp32 and the result is rounded once to
// the weight dtype (the reference rounds the d_out x r product and the low-rank term to G's dtype
// before adding the fp32 sparse correction; the fp32 path here is the more accurate of the two).
//   csr_rows   ascending flat indices -> per-token row offsets, columns, dequantized values
//              (QuantizedValues.dequantize(fp32), stacr/quant.py:17-21,40-46)
//   lowrank    partial M = G^T [C | 1] over token splits (the ones column yields dbias)
//   reduce     M = sum of the partials
//   sparse     per (64 output features x W_i input features) tile: stream G rows that own
//              residual entries in the tile and accumulate v * G[t, :] in LDS
//   expand     dW[o][i] = sum_j M[o][j] Q[i][j] + S[o][i], in nn.Linear or Conv1D orientation
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kSparseO = 64;    // output features per sparse tile (one per lane)
constexpr int kSparseI = 240;   // input features per sparse tile: 240 x 65 fp32 = 61 KiB of LDS
constexpr int kLdsPitch = kSparseO + 1;
constexpr int kTokTile = 64;

template <int IDX64>
__global__ void k_csr_rows(const void *__restrict__ idx, int64_t nnz, int64_t d_in, int64_t rows,
                           const void *__restrict__ data, const float *__restrict__ scale, int bits, int val_dt,
                           uint32_t *__restrict__ rowptr, uint32_t *__restrict__ col, float *__restrict__ val)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    auto flat_at = [&](int64_t k) -> int64_t {
        return IDX64 ? static_cast<const int64_t *>(idx)[k] : (int64_t) static_cast<const int32_t *>(idx)[k];
    };
    const int64_t f = flat_at(e);
    // an index outside rows x d_in maps past the last row and touches no row offset
    const int64_t t = (f < 0 || f >= rows * d_in) ? rows : f / d_in;
    col[e] = (uint32_t)(f - t * d_in);
    float v;
    if (bits == 8) {
        v = (float)static_cast<const int8_t *>(data)[e] * scale[0];
    } else if (bits == 4) {
        const uint32_t byte = static_cast<const uint8_t *>(data)[e >> 1];
        int n = (int)((e & 1) ? (byte >> 4) : (byte & 0xfu));
        n = n > 7 ? n - 16 : n;
        v = (float)n * scale[0];
    } else {
        v = load_any(data, val_dt, e);
    }
    val[e] = v;
    int64_t tprev = -1;
    if (e) {
        const int64_t fp = flat_at(e - 1);
        tprev = (fp < 0 || fp >= rows * d_in) ? rows : fp / d_in;
    }
    for (int64_t tt = tprev + 1; tt <= t && tt < rows; ++tt) rowptr[tt] = (uint32_t)e;
    if (e == nnz - 1)
        for (int64_t tt = t < rows ? t + 1 : rows; tt <= rows; ++tt) rowptr[tt] = (uint32_t)nnz;
}

// Partial M[j][o] = sum over a token split of G[t][o] * C[t][j]; row j == R holds sum G[t][o].
template <int DT, int R>
__global__ __launch_bounds__(kBlock) void k_lowrank(const typename Act<DT>::T *__restrict__ g, int64_t rows,
                                                    int64_t d_out, const typename Act<DT>::T *__restrict__ coeff,
                                                    int rank, int64_t tokens_per_split, float *__restrict__ mpart)
{
    using A = Act<DT>;
    __shared__ float s_c[kTokTile][R];
    const int64_t o = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.y * tokens_per_split;
    const int64_t t1 = min(t0 + tokens_per_split, rows);
    float acc[R + 1];
#pragma unroll
    for (int j = 0; j <= R; ++j) acc[j] = 0.f;
    for (int64_t tb = t0; tb < t1; tb += kTokTile) {
        const int nt = (int)min<int64_t>(kTokTile, t1 - tb);
        __syncthreads();
        for (int i = threadIdx.x; i < kTokTile * R; i += kBlock) {
            const int tt = i / R, j = i - tt * R;
            s_c[tt][j] = (tt < nt && j < rank) ? A::ld(coeff[(tb + tt) * rank + j]) : 0.f;
        }
        __syncthreads();
        if (o < d_out) {
            for (int tt = 0; tt < nt; ++tt) {
                const float gv = A::ld(g[(tb + tt) * d_out + o]);
#pragma unroll
                for (int j = 0; j < R; ++j) acc[j] = fmaf(gv, s_c[tt][j], acc[j]);
                acc[R] += gv;
            }
        }
    }
    if (o < d_out) {
        float *mp = mpart + (int64_t)blockIdx.y * (R + 1) * d_out;
#pragma unroll
        for (int j = 0; j <= R; ++j) mp[j * d_out + o] = acc[j];
    }
}

__global__ void k_reduce_m(const float *__restrict__ mpart, int64_t n_splits, int64_t n, float *__restrict__ m)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float s = 0.f;
        for (int64_t k = 0; k < n_splits; ++k) s += mpart[k * n + i];
        m[i] = s;
    }
}

// Sparse term for one (64 x kSparseI) tile of dW, accumulated in LDS.  Each wave owns a quarter
// of the tile's input features and walks every token in order, so each accumulator has a single
// writer and a fixed summation order (deterministic results, no atomics).
template <int DT>
__global__ __launch_bounds__(kBlock) void k_sparse(const typename Act<DT>::T *__restrict__ g, int64_t rows,
                                                   int64_t d_out, int64_t d_in, uint32_t nnz,
                                                   const uint32_t *__restrict__ rowptr,
                                                   const uint32_t *__restrict__ col, const float *__restrict__ val,
                                                   float *__restrict__ s_out, int transposed)
{
    using A = Act<DT>;
    __shared__ float acc[kSparseI * kLdsPitch];
    for (int i = threadIdx.x; i < kSparseI * kLdsPitch; i += kBlock) acc[i] = 0.f;
    __syncthreads();
    const int64_t o0 = (int64_t)blockIdx.x * kSparseO;
    const uint32_t i0 = blockIdx.y * kSparseI;
    const uint32_t i1 = min<uint32_t>(i0 + kSparseI, (uint32_t)d_in);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr uint32_t span = (kSparseI + kWaves - 1) / kWaves;
    const uint32_t w_lo = min<uint32_t>(i0 + wave * span, i1);
    const uint32_t w_hi = min<uint32_t>(w_lo + span, i1);
    const int64_t o = o0 + lane;
    for (int64_t t = 0; t < rows && w_lo < w_hi; ++t) {
        // clamped so that inconsistent offsets (unsorted indices) cannot read past the arrays
        const uint32_t e1 = min(rowptr[t + 1], nnz);
        uint32_t e = min(rowptr[t], e1);
        while (e < e1 && col[e] < w_lo) ++e;
        if (e >= e1 || col[e] >= w_hi) continue;
        const float gv = o < d_out ? A::ld(g[t * d_out + o]) : 0.f;
        for (; e < e1; ++e) {
            const uint32_t c = col[e];
            if (c >= w_hi) break;
            float *a = &acc[(c - i0) * kLdsPitch + lane];
            *a = *a + val[e] * gv;
        }
    }
    __syncthreads();
    const int ni = (int)(i1 - i0);
    if (!transposed) {
        // S[o][i], i fastest
        for (int k = threadIdx.x; k < kSparseO * ni; k += kBlock) {
            const int oo = k / ni, ii = k - oo * ni;
            if (o0 + oo < d_out) s_out[(o0 + oo) * d_in + i0 + ii] = acc[ii * kLdsPitch + oo];
        }
    } else {
        // S^T[i][o], o fastest
        for (int k = threadIdx.x; k < kSparseO * ni; k += kBlock) {
            const int ii = k / kSparseO, oo = k - ii * kSparseO;
            if (o0 + oo < d_out) s_out[(int64_t)(i0 + ii) * d_out + o0 + oo] = acc[ii * kLdsPitch + oo];
        }
    }
}

// dW = M Q^T (+ S) in the output orientation; also writes dbias from row R of M.
template <int R>
__global__ void k_expand(const float *__restrict__ m, const float *__restrict__ qp, const float *__restrict__ s_in,
                         int64_t d_out, int64_t d_in, int transposed, void *__restrict__ dw, int dw_dt,
                         void *__restrict__ dbias, int db_dt)
{
    const int64_t n = d_out * d_in;
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n; k += (int64_t)gridDim.x * blockDim.x) {
        int64_t o, i;
        if (transposed) {
            i = k / d_out;
            o = k - i * d_out;
        } else {
            o = k / d_in;
            i = k - o * d_in;
        }
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < R; ++j) s = fmaf(m[j * d_out + o], qp[i * R + j], s);
        if (s_in) s += s_in[k];
        store_any(dw, dw_dt, k, s);
        if (dbias && k < d_out) store_any(dbias, db_dt, k, m[R * d_out + k]);
    }
}

template <int DT>
__global__ void k_pad_basis_g(const typename Act<DT>::T *__restrict__ q, int64_t d, int rank, int R, float *__restrict__ qp)
{
    const int64_t n = d * R;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / R;
        const int j = (int)(i - row * R);
        qp[i] = j < rank ? Act<DT>::ld(q[row * rank + j]) : 0.f;
    }
}

int pad_rank(int rank) { return rank <= 4 ? 4 : rank <= 8 ? 8 : rank <= 16 ? 16 : 32; }

int grid_for(int64_t n) { return (int)hmin<int64_t>(8192, hmax<int64_t>(1, (n + kBlock - 1) / kBlock)); }

enum { GW_QP, GW_ROWPTR, GW_COL, GW_VAL, GW_MPART, GW_M, GW_S, GW_N };

struct GPlan {
    int R;
    int64_t o_blocks, n_splits, tokens_per_split;
};

GPlan make_gplan(const StacrGradArgs &a)
{
    GPlan p{};
    p.R = pad_rank(a.rank);
    p.o_blocks = (a.d_out + kBlock - 1) / kBlock;
    const int64_t max_splits = hmax<int64_t>(1, (a.rows + kTokTile - 1) / kTokTile);
    p.n_splits = hmin<int64_t>(max_splits, hmax<int64_t>(1, 1024 / p.o_blocks));
    p.tokens_per_split = (a.rows + p.n_splits - 1) / p.n_splits;
    p.tokens_per_split = (p.tokens_per_split + kTokTile - 1) / kTokTile * kTokTile;
    if (p.tokens_per_split < 1) p.tokens_per_split = kTokTile;
    p.n_splits = hmax<int64_t>(1, (a.rows + p.tokens_per_split - 1) / p.tokens_per_split);
    return p;
}

size_t glayout(const StacrGradArgs &a, const GPlan &p, size_t *off)
{
    size_t cur = 0;
    auto take = [&](int slot, size_t bytes) { off[slot] = cur; cur += (bytes + 255) & ~(size_t)255; };
    const bool sp = a.nnz > 0;
    take(GW_QP, (size_t)a.d_in * p.R * sizeof(float));
    take(GW_ROWPTR, sp ? (size_t)(a.rows + 1) * sizeof(uint32_t) : 0);
    take(GW_COL, sp ? (size_t)a.nnz * sizeof(uint32_t) : 0);
    take(GW_VAL, sp ? (size_t)a.nnz * sizeof(float) : 0);
    take(GW_MPART, (size_t)p.n_splits * (p.R + 1) * a.d_out * sizeof(float));
    take(GW_M, (size_t)(p.R + 1) * a.d_out * sizeof(float));
    take(GW_S, sp ? (size_t)a.d_out * a.d_in * sizeof(float) : 0);
    return cur;
}

template <int DT, int R>
int launch_grad(const StacrGradArgs &a, const GPlan &p, char *ws, const size_t *off)
{
    using T = typename Act<DT>::T;
    hipStream_t s = a.stream;
    float *qp = reinterpret_cast<float *>(ws + off[GW_QP]);
    float *mpart = reinterpret_cast<float *>(ws + off[GW_MPART]);
    float *m = reinterpret_cast<float *>(ws + off[GW_M]);
    float *sbuf = nullptr;
    stacr_launch("k_pad_basis_g", s, [&] { k_pad_basis_g<DT><<<grid_for(a.d_in * R), kBlock, 0, s>>>(static_cast<const T *>(a.q), a.d_in, a.rank, R, qp); });
    if (a.rows > 0) {
        dim3 grid((unsigned)p.o_blocks, (unsigned)p.n_splits);
        stacr_launch("k_lowrank", s, [&] { k_lowrank<DT, R><<<grid, kBlock, 0, s>>>(static_cast<const T *>(a.g), a.rows, a.d_out,
                                                 static_cast<const T *>(a.coeff), a.rank, p.tokens_per_split, mpart); });
        stacr_launch("k_reduce_m", s, [&] { k_reduce_m<<<grid_for((R + 1) * a.d_out), kBlock, 0, s>>>(mpart, p.n_splits, (int64_t)(R + 1) * a.d_out, m); });
    } else {
        stacr_launch("k_reduce_m", s, [&] { k_reduce_m<<<grid_for((R + 1) * a.d_out), kBlock, 0, s>>>(mpart, 0, (int64_t)(R + 1) * a.d_out, m); });
    }
    if (a.nnz > 0) {
        uint32_t *rowptr = reinterpret_cast<uint32_t *>(ws + off[GW_ROWPTR]);
        uint32_t *col = reinterpret_cast<uint32_t *>(ws + off[GW_COL]);
        float *val = reinterpret_cast<float *>(ws + off[GW_VAL]);
        sbuf = reinterpret_cast<float *>(ws + off[GW_S]);
        const int cg = (int)((a.nnz + kBlock - 1) / kBlock);
        if (a.index_bytes == 8)
            stacr_launch("k_csr_rows", s, [&] { k_csr_rows<1><<<cg, kBlock, 0, s>>>(a.idx, a.nnz, a.d_in, a.rows, a.data, a.scale, a.bits, a.val_dtype,
                                               rowptr, col, val); });
        else
            stacr_launch("k_csr_rows", s, [&] { k_csr_rows<0><<<cg, kBlock, 0, s>>>(a.idx, a.nnz, a.d_in, a.rows, a.data, a.scale, a.bits, a.val_dtype,
                                               rowptr, col, val); });
        dim3 grid((unsigned)((a.d_out + kSparseO - 1) / kSparseO), (unsigned)((a.d_in + kSparseI - 1) / kSparseI));
        stacr_launch("k_sparse", s, [&] { k_sparse<DT><<<grid, kBlock, 0, s>>>(static_cast<const T *>(a.g), a.rows, a.d_out, a.d_in, (uint32_t)a.nnz,
                                             rowptr, col, val,
                                             sbuf, a.transposed); });
    }
    stacr_launch("k_expand", s, [&] { k_expand<R><<<grid_for(a.d_out * a.d_in), kBlock, 0, s>>>(m, qp, sbuf, a.d_out, a.d_in, a.transposed, a.dw,
                                                             a.dw_dtype, a.dbias, a.dbias_dtype); });
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
