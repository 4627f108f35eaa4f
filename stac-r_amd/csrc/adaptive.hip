// Adaptive-engine pieces around the save / weight-gradient kernels:
//   * per-tensor quantizers with the scale in the tensor's own dtype (stacr/adaptive.py:44-135)
//   * CSR and delta index codecs (stacr/index_compression.py:193-345)
//   * the residual-energy and per-rank coefficient-energy sums of the adaptive forward
//     (stacr/adaptive.py:1388-1393,1953-1958)
#include <float.h>

#include "internal.h"

using namespace stacr;

namespace {

// ------------------------------------------------------------------ dtype-native arithmetic
__device__ __forceinline__ float rnd_dt(int dt, float f)
{
    if (dt == STACR_DTYPE_BF16) return bf16_bits_to_f(f_to_bf16_bits(f));
    if (dt == STACR_DTYPE_F16) return f16_bits_to_f(f_to_f16_bits(f));
    return f;
}

// Scale record shared by the quantizer and dequantizer: the value and the dtype it lives in.
// code = STACR_DTYPE_* of the input normally; STACR_DTYPE_F32 when a 16-bit scale underflowed
// and the reference recomputed it in fp32; STACR_SCALE_F64 when an fp32 scale underflowed.
struct ScaleRec {
    double value;
    int32_t code;
    int32_t pad;
};

struct QScale {
    int mode;      // 0: all zero; 1: dtype-native scale; 2: fp32 (promoted); 3: fp64 (promoted)
    float s;       // modes 1, 2
    double s64;    // mode 3
};

__device__ __forceinline__ QScale quant_scale_dt(int dt, uint32_t amax_bits, float qmax)
{
    QScale q{};
    const float amax = __uint_as_float(amax_bits);
    const float s = rnd_dt(dt, __fdiv_rn(amax, qmax));
    if (s == 0.f) {
        if (amax == 0.f) {
            q.mode = 0;
        } else if (dt != STACR_DTYPE_F32) {
            q.mode = 2;
            q.s = __fdiv_rn(amax, qmax);
        } else {
            q.mode = 3;
            q.s64 = __ddiv_rn((double)amax, (double)qmax);
        }
    } else {
        q.mode = 1;
        q.s = s;
    }
    return q;
}

// round(v / scale) clamped to [-qmax, qmax], in the arithmetic the reference uses for the mode.
__device__ __forceinline__ int quant_one_dt(int dt, const QScale &q, float v, float qmax)
{
    if (q.mode == 0) return 0;
    float t;
    if (q.mode == 1) {
        t = rintf(rnd_dt(dt, __fdiv_rn(v, q.s)));
    } else if (q.mode == 2) {
        t = rintf(__fdiv_rn(v, q.s));
    } else {
        const double d = rint(__ddiv_rn((double)v, q.s64));
        t = (float)fmin(fmax(d, -(double)qmax), (double)qmax);
    }
    t = fminf(fmaxf(t, -qmax), qmax);
    return (int)t;
}

// Largest |v| as fp32 bits (NaN sorts above inf, as the integer order of the bits gives): per
// workgroup, then one device atomic per workgroup (the grid is capped, so few reach one address).
constexpr int kAmaxWgs = 256;
__global__ __launch_bounds__(kBlock) void k_aq_amax(const void *__restrict__ v, int dt, int64_t n,
                                                    uint32_t *__restrict__ amax)
{
    __shared__ uint32_t s_m[kWaves];
    uint32_t m = 0u;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        m = max(m, __float_as_uint(load_any(v, dt, i)) & 0x7fffffffu);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t b = s_m[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) b = max(b, s_m[w]);
        if (b) atomicMax(amax, b);
    }
}

// bits 8: one int8 per value.  bits 4: (q + 8) nibbles, even entry low, odd length padded with 8.
__global__ void k_aq_quant(const void *__restrict__ v, int dt, int64_t n, int bits,
                           const uint32_t *__restrict__ amax, void *__restrict__ data, ScaleRec *__restrict__ scale)
{
    const float qmax = bits == 4 ? 7.f : 127.f;
    const QScale q = quant_scale_dt(dt, *amax, qmax);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        ScaleRec r{};
        if (q.mode == 0) { r.value = 1.0; r.code = dt; }
        else if (q.mode == 1) { r.value = q.s; r.code = dt; }
        else if (q.mode == 2) { r.value = q.s; r.code = STACR_DTYPE_F32; }
        else { r.value = q.s64; r.code = STACR_SCALE_F64; }
        *scale = r;
    }
    if (bits == 8) {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
            static_cast<int8_t *>(data)[i] = (int8_t)quant_one_dt(dt, q, load_any(v, dt, i), qmax);
    } else {
        const int64_t nb = (n + 1) / 2;
        for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
            const int lo = quant_one_dt(dt, q, load_any(v, dt, 2 * b), qmax) + 8;
            const int hi = 2 * b + 1 < n ? quant_one_dt(dt, q, load_any(v, dt, 2 * b + 1), qmax) + 8 : 8;
            static_cast<uint8_t *>(data)[b] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// data.to(scale dtype) * scale, then to the output dtype (stacr/adaptive.py:79-90,123-131).
__global__ void k_aq_dequant(const void *__restrict__ data, int bits, const ScaleRec *__restrict__ scale, int64_t n,
                             void *__restrict__ out, int out_dt)
{
    const ScaleRec r = *scale;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        int qv;
        if (bits == 8) {
            qv = static_cast<const int8_t *>(data)[i];
        } else {
            const uint32_t byte = static_cast<const uint8_t *>(data)[i >> 1];
            qv = (int)((i & 1) ? (byte >> 4) & 0xfu : byte & 0xfu) - 8;
        }
        float y;
        if (r.code == STACR_SCALE_F64) {
            y = (float)((double)qv * r.value);
        } else {
            y = rnd_dt(r.code, (float)qv * (float)r.value);
        }
        store_any(out, out_dt, i, y);
    }
}

// ------------------------------------------------------------------ index codecs
__device__ __forceinline__ int64_t ld_int(const void *p, int bytes, int64_t i)
{
    if (bytes == 8) return static_cast<const int64_t *>(p)[i];
    if (bytes == 4) return static_cast<const int32_t *>(p)[i];
    return static_cast<const int16_t *>(p)[i];
}

__device__ __forceinline__ void st_int(void *p, int bytes, int64_t i, int64_t v)
{
    if (bytes == 8) static_cast<int64_t *>(p)[i] = v;
    else if (bytes == 4) static_cast<int32_t *>(p)[i] = (int32_t)v;
    else static_cast<int16_t *>(p)[i] = (int16_t)v;
}

// CSR of row-sorted flat indices: ptr[t] = entries with row < t (t = 0..rows), col = idx mod N.
__global__ void k_csr_encode(const void *__restrict__ idx, int idx_bytes, int64_t nnz, int64_t rows, int64_t n_cols,
                             void *__restrict__ ptr, int ptr_bytes, void *__restrict__ cols, int col_bytes)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    const int64_t f = ld_int(idx, idx_bytes, e);
    const int64_t t = min(max(f / n_cols, (int64_t)0), rows);
    st_int(cols, col_bytes, e, f - (f / n_cols) * n_cols);
    const int64_t tprev = e ? min(max(ld_int(idx, idx_bytes, e - 1) / n_cols, (int64_t)0), rows) : -1;
    for (int64_t tt = tprev + 1; tt <= t; ++tt) st_int(ptr, ptr_bytes, tt, e);
    if (e == nnz - 1)
        for (int64_t tt = t + 1; tt <= rows; ++tt) st_int(ptr, ptr_bytes, tt, nnz);
}

__global__ void k_fill_int(void *__restrict__ p, int bytes, int64_t n, int64_t v)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        st_int(p, bytes, i, v);
}

// idx[e] = row(e) * N + col[e], row(e) found by binary search in ptr.
__global__ void k_csr_decode(const void *__restrict__ ptr, int ptr_bytes, const void *__restrict__ cols, int col_bytes,
                             int64_t rows, int64_t n_cols, int64_t nnz, void *__restrict__ idx, int idx_bytes)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    int64_t lo = 0, hi = rows;  // last t with ptr[t] <= e
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) / 2;
        if (ld_int(ptr, ptr_bytes, mid) <= e) lo = mid;
        else hi = mid;
    }
    st_int(idx, idx_bytes, e, lo * n_cols + ld_int(cols, col_bytes, e));
}

// Largest gap between consecutive indices (the indices are sorted, so gaps are >= 0).
__global__ void k_delta_max(const void *__restrict__ idx, int idx_bytes, int64_t nnz, unsigned long long *__restrict__ out)
{
    unsigned long long m = 0ull;
    for (int64_t e = 1 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nnz; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t d = ld_int(idx, idx_bytes, e) - ld_int(idx, idx_bytes, e - 1);
        m = max(m, (unsigned long long)(d < 0 ? 0 : d));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(m, off, 64);
        m = max(m, o);
    }
    if ((threadIdx.x & 63) == 0 && m) atomicMax(out, m);
}

__global__ void k_delta_encode(const void *__restrict__ idx, int idx_bytes, int64_t nnz, void *__restrict__ base,
                               int base_bytes, void *__restrict__ deltas, int delta_bytes)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    const int64_t f = ld_int(idx, idx_bytes, e);
    if (e == 0) st_int(base, base_bytes, 0, f);
    else st_int(deltas, delta_bytes, e - 1, f - ld_int(idx, idx_bytes, e - 1));
}

constexpr int kScanBlock = 4096;  // entries per workgroup in the delta decode scan

// Pass 1 of the decode scan: the sum of each block's deltas.
__global__ __launch_bounds__(kBlock) void k_delta_block_sums(const void *__restrict__ deltas, int delta_bytes,
                                                             int64_t n_deltas, int64_t *__restrict__ sums)
{
    __shared__ long long s_part[kWaves];
    const int64_t b0 = (int64_t)blockIdx.x * kScanBlock;
    long long s = 0;
    for (int64_t i = b0 + threadIdx.x; i < min(b0 + kScanBlock, n_deltas); i += kBlock) s += ld_int(deltas, delta_bytes, i);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long t = 0;
        for (int w = 0; w < kWaves; ++w) t += s_part[w];
        sums[blockIdx.x] = t;
    }
}

// Pass 2: idx[0] = base; idx[e] = base + (sum of deltas[0..e-1]).
__global__ __launch_bounds__(kBlock) void k_delta_decode(const void *__restrict__ base, int base_bytes,
                                                         const void *__restrict__ deltas, int delta_bytes,
                                                         int64_t nnz, const int64_t *__restrict__ sums,
                                                         void *__restrict__ idx, int idx_bytes)
{
    __shared__ long long s_wave[kWaves];
    __shared__ long long s_carry;
    const int64_t n_deltas = nnz - 1;
    const int64_t b0 = (int64_t)blockIdx.x * kScanBlock;
    if (threadIdx.x == 0) {
        long long c = ld_int(base, base_bytes, 0);
        for (int64_t b = 0; b < blockIdx.x; ++b) c += sums[b];
        s_carry = c;
        if (blockIdx.x == 0) st_int(idx, idx_bytes, 0, c);
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t c0 = b0; c0 < min(b0 + kScanBlock, n_deltas); c0 += kBlock) {
        const int64_t i = c0 + threadIdx.x;
        const long long v = i < n_deltas ? ld_int(deltas, delta_bytes, i) : 0;
        long long x = v;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const long long y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) s_wave[wave] = x;
        __syncthreads();
        long long before = 0, tot = 0;
        for (int w = 0; w < kWaves; ++w) {
            before += w < wave ? s_wave[w] : 0;
            tot += s_wave[w];
        }
        const long long carry = s_carry;
        if (i < n_deltas) st_int(idx, idx_bytes, i + 1, carry + before + x);
        __syncthreads();
        if (threadIdx.x == 0) s_carry = carry + tot;
        __syncthreads();
    }
}

// ------------------------------------------------------------------ energies
// Per workgroup: sum of rnd(x^2), sum of rnd(c^2) (products rounded to the activation dtype, as a
// dtype-native multiply does) and sum over rows of fp32 c_j^2 per rank.  Deterministic: partial
// sums per workgroup, then one workgroup adds them in order.
constexpr int kEnergyWgs = 512;

__global__ __launch_bounds__(kBlock) void k_energy_partial(const void *__restrict__ x, const void *__restrict__ c, int dt,
                                                           int64_t rows, int64_t feats, int rank,
                                                           float *__restrict__ part)
{
    __shared__ float s_red[kWaves][2 + STACR_MAX_RANK];
    const int64_t nx = rows * feats, nc = rows * rank;
    float sx = 0.f, sc = 0.f;
    float sr[STACR_MAX_RANK];
#pragma unroll
    for (int j = 0; j < STACR_MAX_RANK; ++j) sr[j] = 0.f;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nx; i += stride) {
        const float v = load_any(x, dt, i);
        sx += rnd_dt(dt, v * v);
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nc; i += stride) {
        const float v = load_any(c, dt, i);
        sc += rnd_dt(dt, v * v);
        const int j = (int)(i % rank);
#pragma unroll
        for (int jj = 0; jj < STACR_MAX_RANK; ++jj)
            if (jj == j) sr[jj] = fmaf(v, v, sr[jj]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        sx += __shfl_xor(sx, off, 64);
        sc += __shfl_xor(sc, off, 64);
#pragma unroll
        for (int j = 0; j < STACR_MAX_RANK; ++j) sr[j] += __shfl_xor(sr[j], off, 64);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        s_red[wave][0] = sx;
        s_red[wave][1] = sc;
#pragma unroll
        for (int j = 0; j < STACR_MAX_RANK; ++j) s_red[wave][2 + j] = sr[j];
    }
    __syncthreads();
    if (threadIdx.x < 2 + rank) {
        float t = 0.f;
        for (int w = 0; w < kWaves; ++w) t += s_red[w][threadIdx.x];
        part[(int64_t)blockIdx.x * (2 + STACR_MAX_RANK) + threadIdx.x] = t;
    }
}

// out[0] = residual energy sqrt(max(|X|^2 - |C|^2, 0)) / (sqrt(|X|^2) + 1e-8) in the activation
// dtype's arithmetic; out[1] = |X|^2, out[2] = |C|^2 (rounded to the dtype as torch's dtype-native
// sum returns them); out[3 + j] = mean over rows of c_j^2 in fp32.
__global__ void k_energy_final(const float *__restrict__ part, int nwg, int dt, int64_t rows, int rank,
                               float *__restrict__ out)
{
    const int t = threadIdx.x;
    if (t >= 2 + rank) return;
    float s = 0.f;  // partial sums added in a fixed order
    for (int w = 0; w < nwg; ++w) s += part[(int64_t)w * (2 + STACR_MAX_RANK) + t];
    if (t >= 2) out[3 + (t - 2)] = rows ? __fdiv_rn(s, (float)rows) : 0.f;
    else out[1 + t] = rnd_dt(dt, s);
}

__global__ void k_energy_ratio(int dt, float *__restrict__ out)
{
    const float x2 = out[1], c2 = out[2];
    const float d0 = rnd_dt(dt, x2 - c2);
    const float diff = isnan(d0) ? d0 : fmaxf(d0, 0.f);  // torch.clamp keeps NaN
    const float num = rnd_dt(dt, __fsqrt_rn(diff));
    const float den = rnd_dt(dt, rnd_dt(dt, __fsqrt_rn(x2)) + 1e-8f);
    out[0] = rnd_dt(dt, __fdiv_rn(num, den));
}

// The energies from a save's per-workgroup partials ([kEnergyStride] each: sum of rnd(x^2), sum of
// rnd(c^2), sum of c_j^2 per basis column), with out[] as k_energy_final and k_energy_ratio write it.
// Thread (value v, stripe st) adds partials st, st + 16, ... in order, 16 loads at a time; the 16
// stripes are then added in order.
constexpr int kFoldStripes = 16;
constexpr int kFoldSlices = 64;  // first stage: workgroups, each over a contiguous slice of partials

// First stage: workgroup b adds the partials of its slice (stripes of 16 in order, then the stripes
// in order) into part2[b] ([kEnergyStride]).
__global__ __launch_bounds__(1024) void k_energy_fold_slices(const float *__restrict__ part, int64_t n, int rank,
                                                             float *__restrict__ part2)
{
    __shared__ float s_t[kFoldStripes][64];
    const int v = threadIdx.x & 63, st = threadIdx.x >> 6;
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t w0 = (int64_t)blockIdx.x * per, w1 = w0 + per < n ? w0 + per : n;
    float t = 0.f;
    if (v < 2 + rank) {
        for (int64_t c0 = w0 + st; c0 < w1; c0 += 16 * kFoldStripes) {
            float vals[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const int64_t w = c0 + (int64_t)c * kFoldStripes;
                vals[c] = w < w1 ? part[w * kEnergyStride + v] : 0.f;
            }
#pragma unroll
            for (int c = 0; c < 16; ++c) t += vals[c];
        }
    }
    s_t[st][v] = t;
    __syncthreads();
    if (threadIdx.x < kEnergyStride) {
        float sum = 0.f;
        for (int j = 0; j < kFoldStripes; ++j) sum += s_t[j][threadIdx.x];
        part2[(int64_t)blockIdx.x * kEnergyStride + threadIdx.x] = sum;
    }
}

__global__ __launch_bounds__(1024) void k_energy_fold(const float *__restrict__ part, int64_t n, int dt, int64_t rows,
                                                      int rank, float *__restrict__ out)
{
    __shared__ float s_t[64][kFoldStripes];
    __shared__ float s_sum[2];
    const int v = threadIdx.x / kFoldStripes, st = threadIdx.x % kFoldStripes;
    float t = 0.f;
    if (v < 2 + rank) {
        for (int64_t w0 = st; w0 < n; w0 += 16 * kFoldStripes) {
            float vals[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const int64_t w = w0 + (int64_t)c * kFoldStripes;
                vals[c] = w < n ? part[w * kEnergyStride + v] : 0.f;
            }
#pragma unroll
            for (int c = 0; c < 16; ++c) t += vals[c];
        }
    }
    s_t[v][st] = t;
    __syncthreads();
    const int k = threadIdx.x;
    if (k < 2 + rank) {
        float sum = 0.f;
        for (int j = 0; j < kFoldStripes; ++j) sum += s_t[k][j];
        if (k >= 2) out[3 + (k - 2)] = rows ? __fdiv_rn(sum, (float)rows) : 0.f;
        else s_sum[k] = rnd_dt(dt, sum);
    }
    __syncthreads();
    if (k == 0) {
        const float x2 = s_sum[0], c2 = s_sum[1];
        out[1] = x2;
        out[2] = c2;
        const float d0 = rnd_dt(dt, x2 - c2);
        const float diff = isnan(d0) ? d0 : fmaxf(d0, 0.f);  // torch.clamp keeps NaN
        const float num = rnd_dt(dt, __fsqrt_rn(diff));
        const float den = rnd_dt(dt, rnd_dt(dt, __fsqrt_rn(x2)) + 1e-8f);
        out[0] = rnd_dt(dt, __fdiv_rn(num, den));
    }
}

int blocks_for(int64_t n) { return (int)hmax<int64_t>(1, hmin<int64_t>((n + kBlock - 1) / kBlock, 4096)); }

}  // namespace

// ------------------------------------------------------------------ launchers
int stacr_aq_quantize_launch(const void *v, int dtype, int64_t n, int bits, void *data, void *scale, void *ws,
                             hipStream_t s)
{
    uint32_t *amax = static_cast<uint32_t *>(ws);
    stacr_launch("k_fill_int", s, [&] { k_fill_int<<<1, 64, 0, s>>>(amax, 4, 1, 0); });
    if (n > 0)
        stacr_launch("k_aq_amax", s, [&] {
            k_aq_amax<<<hmin(blocks_for(n), kAmaxWgs), kBlock, 0, s>>>(v, dtype, n, amax);
        });
    const int64_t work = bits == 4 ? (n + 1) / 2 : n;
    stacr_launch("k_aq_quant", s, [&] {
        k_aq_quant<<<blocks_for(work), kBlock, 0, s>>>(v, dtype, n, bits, amax, data, static_cast<ScaleRec *>(scale));
    });
    return stacr_hip_check(hipGetLastError(), "adaptive quantizer");
}

int stacr_fill_int_launch(void *p, int bytes, int64_t n, int64_t v, hipStream_t s)
{
    if (n > 0) stacr_launch("k_fill_int", s, [&] { k_fill_int<<<blocks_for(n), kBlock, 0, s>>>(p, bytes, n, v); });
    return stacr_hip_check(hipGetLastError(), "fill");
}

int stacr_aq_dequantize_launch(const void *data, int bits, const void *scale, int64_t n, void *out, int out_dt,
                               hipStream_t s)
{
    if (n > 0)
        stacr_launch("k_aq_dequant", s, [&] {
            k_aq_dequant<<<blocks_for(n), kBlock, 0, s>>>(data, bits, static_cast<const ScaleRec *>(scale), n, out, out_dt);
        });
    return stacr_hip_check(hipGetLastError(), "adaptive dequantizer");
}

int stacr_csr_encode_launch(const void *idx, int idx_bytes, int64_t nnz, int64_t rows, int64_t n_cols, void *ptr,
                            int ptr_bytes, void *cols, int col_bytes, hipStream_t s)
{
    if (nnz == 0) {
        stacr_launch("k_fill_int", s, [&] { k_fill_int<<<blocks_for(rows + 1), kBlock, 0, s>>>(ptr, ptr_bytes, rows + 1, 0); });
    } else {
        stacr_launch("k_csr_encode", s, [&] {
            k_csr_encode<<<(int)((nnz + kBlock - 1) / kBlock), kBlock, 0, s>>>(idx, idx_bytes, nnz, rows, n_cols, ptr,
                                                                            ptr_bytes, cols, col_bytes);
        });
    }
    return stacr_hip_check(hipGetLastError(), "csr encode");
}

int stacr_csr_decode_launch(const void *ptr, int ptr_bytes, const void *cols, int col_bytes, int64_t rows,
                            int64_t n_cols, int64_t nnz, void *idx, int idx_bytes, hipStream_t s)
{
    if (nnz > 0)
        stacr_launch("k_csr_decode", s, [&] {
            k_csr_decode<<<(int)((nnz + kBlock - 1) / kBlock), kBlock, 0, s>>>(ptr, ptr_bytes, cols, col_bytes, rows,
                                                                            n_cols, nnz, idx, idx_bytes);
        });
    return stacr_hip_check(hipGetLastError(), "csr decode");
}

int stacr_delta_max_launch(const void *idx, int idx_bytes, int64_t nnz, void *out, hipStream_t s)
{
    stacr_launch("k_fill_int", s, [&] { k_fill_int<<<1, 64, 0, s>>>(out, 8, 1, 0); });
    if (nnz > 1)
        stacr_launch("k_delta_max", s, [&] {
            k_delta_max<<<blocks_for(nnz), kBlock, 0, s>>>(idx, idx_bytes, nnz, static_cast<unsigned long long *>(out));
        });
    return stacr_hip_check(hipGetLastError(), "delta max");
}

int stacr_delta_encode_launch(const void *idx, int idx_bytes, int64_t nnz, void *base, int base_bytes, void *deltas,
                              int delta_bytes, hipStream_t s)
{
    if (nnz > 0)
        stacr_launch("k_delta_encode", s, [&] {
            k_delta_encode<<<(int)((nnz + kBlock - 1) / kBlock), kBlock, 0, s>>>(idx, idx_bytes, nnz, base, base_bytes,
                                                                              deltas, delta_bytes);
        });
    return stacr_hip_check(hipGetLastError(), "delta encode");
}

size_t stacr_delta_decode_ws(int64_t nnz) { return (size_t)hmax<int64_t>(1, (nnz - 1 + kScanBlock - 1) / kScanBlock) * 8; }

int stacr_delta_decode_launch(const void *base, int base_bytes, const void *deltas, int delta_bytes, int64_t nnz,
                              void *idx, int idx_bytes, void *ws, hipStream_t s)
{
    if (nnz <= 0) return STACR_OK;
    const int64_t nd = nnz - 1;
    const int nb = (int)hmax<int64_t>(1, (nd + kScanBlock - 1) / kScanBlock);
    int64_t *sums = static_cast<int64_t *>(ws);
    if (nd > 0)
        stacr_launch("k_delta_block_sums", s, [&] { k_delta_block_sums<<<nb, kBlock, 0, s>>>(deltas, delta_bytes, nd, sums); });
    stacr_launch("k_delta_decode", s, [&] {
        k_delta_decode<<<nb, kBlock, 0, s>>>(base, base_bytes, deltas, delta_bytes, nnz, sums, idx, idx_bytes);
    });
    return stacr_hip_check(hipGetLastError(), "delta decode");
}

size_t stacr_energy_ws() { return (size_t)kEnergyWgs * (2 + STACR_MAX_RANK) * sizeof(float); }

int stacr_energy_launch(const void *x, const void *c, int dtype, int64_t rows, int64_t feats, int rank, float *out,
                        void *ws, hipStream_t s)
{
    float *part = static_cast<float *>(ws);
    stacr_launch("k_energy_partial", s, [&] {
        k_energy_partial<<<kEnergyWgs, kBlock, 0, s>>>(x, c, dtype, rows, feats, rank, part);
    });
    stacr_launch("k_energy_final", s, [&] { k_energy_final<<<1, 64, 0, s>>>(part, kEnergyWgs, dtype, rows, rank, out); });
    stacr_launch("k_energy_ratio", s, [&] { k_energy_ratio<<<1, 1, 0, s>>>(dtype, out); });
    return stacr_hip_check(hipGetLastError(), "energy");
}

size_t stacr_energy_fold_ws() { return (size_t)kFoldSlices * kEnergyStride * sizeof(float); }

int stacr_energy_fold_launch(const float *part, int64_t n, int dtype, int64_t rows, int rank, float *out, void *ws,
                             hipStream_t s)
{
    if (n > 4 * kFoldSlices) {  // many partials: 64 slices in parallel first
        float *part2 = static_cast<float *>(ws);
        stacr_launch("k_energy_fold_slices", s, [&] {
            k_energy_fold_slices<<<kFoldSlices, 1024, 0, s>>>(part, n, rank, part2);
        });
        part = part2;
        n = kFoldSlices;
    }
    stacr_launch("k_energy_fold", s, [&] { k_energy_fold<<<1, 1024, 0, s>>>(part, n, dtype, rows, rank, out); });
    return stacr_hip_check(hipGetLastError(), "energy fold");
}
