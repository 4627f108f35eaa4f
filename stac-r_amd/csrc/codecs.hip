// Compact forms of a save's outputs: a bit-packed delta stream of the residual indices and int8
// coefficients with one scale per row.  The reference keeps flat int32 indices (stacr/layers.py:41)
// and byte-wide delta / CSR codecs (stacr/index_compression.py:193-269); these are denser forms of
// the same data, decoded back exactly (indices) or by the stated rule (coefficients).
//
// Index stream.  Sorted (non-decreasing, non-negative) flat indices are cut into blocks of 256.
// Block b keeps base[b] = idx[256 b] (int64) and its entries' deltas d_0 = 0,
// d_j = idx[256 b + j] - idx[256 b + j - 1], each stored in w_b bits, w_b the bit length of the
// block's largest delta (0 when every delta is 0).  The block's 256 slots take 256 w_b bits =
// 8 w_b words; slot j sits at bits [j w_b, (j + 1) w_b) of the block's words, least significant bit
// first (bit k in word k / 32 at position k % 32); slots past the last entry are 0.  word_off[b]
// is the block's first word (word_off[0] = 0, word_off[nb] the stream's length), so w_b =
// (word_off[b + 1] - word_off[b]) / 8.  Decoding is base[b] plus the block's inclusive prefix sum
// of the deltas: the sorted indices again (decompress_indices' delta rule, :327-342, base plus
// cumulative deltas).  Three launches encode: per-block widths and flags, one workgroup's prefix
// sum of the word counts, the packing; one launch decodes.  Every block is one workgroup of 256
// threads, thread j owning slot j.
//
// Row-quantized coefficients.  Per row r of C (rows x rank): m = max_j |c_rj| in fp32 (NaN if any
// entry is NaN), s_r = (m finite and > 0 ? m : 1) / 127, q_rj = clamp(round_half_even(c_rj / s_r),
// -127, 127) (a NaN quotient gives 0); dequantized c_rj = q_rj * s_r in fp32, rounded once to the
// output dtype.  The safe-scale rule is the C1 checkpoint codec's (stacr/protocols/checkpointing.py:
// 374-393), taken per row instead of per basis component.
#include "internal.h"

using namespace stacr;

namespace {

constexpr int kStreamBlock = 256;   // entries per block (= threads per workgroup)
constexpr int kScanThreads = 1024;  // the word-count prefix sum runs in one workgroup
// flag bits of a block's word count (bits 28..30) and of the stream status
constexpr uint32_t kFlagUnsorted = 1u, kFlagWide = 2u, kFlagNegative = 4u;
constexpr int kFlagShift = 28;

__device__ __forceinline__ int64_t load_index(const void *idx, int idx64, int64_t e)
{
    return idx64 ? static_cast<const int64_t *>(idx)[e] : (int64_t) static_cast<const int32_t *>(idx)[e];
}

// Slot j's delta and the flags it raises (a delta that cannot be stored is 0 in the stream).
__device__ __forceinline__ uint32_t slot_delta(const void *idx, int idx64, int64_t nnz, int64_t b, int j,
                                               int64_t *value, uint32_t *flags)
{
    const int64_t e = b * kStreamBlock + j;
    *flags = 0u;
    *value = 0;
    if (e >= nnz) return 0u;
    const int64_t v = load_index(idx, idx64, e);
    const int64_t prev = j > 0 ? load_index(idx, idx64, e - 1) : v;
    *value = v;
    const int64_t d = v - prev;
    if (v < 0) *flags |= kFlagNegative;
    if (d < 0) *flags |= kFlagUnsorted;
    if (d > (int64_t)0xffffffffLL) *flags |= kFlagWide;
    return (d < 0 || d > (int64_t)0xffffffffLL) ? 0u : (uint32_t)d;
}

__device__ __forceinline__ uint32_t bit_length(uint32_t v) { return v ? 32u - (uint32_t)__clz((int)v) : 0u; }

// Per block: base[b], and 8 w_b | flags << 28 into word_off[b + 1] (the scan turns the counts
// into offsets).
__global__ __launch_bounds__(kStreamBlock) void k_stream_width(const void *__restrict__ idx, int idx64, int64_t nnz,
                                                               int64_t *__restrict__ base,
                                                               uint32_t *__restrict__ word_off)
{
    __shared__ uint32_t s_max[kStreamBlock / 64], s_flags[kStreamBlock / 64];
    const int64_t b = blockIdx.x;
    const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
    int64_t v;
    uint32_t flags;
    uint32_t d = slot_delta(idx, idx64, nnz, b, j, &v, &flags);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        d = max(d, (uint32_t)__shfl_xor((int)d, off, 64));
        flags |= (uint32_t)__shfl_xor((int)flags, off, 64);
    }
    if (lane == 0) {
        s_max[wave] = d;
        s_flags[wave] = flags;
    }
    __syncthreads();
    if (j == 0) {
        uint32_t m = 0u, f = 0u;
#pragma unroll
        for (int w = 0; w < kStreamBlock / 64; ++w) {
            m = max(m, s_max[w]);
            f |= s_flags[w];
        }
        base[b] = v;
        word_off[b + 1] = 8u * bit_length(m) | f << kFlagShift;
    }
}

// One workgroup: word_off[1..nb] from word counts to inclusive sums (in place, each thread over
// its own run of blocks), word_off[0] = 0, and the OR of the blocks' flags into *status.
__global__ __launch_bounds__(kScanThreads) void k_stream_offsets(int64_t nb, uint32_t *__restrict__ word_off,
                                                                 uint32_t *__restrict__ status)
{
    __shared__ uint32_t s_tot[kScanThreads / 64];
    const int t = threadIdx.x;
    const int64_t seg = (nb + kScanThreads - 1) / kScanThreads;
    const int64_t lo = min((int64_t)t * seg, nb), hi = min(lo + seg, nb);
    uint32_t sum = 0u, flags = 0u;
    for (int64_t i = lo; i < hi; ++i) {
        const uint32_t c = word_off[1 + i];
        sum += c & ((1u << kFlagShift) - 1u);
        flags |= c >> kFlagShift;
    }
    uint32_t total;
    uint32_t run = block_exclusive_scan<kScanThreads>(sum, s_tot, &total);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) flags |= (uint32_t)__shfl_xor((int)flags, off, 64);
    if ((t & 63) == 0) s_tot[t >> 6] = flags;
    __syncthreads();
    for (int64_t i = lo; i < hi; ++i) {
        run += word_off[1 + i] & ((1u << kFlagShift) - 1u);
        word_off[1 + i] = run;
    }
    if (t == 0) {
        uint32_t f = 0u;
#pragma unroll
        for (int w = 0; w < kScanThreads / 64; ++w) f |= s_tot[w];
        word_off[0] = 0u;
        *status = f;
    }
}

// Per block: the deltas OR-ed into the block's words in LDS, then written out by the first 8 w_b
// threads.
__global__ __launch_bounds__(kStreamBlock) void k_stream_pack(const void *__restrict__ idx, int idx64, int64_t nnz,
                                                              const uint32_t *__restrict__ word_off,
                                                              uint32_t *__restrict__ words)
{
    __shared__ uint32_t s_w[kStreamBlock];  // 8 w_b <= 256 words
    const int64_t b = blockIdx.x;
    const int j = threadIdx.x;
    const uint32_t off = word_off[b], w = (word_off[b + 1] - off) / 8u;
    int64_t v;
    uint32_t flags;
    const uint32_t d = slot_delta(idx, idx64, nnz, b, j, &v, &flags);
    s_w[j] = 0u;
    __syncthreads();
    if (w > 0u && d != 0u) {  // d < 2^w by the choice of w
        const uint32_t pos = (uint32_t)j * w, word = pos >> 5, sh = pos & 31u;
        atomicOr(&s_w[word], d << sh);
        if (sh + w > 32u) atomicOr(&s_w[word + 1], d >> (32u - sh));
    }
    __syncthreads();
    if ((uint32_t)j < 8u * w) words[off + j] = s_w[j];
}

// Inclusive prefix sum of 64-bit values over the workgroup.
__device__ __forceinline__ uint64_t block_inclusive_scan64(uint64_t v, uint64_t *s_tot)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t y = __shfl_up(v, off, 64);
        if (lane >= off) v += y;
    }
    if (lane == 63) s_tot[wave] = v;
    __syncthreads();
    uint64_t before = 0u;
#pragma unroll
    for (int w = 0; w < kStreamBlock / 64; ++w) before += w < wave ? s_tot[w] : 0u;
    return before + v;
}

__global__ __launch_bounds__(kStreamBlock) void k_stream_unpack(const int64_t *__restrict__ base,
                                                                const uint32_t *__restrict__ word_off,
                                                                const uint32_t *__restrict__ words, int64_t nnz,
                                                                void *__restrict__ out, int out64)
{
    __shared__ uint64_t s_tot[kStreamBlock / 64];
    const int64_t b = blockIdx.x;
    const int j = threadIdx.x;
    const uint32_t off = word_off[b], w = (word_off[b + 1] - off) / 8u;
    uint32_t d = 0u;
    if (w > 0u) {  // the slot's bits lie inside the block's 8 w words
        const uint32_t pos = (uint32_t)j * w, word = pos >> 5, sh = pos & 31u;
        uint64_t bits = words[off + word] >> sh;
        if (sh + w > 32u) bits |= (uint64_t)words[off + word + 1] << (32u - sh);
        d = (uint32_t)(bits & (w == 32u ? 0xffffffffull : ((1ull << w) - 1ull)));
    }
    const uint64_t s = block_inclusive_scan64(d, s_tot);
    const int64_t e = b * kStreamBlock + j;
    if (e < nnz) {
        const int64_t v = base[b] + (int64_t)s;
        if (out64) static_cast<int64_t *>(out)[e] = v;
        else static_cast<int32_t *>(out)[e] = (int32_t)v;
    }
}

// ------------------------------------------------------------------ row-quantized coefficients
constexpr int kRowThreads = 256;

template <int DT>
__global__ __launch_bounds__(kRowThreads) void k_rows_quantize(const typename Act<DT>::T *__restrict__ c, int64_t rows,
                                                               int rank, int8_t *__restrict__ codes,
                                                               float *__restrict__ scales)
{
    const int64_t r = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    if (r >= rows) return;
    const typename Act<DT>::T *row = c + r * rank;
    float m = 0.f;
    bool nan = false;
    for (int j = 0; j < rank; ++j) {
        const float a = fabsf(Act<DT>::ld(row[j]));
        nan |= a != a;
        m = fmaxf(m, a);
    }
    const float safe = (!nan && m > 0.f && m <= 3.402823466e38f) ? m : 1.f;
    const float s = safe / 127.f;
    scales[r] = s;
    for (int j = 0; j < rank; ++j) {
        const float qv = rintf(Act<DT>::ld(row[j]) / s);
        const float cl = qv != qv ? 0.f : fminf(fmaxf(qv, -127.f), 127.f);
        codes[r * rank + j] = (int8_t)(int)cl;
    }
}

template <int DT>
__global__ __launch_bounds__(kRowThreads) void k_rows_dequantize(const int8_t *__restrict__ codes,
                                                                 const float *__restrict__ scales, int64_t rows,
                                                                 int rank, typename Act<DT>::T *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
    if (i >= rows * rank) return;
    out[i] = Act<DT>::st((float)codes[i] * scales[i / rank]);
}

int64_t stream_blocks(int64_t nnz) { return (nnz + kStreamBlock - 1) / kStreamBlock; }

}  // namespace

extern "C" int stacr_index_stream_sizes(int64_t nnz, int64_t *blocks, int64_t *max_words)
{
    if (nnz < 0 || nnz >= ((int64_t)1 << 31) || !blocks || !max_words)
        return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_sizes: nnz outside 0..2^31-1 or NULL output");
    *blocks = stream_blocks(nnz);
    *max_words = *blocks * 8 * 32;
    return STACR_OK;
}

extern "C" int stacr_index_stream_encode(const void *idx, int idx_bytes, int64_t nnz, void *base, void *word_off,
                                         void *words, void *status, void *stream)
{
    if (idx_bytes != 4 && idx_bytes != 8) return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_encode: idx_bytes must be 4 or 8");
    if (nnz < 0 || nnz >= ((int64_t)1 << 31)) return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_encode: nnz outside 0..2^31-1");
    if (!word_off || !status || (nnz > 0 && (!idx || !base || !words)))
        return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_encode: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = stream_blocks(nnz);
    const int idx64 = idx_bytes == 8;
    if (nb > 0)
        stacr_launch("k_stream_width", s, [&] {
            k_stream_width<<<(unsigned)nb, kStreamBlock, 0, s>>>(idx, idx64, nnz, static_cast<int64_t *>(base),
                                                                  static_cast<uint32_t *>(word_off));
        });
    stacr_launch("k_stream_offsets", s, [&] {
        k_stream_offsets<<<1, kScanThreads, 0, s>>>(nb, static_cast<uint32_t *>(word_off), static_cast<uint32_t *>(status));
    });
    if (nb > 0)
        stacr_launch("k_stream_pack", s, [&] {
            k_stream_pack<<<(unsigned)nb, kStreamBlock, 0, s>>>(idx, idx64, nnz, static_cast<const uint32_t *>(word_off),
                                                                 static_cast<uint32_t *>(words));
        });
    return stacr_hip_check(hipGetLastError(), "index stream encode");
}

extern "C" int stacr_index_stream_decode(const void *base, const void *word_off, const void *words, int64_t nnz,
                                         void *idx, int idx_bytes, void *stream)
{
    if (idx_bytes != 4 && idx_bytes != 8) return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_decode: idx_bytes must be 4 or 8");
    if (nnz < 0 || nnz >= ((int64_t)1 << 31)) return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_decode: nnz outside 0..2^31-1");
    if (nnz == 0) return STACR_OK;
    if (!base || !word_off || !words || !idx) return stacr_fail(STACR_ERR_INVALID, "stacr_index_stream_decode: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nb = stream_blocks(nnz);
    stacr_launch("k_stream_unpack", s, [&] {
        k_stream_unpack<<<(unsigned)nb, kStreamBlock, 0, s>>>(static_cast<const int64_t *>(base),
                                                               static_cast<const uint32_t *>(word_off),
                                                               static_cast<const uint32_t *>(words), nnz, idx,
                                                               idx_bytes == 8);
    });
    return stacr_hip_check(hipGetLastError(), "index stream decode");
}

extern "C" int stacr_quantize_rows_int8(const void *coeff, int dtype, int64_t rows, int rank, void *codes, void *scales,
                                        void *stream)
{
    if (dtype != STACR_DTYPE_F32 && dtype != STACR_DTYPE_BF16 && dtype != STACR_DTYPE_F16)
        return stacr_fail(STACR_ERR_INVALID, "stacr_quantize_rows_int8: unsupported dtype code %d", dtype);
    if (rows < 0 || rank < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_quantize_rows_int8: bad shape");
    if (rows == 0) return STACR_OK;
    if (!coeff || !codes || !scales) return stacr_fail(STACR_ERR_INVALID, "stacr_quantize_rows_int8: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const unsigned grid = (unsigned)((rows + kRowThreads - 1) / kRowThreads);
    int8_t *q = static_cast<int8_t *>(codes);
    float *sc = static_cast<float *>(scales);
    stacr_launch("k_rows_quantize", s, [&] {
        if (dtype == STACR_DTYPE_F32)
            k_rows_quantize<STACR_DTYPE_F32><<<grid, kRowThreads, 0, s>>>(static_cast<const float *>(coeff), rows, rank, q, sc);
        else if (dtype == STACR_DTYPE_BF16)
            k_rows_quantize<STACR_DTYPE_BF16><<<grid, kRowThreads, 0, s>>>(static_cast<const uint16_t *>(coeff), rows, rank, q, sc);
        else
            k_rows_quantize<STACR_DTYPE_F16><<<grid, kRowThreads, 0, s>>>(static_cast<const uint16_t *>(coeff), rows, rank, q, sc);
    });
    return stacr_hip_check(hipGetLastError(), "row quantization");
}

extern "C" int stacr_dequantize_rows_int8(const void *codes, const void *scales, int64_t rows, int rank, void *out,
                                          int out_dtype, void *stream)
{
    if (out_dtype != STACR_DTYPE_F32 && out_dtype != STACR_DTYPE_BF16 && out_dtype != STACR_DTYPE_F16)
        return stacr_fail(STACR_ERR_INVALID, "stacr_dequantize_rows_int8: unsupported dtype code %d", out_dtype);
    if (rows < 0 || rank < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_dequantize_rows_int8: bad shape");
    if (rows == 0) return STACR_OK;
    if (!codes || !scales || !out) return stacr_fail(STACR_ERR_INVALID, "stacr_dequantize_rows_int8: NULL pointer argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const unsigned grid = (unsigned)((rows * rank + kRowThreads - 1) / kRowThreads);
    const int8_t *q = static_cast<const int8_t *>(codes);
    const float *sc = static_cast<const float *>(scales);
    stacr_launch("k_rows_dequantize", s, [&] {
        if (out_dtype == STACR_DTYPE_F32)
            k_rows_dequantize<STACR_DTYPE_F32><<<grid, kRowThreads, 0, s>>>(q, sc, rows, rank, static_cast<float *>(out));
        else if (out_dtype == STACR_DTYPE_BF16)
            k_rows_dequantize<STACR_DTYPE_BF16><<<grid, kRowThreads, 0, s>>>(q, sc, rows, rank, static_cast<uint16_t *>(out));
        else
            k_rows_dequantize<STACR_DTYPE_F16><<<grid, kRowThreads, 0, s>>>(q, sc, rows, rank, static_cast<uint16_t *>(out));
    });
    return stacr_hip_check(hipGetLastError(), "row dequantization");
}
