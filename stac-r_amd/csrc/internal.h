// Internal device helpers and launcher declarations shared by the HIP translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "stacr_amd.h"

namespace stacr {

// host-side min/max (the HIP headers' min/max are device functions)
template <typename T> inline T hmin(T a, T b) { return a < b ? a : b; }
template <typename T> inline T hmax(T a, T b) { return a < b ? b : a; }

constexpr int kBlock = 256;             // threads per workgroup (4 wave64)
constexpr int kWaves = kBlock / 64;
constexpr int kBins = 2048;             // histogram bins of the first two radix digits
// 31-bit magnitude key = fp32 bits of |r|; digits: [30:20] (11 b), [19:9] (11 b), [8:0] (9 b)
constexpr int kDigitShift[3] = {20, 9, 0};
constexpr int kDigitBins[3] = {2048, 2048, 512};
constexpr int kListBlock = 4096;        // list entries per workgroup in the trim pass

// ------------------------------------------------------------------ element types
__device__ __forceinline__ float bf16_bits_to_f(uint32_t v) { return __uint_as_float(v << 16); }
// fp32 -> bf16 bits, round to nearest even, a NaN keeping its sign and payload with the quiet bit
// set.  One v_cvt_pk_bf16_f32 on gfx950; it gives the same bits as the integer form
// ((u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN: (u >> 16) | 0x40) for every input, which was checked
// on the GPU over 2^20 patterns covering NaN payloads, infinities, denormals and ties.
__device__ __forceinline__ uint32_t f_to_bf16_bits(float f)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float f16_bits_to_f(uint32_t v)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)v);
}
__device__ __forceinline__ uint32_t f_to_f16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT> struct Act;
template <> struct Act<STACR_DTYPE_F32> {
    using T = float;
    static constexpr int kVec = 4;  // elements per 16-byte load
    static __device__ __forceinline__ float ld(T v) { return v; }
    static __device__ __forceinline__ T st(float f) { return f; }
    static __device__ __forceinline__ float rnd(float f) { return f; }
};
template <> struct Act<STACR_DTYPE_BF16> {
    using T = uint16_t;
    static constexpr int kVec = 8;
    static __device__ __forceinline__ float ld(T v) { return bf16_bits_to_f(v); }
    static __device__ __forceinline__ T st(float f) { return (T)f_to_bf16_bits(f); }
    static __device__ __forceinline__ float rnd(float f) { return bf16_bits_to_f(f_to_bf16_bits(f)); }
};
template <> struct Act<STACR_DTYPE_F16> {
    using T = uint16_t;
    static constexpr int kVec = 8;
    static __device__ __forceinline__ float ld(T v) { return f16_bits_to_f(v); }
    static __device__ __forceinline__ T st(float f) { return (T)f_to_f16_bits(f); }
    static __device__ __forceinline__ float rnd(float f) { return f16_bits_to_f(f_to_f16_bits(f)); }
};

// V consecutive elements starting at p, widened to fp32 (16-byte load when V == kVec).
template <int DT, int V>
__device__ __forceinline__ void load_vec(const typename Act<DT>::T *__restrict__ p, float (&x)[V])
{
    using A = Act<DT>;
    if constexpr (V == 1) {
        x[0] = A::ld(p[0]);
    } else if constexpr (sizeof(typename A::T) == 4) {
        static_assert(V == 4, "fp32 vector width is 4");
        const float4 v = *reinterpret_cast<const float4 *>(p);
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    } else {
        static_assert(V == 8, "16-bit vector width is 8");
        const uint4 v = *reinterpret_cast<const uint4 *>(p);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[2 * k] = A::ld((typename A::T)(w[k] & 0xffffu));
            x[2 * k + 1] = A::ld((typename A::T)(w[k] >> 16));
        }
    }
}

__device__ __forceinline__ float load_any(const void *p, int dt, int64_t i)
{
    if (dt == STACR_DTYPE_F32) return static_cast<const float *>(p)[i];
    const uint16_t v = static_cast<const uint16_t *>(p)[i];
    return dt == STACR_DTYPE_BF16 ? bf16_bits_to_f(v) : f16_bits_to_f(v);
}

__device__ __forceinline__ void store_any(void *p, int dt, int64_t i, float f)
{
    if (dt == STACR_DTYPE_F32) {
        static_cast<float *>(p)[i] = f;
    } else {
        static_cast<uint16_t *>(p)[i] =
            (uint16_t)(dt == STACR_DTYPE_BF16 ? f_to_bf16_bits(f) : f_to_f16_bits(f));
    }
}

// Sum 64 values (v = i * R + j) over the 64 lanes of a wave: six halving exchanges leave lane l
// with the wave's total of value l.
__device__ __forceinline__ float wave_reduce_scatter64(float (&a)[64])
{
    const int lane = threadIdx.x & 63;
    // Stages 32 and 16 in the VALU: v_permlane32_swap(x, y) gives lanes 0..31 (x[l], x[l + 32])
    // and lanes 32..63 (y[l - 32], y[l]); v_permlane16_swap does the same between even and odd
    // 16-lane rows (checked on the GPU).  With x the lower half and y the upper, the sum of the
    // pair is, in every lane, the total of the half that lane keeps (lane bit clear: lower).
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[k]), __float_as_uint(a[k + 32]), false, false);
        a[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[k]), __float_as_uint(a[k + 16]), false, false);
        a[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    // stages 8, 4, 2, 1: both halves cross (the select then picks between computed sums, never
    // between array elements, which keeps a[] in registers)
#pragma unroll
    for (int st = 2; st < 6; ++st) {
        const int o = 32 >> st;
        const bool upper = (lane & o) != 0;
#pragma unroll
        for (int k = 0; k < o; ++k) {
            const float lo = a[k] + __shfl_xor(a[k], o, 64);
            const float hi = a[k + o] + __shfl_xor(a[k + o], o, 64);
            a[k] = upper ? hi : lo;
        }
    }
    return a[0];
}

// Inclusive prefix sum over the 64 lanes of a wave in data-parallel moves (no LDS round trips):
// within each row of 16 lanes, adds of the value 1, 2, 4 and 8 lanes down (row_shr; a lane with no
// such lane in its row adds 0), then lane 15's total into rows 1 and 3 and lane 31's into rows 2
// and 3 (row_bcast:15 / row_bcast:31, the rows chosen by the row mask; the other rows add 0).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x)
{
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// ------------------------------------------------------------------ block primitives
// Exclusive prefix sum over the NT threads of a workgroup (NT a multiple of 64); *total receives
// the sum.  s_tot needs NT / 64 entries.  Every thread must call it (it contains __syncthreads).
template <int NT = kBlock>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *s_tot, uint32_t *total)
{
    constexpr int NWAVE = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t x = wave_inclusive_scan(v);
    if (lane == 63) s_tot[wave] = x;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
        const uint32_t t = s_tot[w];
        before += w < wave ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + x - v;
}

template <int NT = kBlock>
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t *s_tot)
{
    uint32_t total;
    block_exclusive_scan<NT>(v, s_tot, &total);
    return total;
}

// Two 16-bit products (packed pairs of the activation / gradient type) added to an fp32 sum
// (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
{
    if constexpr (DT == STACR_DTYPE_BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 v2;
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 v2;
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
    }
}

// ------------------------------------------------------------------ save geometry
// A workgroup owns `rows_per_wg` consecutive rows inside one selection chunk.  Inside it, the
// 256 threads form rpi = 256 / L row slots of L threads; each thread walks `mv` vectors of V
// elements per row at columns (m * L + u) * V.  Either rpi == 1 or mv == 1, so visiting the
// vectors in m-major, thread-minor order enumerates elements in ascending flat index.
struct SaveGeom {
    int64_t rows, d;
    int64_t chunk_rows;     // rows per selection chunk (global_topk: all rows)
    int64_t n_chunks;
    int64_t rows_per_wg;
    int64_t wgs_per_chunk;  // uniform; trailing workgroups of the last chunk may be empty
    int L, log2L, rpi, mv;
    int rank;
    // copies of each chunk histogram level and of the max key (batched passes): workgroup w adds
    // into copy w % hcopies, and readers sum the copies.  Device-scope atomics from hundreds of
    // workgroups on one address serialize; eight copies cut that to a few tens per address.
    int hcopies;
};

// Per-chunk selection state after each radix level: prefix of the key found so far and the
// number of elements still to take from inside that prefix.
struct SelState {
    uint32_t prefix;
    uint32_t need;
};

struct WgCount {
    uint32_t gt;  // elements with key > threshold
    uint32_t eq;  // elements with key == threshold
};

struct WgOffset {
    uint32_t off;   // first output position of the workgroup
    uint32_t take;  // ties (key == threshold) it keeps, lowest flat index first
};

}  // namespace stacr

// ------------------------------------------------------------------ error reporting
int stacr_fail(int code, const char *fmt, ...);
int stacr_hip_check(hipError_t err, const char *what);

// ------------------------------------------------------------------ timing hook (profile.hip)
bool stacr_prof_on();
void stacr_prof_before(hipStream_t s);
void stacr_prof_after(const char *name, hipStream_t s);

// Every kernel launch goes through here so the optional timing hook can bracket it.
template <typename F>
inline void stacr_launch(const char *name, hipStream_t s, F &&launch)
{
    const bool timed = stacr_prof_on();
    if (timed) stacr_prof_before(s);
    launch();
    if (timed) stacr_prof_after(name, s);
}

// ------------------------------------------------------------------ launchers (save.hip)
struct StacrSaveArgs {
    const void *x;
    const void *q;
    int dtype;
    int64_t rows, feats;
    int rank;
    int mode;
    int64_t chunk_rows;  // effective (global_topk: rows)
    int64_t k_total, k_full, k_last, k_sum;
    int bits;
    const void *coeff_in;  // non-NULL: use these coefficients instead of projecting X
    void *coeff, *idx;
    int index_bytes;
    void *data;
    float *scale;
    void *workspace;
    size_t workspace_bytes;
    hipStream_t stream;
    // optional entry census for the weight gradient (NULL: none); *census_written (host) tells
    // whether this save filled it
    uint32_t *census = nullptr;
    int *census_written = nullptr;
    // The basis q has q_ld columns a row (0: rank); the save uses its first `rank`.  Optional outputs
    // of the projection pass where it can write them (the wide pass; *written (host) tells):
    //   y_out        rows x y_cols fp32, X q[:, :y_cols] before rounding (rank <= y_cols <= q_ld), for
    //                an Oja refresh on the same X and basis
    //   energy_part  per projection workgroup [kEnergyStride]: sum of rnd(x^2), sum of rnd(c^2), and
    //                sum of c_j^2 per basis column j < rank (fp32, C as saved)
    int q_ld = 0, y_cols = 0;
    float *y_out = nullptr;
    int *y_written = nullptr;
    float *energy_part = nullptr;
    int *energy_written = nullptr;
};
constexpr int kEnergyStride = 2 + STACR_MAX_RANK;  // floats of one energy partial
// Projection workgroups whose energy partials stacr_save_launch writes for these arguments (0 when
// the plan's projection pass does not form them)
int64_t stacr_save_energy_slots(const StacrSaveArgs &a);
size_t stacr_save_ws_layout(const StacrSaveArgs &a, size_t *offsets);

// Entry census: what the weight gradient's matrix-core plan needs to know about a save's residual
// entries, written by the save's emission pass when it can (bf16 candidate passes, no trim):
// per-feature entry counts in kCensusCopies copies ([copy][feats], summed by the reader), then
// the first entry of every block of kCensusRows token rows ([ceil(rows / kCensusRows) + 1], the
// last = the entry count).
constexpr int kCensusCopies = 8;
constexpr int kCensusRows = 512;
inline int64_t census_words(int64_t rows, int64_t feats)
{
    return (int64_t)kCensusCopies * feats + (rows + kCensusRows - 1) / kCensusRows + 1;
}
int stacr_save_launch(const StacrSaveArgs &a);
int stacr_quantize_launch(const void *v, int dtype, int64_t n, int bits, void *data, float *scale, void *workspace,
                          hipStream_t s);

// ------------------------------------------------------------------ launchers (weight_grad.hip)
struct StacrGradArgs {
    const void *g;
    int dtype;
    int64_t rows, d_out;
    const void *coeff, *q;
    int64_t d_in;
    int rank;
    const void *idx;
    int index_bytes;
    const void *data;
    const float *scale;
    int bits, val_dtype;
    int64_t nnz;
    int transposed;
    void *dw;
    int dw_dtype;
    void *dbias;
    int dbias_dtype;
    void *workspace;
    size_t workspace_bytes;
    hipStream_t stream;
    const uint32_t *census = nullptr;  // optional entry census from the save (see above)
};
size_t stacr_grad_ws_layout(const StacrGradArgs &a, size_t *offsets);
int stacr_grad_launch(const StacrGradArgs &a);
// the matrix-core path of weight_grad_tiles.hip (16-bit G, rank + bias column <= 16, d_out % 16 == 0)
bool stacr_tiles_eligible(const StacrGradArgs &a);
size_t stacr_tiles_ws(const StacrGradArgs &a);
size_t stacr_tiles_ws_bound(int64_t rows, int64_t d_out, int64_t d_in, int64_t nnz);  // any dtype / bias
int stacr_tiles_launch(const StacrGradArgs &a);

// ------------------------------------------------------------------ launchers (adaptive.hip)
// n integers of `bytes` bytes at p set to v by a kernel (no hipMemsetAsync: the callers' launches may
// be captured into a HIP graph)
int stacr_fill_int_launch(void *p, int bytes, int64_t n, int64_t v, hipStream_t s);
int stacr_aq_quantize_launch(const void *v, int dtype, int64_t n, int bits, void *data, void *scale, void *ws,
                             hipStream_t s);
int stacr_aq_dequantize_launch(const void *data, int bits, const void *scale, int64_t n, void *out, int out_dt,
                               hipStream_t s);
int stacr_csr_encode_launch(const void *idx, int idx_bytes, int64_t nnz, int64_t rows, int64_t n_cols, void *ptr,
                            int ptr_bytes, void *cols, int col_bytes, hipStream_t s);
int stacr_csr_decode_launch(const void *ptr, int ptr_bytes, const void *cols, int col_bytes, int64_t rows,
                            int64_t n_cols, int64_t nnz, void *idx, int idx_bytes, hipStream_t s);
int stacr_delta_max_launch(const void *idx, int idx_bytes, int64_t nnz, void *out, hipStream_t s);
int stacr_delta_encode_launch(const void *idx, int idx_bytes, int64_t nnz, void *base, int base_bytes, void *deltas,
                              int delta_bytes, hipStream_t s);
size_t stacr_delta_decode_ws(int64_t nnz);
int stacr_delta_decode_launch(const void *base, int base_bytes, const void *deltas, int delta_bytes, int64_t nnz,
                              void *idx, int idx_bytes, void *ws, hipStream_t s);
// ------------------------------------------------------------------ launchers (selectors.hip)
int stacr_uniform_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                         int rank, int64_t k, void *idx, int idx_bytes, void *values, hipStream_t s);
size_t stacr_block_ws(int64_t rows, int64_t d, int64_t bs, int64_t n_seg, int64_t count_full);
size_t stacr_adaptive_block_ws(int64_t rows, int64_t d, int64_t bs, int64_t n_cand, int64_t k_blocks);
int stacr_adaptive_block_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                                int rank, int64_t bs, int64_t chunk_rows, int64_t count_full, int64_t count_last,
                                int64_t k_blocks, void *idx, int idx_bytes, void *values, int64_t *count, void *ws,
                                hipStream_t s);
int stacr_block_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d, int rank,
                       int64_t bs, int64_t seg_rows, int64_t count_full, int64_t count_last, void *idx,
                       int idx_bytes, void *values, void *ws, hipStream_t s);
int stacr_sample_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                        int rank, const int64_t *pos, int64_t n, void *out, hipStream_t s);
size_t stacr_threshold_ws(int64_t rows, int64_t d);
int stacr_threshold_launch(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t d,
                           int rank, const float *thr, int64_t cap, void *idx, int idx_bytes, void *values,
                           int64_t *count, void *ws, hipStream_t s);

size_t stacr_oja_ws_bytes(int64_t rows, int64_t d, int rank);
int stacr_oja_launch(const void *x, int dtype, int64_t rows, int64_t d, const float *q, int rank, float lr,
                     float *update, float *out, void *ws, hipStream_t s);
// the Oja step on a Y = X Q computed elsewhere (rows x rank fp32): one pass over X
bool stacr_oja_given_y_ok(int dtype, int64_t rows, int64_t d, int rank, const void *x, const void *y);
int stacr_oja_given_y_launch(const void *x, int64_t rows, int64_t d, const float *q, int rank, const float *y,
                             float lr, float *update, float *out, void *ws, hipStream_t s);
size_t stacr_energy_ws();
int stacr_energy_launch(const void *x, const void *c, int dtype, int64_t rows, int64_t feats, int rank, float *out,
                        void *ws, hipStream_t s);
// the energies from a save's per-workgroup partials (n of them, [kEnergyStride] each), added in order
size_t stacr_energy_fold_ws();
int stacr_energy_fold_launch(const float *part, int64_t n, int dtype, int64_t rows, int rank, float *out, void *ws,
                             hipStream_t s);
