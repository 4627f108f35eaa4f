/*
 * stacr_oracle.c -- CPU restatement of the STAC-R activation save / weight-gradient path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed CPU baseline
 * ("port").  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product path (stac-r_amd/) never links or calls it.
 *
 * Every function restates the reference algorithm it cites (paths relative to the
 * reference checkout, Manar-Hamed/STAC-R, package stacr 0.2.0):
 *
 *   orc_py_round          Python round() on a float (half-to-even), used by every k rule
 *   orc_chunk_k           stacr/layers.py:25,33        k per chunk = max(1, min(n, round(b*n)))
 *   orc_residual_plan     stacr/layers.py:16-41,44-54  k_total and the chunk sum for a layer
 *   orc_select            stacr/layers.py:16-41,69-80,100-101   chunk_topk / global_topk
 *   orc_quantize          stacr/quant.py:49-65         symmetric per-tensor int8 / int4 / passthrough
 *   orc_pack_int4         stacr/quant.py:30-37         two's-complement nibbles, even index low
 *   orc_weight_grad       stacr/layers.py:172-193      dW = (G^T C) Q^T + G^T R_s  (fp64 accumulation)
 *   orc_round_dtype       bf16 / fp16 round-to-nearest-even of an fp32 value (dtype-native ops)
 *   orc_residual_act      stacr/layers.py:32,73 and stacr/adaptive.py:1518-1519
 *                         R = X - C Q^T in the activation dtype (fixed fma order, see below)
 *   orc_select_explicit   stacr/adaptive.py:1511-1548  per-chunk top-k_c, then top-k of the union
 *   orc_lowrank           stacr/compressor.py:128      L = C Q^T in the activation dtype (same chain)
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   orc_select     reference known answers tests/test_integration.py:106-114 (global vs chunk),
 *                  tests/test_residual.py:6-11, brute force against numpy lexsort on random data,
 *                  tie rule on all-equal inputs, and the k counts quoted for the five configs.
 *   orc_chunk_k / orc_residual_plan   the reference's stored_bytes residual_count rule
 *                  (stacr/layers.py:417-449, tests/test_memory.py:366-388) and the config k values.
 *   orc_quantize   closed form: tiny-value case tests/test_integration.py:147-152, exact multiples
 *                  of the scale, clamping, and round-half-even ties.
 *   orc_pack_int4  nibble layout known answers; round trip through an independent unpack.
 *   orc_weight_grad  closed forms: budget 1 selects every entry so dW = G^T X; rank-d identity
 *                  basis; and a single non-zero residual entry.
 *   orc_round_dtype  numpy's float16 cast and torch's bfloat16 cast on every fp32 bit pattern class
 *                  (normal, subnormal, ties, overflow, NaN).
 *   orc_residual_act  fp64 projection rounded to the dtype (at most one ulp of the dtype apart),
 *                  torch's own dtype-native mm and subtraction on the CPU (the reference's ops), and
 *                  exact zero for X in the span of an orthonormal basis with exact coefficients.
 *   orc_select_explicit  brute force (numpy lexsort per chunk, then over the union) on random data.
 *   orc_lowrank    torch's own dtype-native mm on the CPU (the reference's unpack op), and
 *                  orc_residual_act with X = L giving exact zeros.
 *
 * Tie rule.  torch.topk(sorted=False) leaves the choice among equal magnitudes unspecified.  The
 * oracle (and the HIP path) breaks ties by the lowest flat index, and returns indices in
 * ascending order.  Magnitude order is the integer order of the fp32 bit pattern with the sign
 * cleared, which places NaN above +inf exactly as torch.topk does.
 *
 * Residual arithmetic.  The reference forms R = X - C Q^T with torch ops in the activation dtype:
 * the product rounded to the dtype, then the difference rounded to the dtype.  The HIP kernels
 * and orc_residual_act both sum the product as an fp32 fused multiply-add chain over
 * j = 0..r-1 from 0, so selection can be compared bit for bit on the same residual.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MODE_CHUNK 0
#define MODE_GLOBAL 1

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Python's round() on a double: nearest integer, ties to even (the default FP rounding mode). */
int64_t orc_py_round(double v) { return (int64_t)nearbyint(v); }

/* stacr/layers.py:33  k = max(1, min(flat.numel(), int(round(float(budget) * flat.numel())))) */
int64_t orc_chunk_k(int64_t n, double budget)
{
    int64_t k = orc_py_round(budget * (double)n);
    if (k > n) k = n;
    if (k < 1) k = 1;
    return k;
}

/*
 * k_total = int(round(budget * rows * feats)) (stacr/layers.py:25,51).  For chunk mode the sum of
 * per-chunk k (stacr/layers.py:30-36) is also returned; when it exceeds k_total the reference
 * trims with a second top-k (stacr/layers.py:38-40).  k_total <= 0 means no residual at all
 * (stacr/layers.py:26-27,52-53).
 */
void orc_residual_plan(int64_t rows, int64_t feats, int mode, double budget, int64_t chunk_rows,
                       int64_t *k_total, int64_t *k_chunk_sum)
{
    int64_t total = rows * feats;
    *k_total = orc_py_round(budget * (double)total);
    *k_chunk_sum = 0;
    if (*k_total <= 0) { *k_total = 0; return; }
    if (mode == MODE_GLOBAL) { *k_chunk_sum = *k_total; return; }
    if (chunk_rows < 1) chunk_rows = 1;
    int64_t s = 0;
    for (int64_t start = 0; start < rows; start += chunk_rows) {
        int64_t stop = start + chunk_rows < rows ? start + chunk_rows : rows;
        s += orc_chunk_k((stop - start) * feats, budget);
    }
    *k_chunk_sum = s;
}

/* Composite sort key: larger magnitude first, then lower flat index first. */
static inline uint64_t composite(float v, uint64_t flat)
{
    uint64_t key = (uint64_t)(f2u(v) & 0x7FFFFFFFu);
    return (key << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)flat);
}

static void swap64(uint64_t *a, uint64_t *b) { uint64_t t = *a; *a = *b; *b = t; }

/* In-place selection: afterwards a[0..k) hold the k largest values (unordered). */
static void select_largest(uint64_t *a, int64_t n, int64_t k)
{
    int64_t lo = 0, hi = n - 1, target = k - 1;
    while (lo < hi) {
        int64_t mid = lo + (hi - lo) / 2;
        /* median of three, descending order */
        if (a[mid] > a[lo]) swap64(&a[mid], &a[lo]);
        if (a[hi] > a[lo]) swap64(&a[hi], &a[lo]);
        if (a[hi] > a[mid]) swap64(&a[hi], &a[mid]);
        uint64_t pivot = a[mid];
        int64_t i = lo, j = hi;
        while (i <= j) {
            while (a[i] > pivot) ++i;
            while (a[j] < pivot) --j;
            if (i <= j) { swap64(&a[i], &a[j]); ++i; --j; }
        }
        if (target <= j) hi = j;
        else if (target >= i) lo = i;
        else break;
    }
}

static int cmp_i64(const void *a, const void *b)
{
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return (x > y) - (x < y);
}

static int cmp_u64_desc(const void *a, const void *b)
{
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return (x < y) - (x > y);
}

/*
 * Exact residual selection.  mode MODE_CHUNK restates _select_sparse_residual
 * (stacr/layers.py:16-41): per chunk of chunk_rows rows, keep the k_c largest |r|, then trim the
 * union to k_total by |r| when it is larger.  MODE_GLOBAL restates the global_topk branch
 * (stacr/layers.py:69-80,100-101), whose streaming merge is an exact global top-k_total.
 * Flat indices must fit in 32 bits for the composite key; the caller checks rows*d < 2^32.
 * Output: count (k_total, or 0 when there is no residual) and idx/val in ascending idx order.
 */
int64_t orc_select(const float *resid, int64_t rows, int64_t d, int mode, double budget,
                   int64_t chunk_rows, int64_t *idx_out, float *val_out)
{
    int64_t k_total, k_sum;
    orc_residual_plan(rows, d, mode, budget, chunk_rows, &k_total, &k_sum);
    if (k_total <= 0 || rows * d == 0) return 0;
    if (mode == MODE_GLOBAL) chunk_rows = rows;
    if (chunk_rows < 1) chunk_rows = 1;
    uint64_t *sel = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)k_sum);
    uint64_t *buf = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)((chunk_rows < rows ? chunk_rows : rows) * d));
    int64_t nsel = 0;
    for (int64_t start = 0; start < rows; start += chunk_rows) {
        int64_t stop = start + chunk_rows < rows ? start + chunk_rows : rows;
        int64_t n = (stop - start) * d, base = start * d;
        int64_t k = mode == MODE_GLOBAL ? k_total : orc_chunk_k(n, budget);
        for (int64_t e = 0; e < n; ++e) buf[e] = composite(resid[base + e], (uint64_t)(base + e));
        select_largest(buf, n, k);
        memcpy(sel + nsel, buf, sizeof(uint64_t) * (size_t)k);
        nsel += k;
    }
    if (nsel > k_total) {            /* stacr/layers.py:38-40 global trim of the union */
        select_largest(sel, nsel, k_total);
        nsel = k_total;
    }
    for (int64_t e = 0; e < nsel; ++e) {
        uint32_t flat = 0xFFFFFFFFu - (uint32_t)(sel[e] & 0xFFFFFFFFu);
        idx_out[e] = (int64_t)flat;
    }
    qsort(idx_out, (size_t)nsel, sizeof(int64_t), cmp_i64);
    for (int64_t e = 0; e < nsel; ++e) val_out[e] = resid[idx_out[e]];
    free(buf);
    free(sel);
    return nsel;
}

/* Sorted (descending) composite keys of a residual, for tests that need the k-th magnitude. */
void orc_sorted_keys(const float *resid, int64_t n, uint64_t *out)
{
    for (int64_t e = 0; e < n; ++e) out[e] = composite(resid[e], (uint64_t)e);
    qsort(out, (size_t)n, sizeof(uint64_t), cmp_u64_desc);
}

/*
 * stacr/quant.py:49-65.  bits 8 or 4: amax = max |v| in fp32; scale = max(amax / qmax, FLT_MIN)
 * in fp32; q = round_half_even(v / scale) clamped to [-qmax-1, qmax].  bits 0: q untouched, the
 * scale is 1.  Division is IEEE fp32 (correctly rounded), as torch performs it.
 */
void orc_quantize(const float *vals, int64_t n, int bits, int8_t *q_out, float *scale_out)
{
    if (bits == 0 || n == 0) { *scale_out = 1.0f; return; }
    float qmax = bits == 4 ? 7.0f : 127.0f;
    float amax = 0.0f;
    int has_nan = 0;
    for (int64_t i = 0; i < n; ++i) {
        float a = fabsf(vals[i]);
        if (a != a) has_nan = 1;
        else if (a > amax) amax = a;
    }
    if (has_nan) amax = NAN;
    volatile float s = amax / qmax;
    float scale = s < 1.17549435e-38f ? 1.17549435e-38f : s;
    if (amax != amax) scale = NAN;
    for (int64_t i = 0; i < n; ++i) {
        volatile float t = vals[i] / scale;
        float r = nearbyintf(t);
        if (r < -qmax - 1.0f) r = -qmax - 1.0f;
        if (r > qmax) r = qmax;
        q_out[i] = (int8_t)(r != r ? 0 : r);
    }
    *scale_out = scale;
}

/* stacr/quant.py:30-37: element 2i in the low nibble, 2i+1 in the high nibble, odd tail padded 0. */
void orc_pack_int4(const int8_t *q, int64_t n, uint8_t *out)
{
    for (int64_t i = 0; i < (n + 1) / 2; ++i) {
        uint8_t lo = (uint8_t)(q[2 * i] & 0x0F);
        uint8_t hi = 2 * i + 1 < n ? (uint8_t)(q[2 * i + 1] & 0x0F) : 0;
        out[i] = (uint8_t)(lo | (hi << 4));
    }
}

/*
 * stacr/layers.py:172-193 in fp64: dW[o][i] = sum_t G[t][o] * (sum_j C[t][j] Q[i][j])
 *                                            + sum_{(t,i) selected} G[t][o] * v.
 * Computed as M = G^T C (d_out x r) then M Q^T, then the sparse scatter, all in double.
 * dbias[o] = sum_t G[t][o] when dbias is not NULL (stacr/layers.py:197-198).
 */
int orc_weight_grad(const float *g, int64_t n, int64_t d_out, const float *c, const float *q,
                    int64_t d_in, int r, const int64_t *idx, const float *vals, int64_t nnz,
                    double *dw, double *dbias)
{
    /* indices come from the kernel under test: reject any outside [0, n*d_in) before using them */
    for (int64_t e = 0; e < nnz; ++e)
        if (idx[e] < 0 || idx[e] >= n * d_in) return -1;
    double *m = (double *)calloc((size_t)(d_out * r), sizeof(double));
    for (int64_t t = 0; t < n; ++t) {
        const float *gt = g + t * d_out;
        const float *ct = c + t * r;
        for (int64_t o = 0; o < d_out; ++o) {
            double gv = gt[o];
            for (int j = 0; j < r; ++j) m[o * r + j] += gv * (double)ct[j];
        }
    }
    for (int64_t o = 0; o < d_out; ++o)
        for (int64_t i = 0; i < d_in; ++i) {
            double s = 0.0;
            for (int j = 0; j < r; ++j) s += m[o * r + j] * (double)q[i * r + j];
            dw[o * d_in + i] = s;
        }
    for (int64_t e = 0; e < nnz; ++e) {
        int64_t t = idx[e] / d_in, i = idx[e] % d_in;
        double v = vals[e];
        const float *gt = g + t * d_out;
        for (int64_t o = 0; o < d_out; ++o) dw[o * d_in + i] += v * (double)gt[o];
    }
    if (dbias) {
        for (int64_t o = 0; o < d_out; ++o) dbias[o] = 0.0;
        for (int64_t t = 0; t < n; ++t)
            for (int64_t o = 0; o < d_out; ++o) dbias[o] += (double)g[t * d_out + o];
    }
    free(m);
    return 0;
}

/* Round an fp32 value to bf16 (code 1) or fp16 (code 2), nearest-even, returned as fp32; code 0
 * returns the value unchanged.  NaN stays NaN; fp16 overflow becomes +-inf. */
float orc_round_dtype(float f, int code)
{
    if (code == 0 || isnan(f)) return f;
    uint32_t u = f2u(f);
    if (code == 1) {
        u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
        return u2f(u);
    }
    const float a = fabsf(f);
    if (isinf(a)) return f;
    if (a < 6.103515625e-05f) {           /* below 2^-14: fp16 subnormal quantum 2^-24 */
        const float q = nearbyintf(f * 16777216.0f) / 16777216.0f;
        return q;
    }
    u = (u + 0xFFFu + ((u >> 13) & 1u)) & 0xFFFFE000u;  /* keep 10 mantissa bits */
    const float r = u2f(u);
    if (fabsf(r) > 65504.0f) return f < 0 ? -INFINITY : INFINITY;
    return r;
}

/* perp = rnd(x - rnd(sum_j c_j q_j)), the projection an fp32 fma chain from 0, j ascending. */
void orc_residual_act(const float *x, const float *c, const float *q, int64_t rows, int64_t d, int r, int code,
                      float *out)
{
    for (int64_t i = 0; i < rows; ++i) {
        const float *ci = c + i * r;
        for (int64_t e = 0; e < d; ++e) {
            const float *qe = q + e * r;
            float p = 0.f;
            for (int j = 0; j < r; ++j) p = fmaf(ci[j], qe[j], p);
            p = orc_round_dtype(p, code);
            out[i * d + e] = orc_round_dtype(x[i * d + e] - p, code);
        }
    }
}

/* L = rnd(C Q^T) in the activation dtype: the same fp32 chain as orc_residual_act
 * (stacr/compressor.py:128, the low-rank part of the dense unpack). */
void orc_lowrank(const float *c, const float *q, int64_t rows, int64_t d, int r, int code, float *out)
{
    for (int64_t i = 0; i < rows; ++i) {
        const float *ci = c + i * r;
        for (int64_t e = 0; e < d; ++e) {
            const float *qe = q + e * r;
            float p = 0.f;
            for (int j = 0; j < r; ++j) p = fmaf(ci[j], qe[j], p);
            out[i * d + e] = orc_round_dtype(p, code);
        }
    }
}

/* Per chunk of chunk_rows rows keep the min(k_chunk, n_c) largest |r| (ties: lowest flat index),
 * then the k_total largest of the union when it holds more.  Ascending idx order. */
int64_t orc_select_explicit(const float *resid, int64_t rows, int64_t d, int64_t chunk_rows, int64_t k_chunk,
                            int64_t k_total, int64_t *idx_out, float *val_out)
{
    if (k_total <= 0 || rows * d == 0 || k_chunk <= 0) return 0;
    if (chunk_rows < 1) chunk_rows = 1;
    const int64_t n_chunks = (rows + chunk_rows - 1) / chunk_rows;
    uint64_t *sel = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(n_chunks * k_chunk));
    uint64_t *buf = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)((chunk_rows < rows ? chunk_rows : rows) * d));
    int64_t nsel = 0;
    for (int64_t start = 0; start < rows; start += chunk_rows) {
        int64_t stop = start + chunk_rows < rows ? start + chunk_rows : rows;
        int64_t n = (stop - start) * d, base = start * d;
        int64_t k = k_chunk < n ? k_chunk : n;
        for (int64_t e = 0; e < n; ++e) buf[e] = composite(resid[base + e], (uint64_t)(base + e));
        select_largest(buf, n, k);
        memcpy(sel + nsel, buf, sizeof(uint64_t) * (size_t)k);
        nsel += k;
    }
    if (nsel > k_total) {
        select_largest(sel, nsel, k_total);
        nsel = k_total;
    }
    for (int64_t e = 0; e < nsel; ++e) idx_out[e] = (int64_t)(0xFFFFFFFFu - (uint32_t)(sel[e] & 0xFFFFFFFFu));
    qsort(idx_out, (size_t)nsel, sizeof(int64_t), cmp_i64);
    for (int64_t e = 0; e < nsel; ++e) val_out[e] = resid[idx_out[e]];
    free(buf);
    free(sel);
    return nsel;
}

