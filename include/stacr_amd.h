/*
 * stacr_amd.h -- C ABI of the MI355X-native STAC-R save / weight-gradient path.
 *
 * Plain C types only: device pointers are `void*`, sizes are int64_t, the HIP stream is passed
 * as `void*` (a hipStream_t, or NULL for the default stream).  The library never allocates:
 * every output and the workspace are supplied by the caller (query the workspace size first).
 * Every entry point returns STACR_OK or an error code; stacr_last_error() gives a thread-local
 * message for the last failure on the calling thread.  Launches are asynchronous on `stream`;
 * no entry point synchronises the device or reads device memory back to the host.
 *
 * Reference interfaces replaced (Manar-Hamed/STAC-R, stacr 0.2.0):
 *   stacr_residual_plan      k rules of stacr/layers.py:25-27,33,51-53
 *   stacr_save               STACRFunction.forward compression, stacr/layers.py:135-148
 *                            (coeff = X.Q, _select_residual :16-41/:44-102, quantize_values
 *                            stacr/quant.py:49-65)
 *   stacr_weight_grad        STACRFunction.backward grad_weight / grad_bias,
 *                            stacr/layers.py:172-198
 *   stacr_adaptive_*         adaptive engine save and quantizers, stacr/adaptive.py:44-159,
 *                            1333-1572,1943-2108
 *   stacr_csr_* / stacr_delta_*   index codecs, stacr/index_compression.py:193-345
 *   stacr_select_uniform / stacr_select_block_sparse / stacr_sample_magnitudes /
 *   stacr_select_threshold   the "uniform", "block_sparse", "sampled" selectors,
 *                            stacr/layers.py:55-99
 *   stacr_adaptive_block_sparse_plan / stacr_adaptive_select_block_sparse
 *                            the adaptive engine's block_sparse selector, stacr/adaptive.py:1788-1938
 *   stacr_oja_step           the Oja step of STACRLinear._refresh_basis, stacr/layers.py:346-348,
 *                            and OjaBasis.update, stacr/oja.py:73-79
 *   stacr_reconstruct        the saved-tensor hooks' dense unpack, stacr/compressor.py:127-133 with
 *                            stacr/residual.py:13-20
 *   stacr_index_stream_*     a bit-packed form of the delta index codec, stacr/index_compression.py:
 *                            231-269 (encode) and :327-342 (decode)
 *   stacr_*_rows_int8        int8 coefficients with a scale per row (the C1 codec's quantizer,
 *                            stacr/protocols/checkpointing.py:374-400, per row)
 *   stacr_c1_*               the C1 checkpoint-boundary codec's device work,
 *                            CheckpointBoundaryCodec.pack_tensor / unpack_record,
 *                            stacr/protocols/checkpointing.py:374-400,411-545
 */
#ifndef STACR_AMD_H
#define STACR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STACR_ABI_VERSION 1

/* element types of activations, gradients, coefficients, basis and outputs */
#define STACR_DTYPE_F32 0
#define STACR_DTYPE_BF16 1
#define STACR_DTYPE_F16 2

/* residual selection modes (stacr/layers.py:13; "topk" is an alias of "chunk_topk") */
#define STACR_MODE_CHUNK_TOPK 0
#define STACR_MODE_GLOBAL_TOPK 1

/* status codes */
#define STACR_OK 0
#define STACR_ERR_INVALID 1     /* bad argument (shape, dtype, null pointer, size) */
#define STACR_ERR_UNSUPPORTED 2 /* valid for the reference but outside this library's limits */
#define STACR_ERR_WORKSPACE 3   /* workspace smaller than the queried size */
#define STACR_ERR_HIP 4         /* a HIP runtime call failed */

/* Largest padded rank the kernels are built for (ranks 1..32 are accepted). */
#define STACR_MAX_RANK 32

int stacr_abi_version(void);

/* Thread-local description of the last error returned on this thread ("" if none). */
const char *stacr_last_error(void);

/*
 * Residual entry counts for a (rows x feats) activation (stacr/layers.py:25-27,33,51-53):
 *   *k_total  = round_half_even(budget * rows * feats)   (0 means "no residual is saved")
 *   *k_saved  = number of entries stacr_save writes: k_total for global_topk; for chunk_topk the
 *               sum over chunks of max(1, min(n_c, round(budget * n_c))), trimmed to k_total.
 * Also reports whether flat indices need int64 (*index_bytes = 8 when rows*feats >= 2^31-1,
 * stacr/layers.py:41,54).
 */
int stacr_residual_plan(int64_t rows, int64_t feats, int mode, double budget, int64_t chunk_rows,
                        int64_t *k_total, int64_t *k_saved, int *index_bytes);

/* Workspace bytes stacr_save needs for this problem. */
int stacr_save_workspace_bytes(int64_t rows, int64_t feats, int rank, int dtype, int mode,
                               double budget, int64_t chunk_rows, int bits, size_t *bytes);

/*
 * One streaming save of the activation X (rows x feats, row-major, `dtype`):
 *   coeff (rows x rank, dtype)   = X . Q, fp32 accumulation, rounded once to dtype
 *   residual r = rnd(X - rnd(coeff . Q^T)) in dtype (the reference's torch ops: product rounded,
 *   then difference rounded; fp32 fused multiply-adds over the rank), selected by |r| per
 *   chunk_topk / global_topk with the
 *   reference's k rules; ties at the cut go to the lowest flat index; output is in ascending
 *   flat-index order:
 *   idx   (k_saved, int32 or int64 per index_bytes) = row * feats + col
 *   data  bits 8: int8 q; bits 4: uint8 packed nibbles (ceil(k/2) bytes, even entry low);
 *         bits 0: values in `dtype`
 *   scale (1 fp32) = max(amax / qmax, FLT_MIN), or 1 for bits 0
 * q is the basis already cast to `dtype` (feats x rank, row-major), as the reference saves it.
 * budget <= 0 or k_total == 0: only coeff is written (idx/data/scale may be NULL).
 * Requires rows*feats < 2^32 and 1 <= rank <= STACR_MAX_RANK.
 */
int stacr_save(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank,
               int mode, double budget, int64_t chunk_rows, int bits, void *coeff, void *idx,
               int index_bytes, void *data, float *scale, void *workspace,
               size_t workspace_bytes, void *stream);

/*
 * stacr_save that can also write an entry census for the weight gradient (no counterpart in the
 * reference: an internal hand-off between the save and the backward of one layer, so that the
 * backward skips its own count of the entries).  The census (census_bytes from
 * stacr_save_census_bytes; uint32 words) holds, per input feature, the number of saved entries
 * (in 8 copies, [copy][feats], to be summed) and the first entry of every block of 512 rows
 * ([ceil(rows / 512) + 1], the last = nnz).  The save fills it when its bf16 candidate passes run
 * without a trim; *census_written (host memory) is set to 1 then, else 0 (pass the census to
 * stacr_weight_grad_census only when it is 1).  Outputs otherwise as stacr_save.
 */
int stacr_save_census_bytes(int64_t rows, int64_t feats, size_t *bytes);
int stacr_save_census(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank, int mode,
                      double budget, int64_t chunk_rows, int bits, void *coeff, void *idx, int index_bytes,
                      void *data, float *scale, void *workspace, size_t workspace_bytes, void *census,
                      size_t census_bytes, int *census_written, void *stream);

/*
 * Selection and quantization only, on caller-supplied coefficients (rows x rank, dtype):
 * the reference's _select_residual(x, coeff, basis, ...) followed by quantize_values
 * (stacr/layers.py:44-102,148).  Same residual arithmetic, rules and outputs as stacr_save;
 * use stacr_save_workspace_bytes for the workspace size.
 */
int stacr_select_residual(const void *x, const void *coeff, const void *q, int dtype, int64_t rows,
                          int64_t feats, int rank, int mode, double budget, int64_t chunk_rows,
                          int bits, void *idx, int index_bytes, void *data, float *scale,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * quantize_values (stacr/quant.py:49-65) for bits 4 or 8 on n values of `dtype`:
 * scale = max(max|v| / qmax, FLT_MIN) (fp32), q = round_half_even(v / scale) clamped to
 * [-qmax-1, qmax]; bits 8 writes n int8, bits 4 writes ceil(n/2) packed bytes (even entry in the
 * low nibble).  Needs 4 workspace bytes.  (bits 0 is a passthrough and needs no kernel.)
 */
int stacr_quantize_values(const void *values, int dtype, int64_t n, int bits, void *data, float *scale,
                          void *workspace, size_t workspace_bytes, void *stream);

/* Workspace bytes stacr_weight_grad needs for this problem. */
int stacr_weight_grad_workspace_bytes(int64_t rows, int64_t d_out, int64_t d_in, int rank,
                                      int64_t nnz, size_t *bytes);

/*
 * Weight gradient from the saved factors (stacr/layers.py:172-198):
 *   dW = (G^T . coeff) . Q^T + G^T . R_s        fp32 accumulation, rounded once to dw_dtype
 *   dbias = sum over rows of G                  (optional; dbias may be NULL)
 * g: rows x d_out (dtype); coeff: rows x rank (dtype); q: d_in x rank (dtype).
 * Sparse residual: idx (nnz, ascending flat indices row*d_in+col, int32 or int64 per
 * index_bytes), data/scale/bits as written by stacr_save; for bits 0 `data` holds values of
 * val_dtype.  nnz may be 0 (low-rank only; idx/data/scale may then be NULL).
 * transposed = 0: dW is d_out x d_in (nn.Linear); 1: d_in x d_out (Transformers Conv1D).
 */
int stacr_weight_grad(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff,
                      const void *q, int64_t d_in, int rank, const void *idx, int index_bytes,
                      const void *data, const float *scale, int bits, int val_dtype, int64_t nnz,
                      int transposed, void *dw, int dw_dtype, void *dbias, int dbias_dtype,
                      void *workspace, size_t workspace_bytes, void *stream);
/* stacr_weight_grad with the census a stacr_save_census call wrote for these entries (same rows,
 * d_in and residual): the matrix-core path takes the counts and block starts from it instead of
 * counting (one launch fewer); the other paths ignore it.  Same results as stacr_weight_grad.
 * census_bytes is the census buffer's size; a buffer smaller than stacr_save_census_bytes(rows,
 * d_in) is refused with STACR_ERR_INVALID (a census of another problem would be read past its end). */
int stacr_weight_grad_census(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff, const void *q,
                             int64_t d_in, int rank, const void *idx, int index_bytes, const void *data,
                             const float *scale, int bits, int val_dtype, int64_t nnz, int transposed, void *dw,
                             int dw_dtype, void *dbias, int dbias_dtype, const void *census, size_t census_bytes,
                             void *workspace, size_t workspace_bytes, void *stream);

/*
 * Allocation-free weight gradient.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, arithmetic and results as stacr_weight_grad, without the workspace:
 * the plan lives in a static device array of STACR_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends.  Problems whose stacr_weight_grad_workspace_bytes exceeds it are rejected with
 * STACR_ERR_UNSUPPORTED.  The entry point allocates nothing (no hipMalloc / hipFree); calls that
 * overlap on one GPU share its scratch and race, so serialize them (one stream, or events).
 */
#define STACR_NOALLOC_SCRATCH_BYTES (48u << 20)
int stacr_weight_grad_noalloc(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff,
                              const void *q, int64_t d_in, int rank, const void *idx, int index_bytes,
                              const void *data, const float *scale, int bits, int val_dtype, int64_t nnz,
                              int transposed, void *dw, int dw_dtype, void *dbias, int dbias_dtype, void *stream);

/* ------------------------------------------------------------------------------------------
 * Adaptive engine (stacr/adaptive.py, stacr/index_compression.py)
 * ---------------------------------------------------------------------------------------- */

/* Scale record written by stacr_adaptive_quantize (16 bytes, device memory): a double holding
 * the scale's value and an int32 naming the dtype the reference keeps it in: the input dtype,
 * STACR_DTYPE_F32 when a 16-bit scale underflowed to 0 and the reference redid the
 * quantization in fp32, or STACR_SCALE_F64 when an fp32 scale underflowed. */
#define STACR_SCALE_F64 3

/*
 * Residual entry counts of the adaptive engine's "topk" mode (stacr/adaptive.py:1357-1365,
 * 1492,1524-1530): k = floor(rows*feats*budget) (0: no residual), chunk = min(chunk_rows, rows),
 * per-chunk k = max(1, ceil(k*chunk/rows)) capped at the chunk's element count; the union is cut
 * to k when larger.  *k_saved is the number of entries stacr_adaptive_save writes; *index_bytes
 * is 2 below 32768 elements, 4 up to 2^31, else 8 (_choose_index_dtype, :138-159).
 */
int stacr_adaptive_residual_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows,
                                 int64_t *k, int64_t *k_saved, int *index_bytes);

int stacr_adaptive_save_workspace_bytes(int64_t rows, int64_t feats, int rank, int dtype, double budget,
                                        int64_t chunk_rows, size_t *bytes);

/*
 * Adaptive-engine STAC-R save (stacr/adaptive.py:1333-1572, residual_mode "topk", standard
 * chunked top-k): coeff = X.Q rounded once to dtype (or taken from coeff_in when non-NULL);
 * residual in the activation dtype, r = rnd(x - rnd(c.q)); per-chunk top-k then the top-k of
 * the union; ties to the lowest flat index; ascending flat order.  idx (k_saved) in index_bytes
 * (2, 4 or 8); values (k_saved, dtype).  energy (fp32[3 + rank], device): [0] residual energy
 * sqrt(max(|X|^2-|C|^2,0))/(sqrt(|X|^2)+1e-8) in the dtype's arithmetic (:1388-1393), [1] |X|^2,
 * [2] |C|^2, [3 + j] mean over rows of c_j^2 in fp32 (:1953-1958); energy may be NULL.
 */
int stacr_adaptive_save(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank,
                        double budget, int64_t chunk_rows, const void *coeff_in, void *coeff, void *idx,
                        int index_bytes, void *values, float *energy, void *workspace, size_t workspace_bytes,
                        void *stream);

/*
 * stacr_adaptive_save on a basis q of q_cols columns (feats x q_cols, row-major; rank <= q_cols <= 32)
 * of which the save uses the first `rank` (the active rank, stacr/adaptive.py:3116-3160: the layer
 * saves on basis[:, :active]).  When y is non-NULL and the projection pass can write it (16-bit X on
 * the wide projection pass: rank or q_cols 16, or feats > 2048; *y_written = 1), y (rows x q_cols
 * fp32) receives X q before rounding: the Y = X B of the adaptive layer's post-forward Oja refresh
 * (:3311-3395), which stacr_oja_step_given_y then finishes in one more pass over X.  The energies
 * come from the same projection pass where it runs (one read of X), else from a pass of their own.
 * Workspace: stacr_adaptive_save_y_workspace_bytes.
 */
int stacr_adaptive_save_y_workspace_bytes(int64_t rows, int64_t feats, int q_cols, int rank, int dtype,
                                          double budget, int64_t chunk_rows, size_t *bytes);
int stacr_adaptive_save_y(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int q_cols,
                          int rank, double budget, int64_t chunk_rows, const void *coeff_in, void *coeff,
                          void *idx, int index_bytes, void *values, float *energy, float *y, int *y_written,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * quantize_int8 / quantize_int4 (stacr/adaptive.py:44-120): scale = max|v| / qmax computed and
 * rounded in the input dtype; q = round(v / scale) with the quotient rounded to the input dtype,
 * clamped to [-qmax, qmax] (qmax 127 or 7); int4 stores q + 8 as nibbles, even entry low, odd
 * length padded with 8 (all zero: every byte 0x88).  All-zero input: q = 0, scale 1.  A scale
 * that underflows to 0 is recomputed in fp32 (16-bit inputs) or fp64 (fp32 inputs), as the
 * reference's recursion does.  data: int8[n] or uint8[ceil(n/2)]; scale: 16-byte record (see
 * STACR_SCALE_F64).  Needs 4 workspace bytes.
 */
int stacr_adaptive_quantize(const void *values, int dtype, int64_t n, int bits, void *data, void *scale,
                            void *workspace, size_t workspace_bytes, void *stream);

/* dequantize_int8 / dequantize_int4 (stacr/adaptive.py:79-90,123-131): q.to(scale dtype) * scale,
 * then converted to out_dtype.  n is the element count (orig_len for int4). */
int stacr_adaptive_dequantize(const void *data, int bits, const void *scale, int64_t n, void *out, int out_dtype,
                              void *stream);

/*
 * CSR index compression of row-sorted flat indices (stacr/index_compression.py:193-229):
 * row_ptrs[t] = entries in rows < t (t = 0..rows; int32 when nnz < 2^31 else int64 -> ptr_bytes),
 * cols = idx mod n_cols (int16 when n_cols < 32768, int32 up to 2^31, else int64 -> col_bytes).
 * The MI355X save already emits ascending indices, which are row-sorted.
 */
int stacr_csr_encode(const void *idx, int idx_bytes, int64_t nnz, int64_t rows, int64_t n_cols, void *row_ptrs,
                     int ptr_bytes, void *cols, int col_bytes, void *stream);
/* CSR back to flat indices row * n_cols + col (decompress_indices, :296-325). */
int stacr_csr_decode(const void *row_ptrs, int ptr_bytes, const void *cols, int col_bytes, int64_t rows,
                     int64_t n_cols, int64_t nnz, void *idx, int idx_bytes, void *stream);

/* Largest gap between consecutive sorted indices (int64, device), used to choose the delta width. */
int stacr_delta_max(const void *idx, int idx_bytes, int64_t nnz, void *max_delta, void *stream);
/* Delta encoding of sorted indices (:231-269): base = idx[0]; deltas[e-1] = idx[e] - idx[e-1]. */
int stacr_delta_encode(const void *idx, int idx_bytes, int64_t nnz, void *base, int base_bytes, void *deltas,
                       int delta_bytes, void *stream);
int stacr_delta_decode_workspace_bytes(int64_t nnz, size_t *bytes);
/* base + prefix sums of the deltas (decompress_indices, :327-342). */
int stacr_delta_decode(const void *base, int base_bytes, const void *deltas, int delta_bytes, int64_t nnz,
                       void *idx, int idx_bytes, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- other residual selectors
 * The projection engine's "uniform", "block_sparse" and "sampled" residual modes
 * (_select_residual, stacr/layers.py:44-101).  Inputs are the save's factors: x (rows x feats),
 * coeff (rows x rank, from stacr_save with budget 0) and q (feats x rank), all in `dtype`.  The
 * residual is r = rnd(x - rnd(coeff q^T)) in that dtype, as the reference's torch ops form it.
 * Indices are flat row*feats + col, ascending; index_bytes is 4 when rows*feats < 2^31 - 1, else 8
 * (stacr/layers.py:52).  Values are residual entries in `dtype`; the caller quantizes them with
 * stacr_quantize_values as the reference does (stacr/layers.py:146). */

/* uniform (:89-98): the k positions floor(i * rows * feats / k), i = 0..k-1, with
 * k = round(budget * rows * feats) chosen by the caller. */
int stacr_select_uniform(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                         int rank, int64_t k, void *idx, int index_bytes, void *values, void *stream);
/* block_sparse counts (:81-88): per chunk of chunk_rows rows, count = max(1, round(budget * blocks));
 * entries = sum of count * block_size.  Requires feats % block_size == 0 (otherwise the reference
 * falls back to chunk_topk, :67-68) and 0 < budget <= 1. */
int stacr_block_sparse_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows, int64_t block_size,
                            int64_t *count_full, int64_t *count_last, int64_t *entries, size_t *workspace_bytes);
/* block_sparse selection: per chunk the `count` blocks of block_size consecutive elements with the
 * largest energy rnd(sum rnd(r^2)) (ties: lowest block), every element of each chosen block. */
int stacr_select_block_sparse(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                              int rank, double budget, int64_t chunk_rows, int64_t block_size, void *idx,
                              int index_bytes, void *values, void *workspace, size_t workspace_bytes, void *stream);
/* The adaptive engine's block_sparse (stacr/adaptive.py:1788-1938), its default residual mode.
 * Blocks are `block_size` columns of one row (the row's last block padded with zeros when
 * feats % block_size != 0).  k = floor(rows*feats*budget); k_blocks = max(1, ceil(k/block_size));
 * per chunk of chunk_rows rows the max(1, ceil(k_blocks*chunk/rows)) blocks of largest energy
 * rnd(sum rnd(r^2)) (ties: lowest block), then the k_blocks largest of all those candidates.  Every
 * stored column of the kept blocks is written, ascending: *max_entries = kept blocks * block_size
 * is exact when feats % block_size == 0 and an upper bound otherwise; the number written goes to
 * the device int64 *count.  index_bytes follows _choose_index_dtype (2 below 32768 elements, 4 up
 * to 2^31, else 8); *k_blocks = 0 means no residual (no kernel runs, *count = 0). */
int stacr_adaptive_block_sparse_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows,
                                     int64_t block_size, int64_t *k_blocks, int64_t *max_entries, int *index_bytes,
                                     size_t *workspace_bytes);
int stacr_adaptive_select_block_sparse(const void *x, const void *coeff, const void *q, int dtype, int64_t rows,
                                       int64_t feats, int rank, double budget, int64_t chunk_rows, int64_t block_size,
                                       void *idx, int index_bytes, void *values, int64_t *count, void *workspace,
                                       size_t workspace_bytes, void *stream);
/* sampled (:55-66), step 1: out[i] = |r| at flat position positions[i] (int64, device), in dtype.
 * The caller draws the positions (torch.randint with the reference's seeded generator) and takes
 * the quantile of the magnitudes (torch.quantile), as the reference does.  A position outside
 * [0, rows*feats) yields NaN. */
int stacr_sample_magnitudes(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                            int rank, const int64_t *positions, int64_t n, void *out, void *stream);
int stacr_threshold_workspace_bytes(int64_t rows, int64_t feats, size_t *bytes);
/* sampled, step 2: the first `cap` flat positions (ascending) with |r| >= threshold, the fp32
 * device scalar *threshold compared after rounding to dtype (torch's promotion for
 * `magnitude >= threshold`).  *count (int64, device) receives min(cap, passing entries); with
 * cap = 0 nothing is written and *count receives every passing entry (a count-only call, which
 * sizes the outputs of the adaptive engine's threshold selections, stacr/adaptive.py:1416-1517,
 * 1574-1622,1628-1786: count, then select with cap = count). */
int stacr_select_threshold(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                           int rank, const float *threshold, int64_t cap, void *idx, int index_bytes, void *values,
                           int64_t *count, void *workspace, size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- basis refresh (Oja step) */

/* Workspace of stacr_oja_step for this shape (about rows*rank*4 + 4 MiB at rank 16). */
int stacr_oja_workspace_bytes(int64_t rows, int64_t feats, int rank, size_t *bytes);
/*
 * One Oja subspace step on activations X (rows x feats, dtype) and basis Q (feats x rank, fp32,
 * row-major), replacing the fp32 torch arithmetic of STACRLinear._refresh_basis
 * (stacr/layers.py:346-348) and OjaBasis.update (stacr/oja.py:73-79):
 *   Y = X Q;  update = X^T Y / max(1, rows) - Q (Y^T Y / max(1, rows));  out = Q + lr * update.
 * update and out are feats x rank fp32.  The caller re-orthonormalizes `out` (reduced QR,
 * stacr/oja.py:8-11, a library call).  Deterministic: every sum has a fixed order.
 */
int stacr_oja_step(const void *x, int dtype, int64_t rows, int64_t feats, const float *q, int rank, float lr,
                   float *update, float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * stacr_oja_step on a Y = X Q the caller already holds (rows x rank fp32, row-major; the adaptive
 * engine's save computes it in its projection pass, stacr_adaptive_save_y), so X is read once:
 * X^T Y and Y^T Y, then U and M as stacr_oja_step.  The post-forward Oja refresh of the adaptive
 * layer, stacr/adaptive.py:3311-3395, with its Y taken from the forward's projection.  Needs bf16
 * X (16-byte aligned, features a multiple of 8 and <= 8192), rank <= 16, rows > 0 and Y 16-byte
 * aligned with rows * rank a multiple of 4; otherwise STACR_ERR_UNSUPPORTED (use stacr_oja_step).
 * Workspace as stacr_oja_workspace_bytes.
 */
int stacr_oja_step_given_y(const void *x, int dtype, int64_t rows, int64_t feats, const float *q, int rank,
                           const float *y, float lr, float *update, float *out, void *workspace,
                           size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------- dense reconstruction */

/*
 * The dense activation a saved-tensor compressor hands back to autograd, replacing
 * STACRCompressor.unpack (stacr/compressor.py:127-133) and SparseResidual.dense
 * (stacr/residual.py:13-20):
 *   out = coeff Q^T                      (rows x feats, dtype; each element an fp32 chain over the
 *                                         rank, rounded once)
 *   out = out + dense(idx, values)       when has_residual (every element gets the addition, so
 *                                         -0 becomes +0 away from the entries, as in the reference)
 * coeff: rows x rank, q: feats x rank, values: nnz elements, all in dtype; idx: nnz flat indices
 * into rows x feats (index_bytes 4 or 8), unique (entries outside the tensor are skipped).
 * No workspace.
 */
int stacr_reconstruct(const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats, int rank,
                      const void *idx, int index_bytes, const void *values, int64_t nnz, int has_residual,
                      void *out, void *stream);

/* ---------------------------------------------------------------- compact save outputs
 * Bit-packed delta stream of sorted flat indices (a denser form of the delta codec,
 * stacr/index_compression.py:231-269; decoding gives decompress_indices' base + cumulative deltas,
 * :327-342).  Blocks of 256 entries: base[b] = idx[256 b] (int64); slot j holds
 * d_j = idx[256 b + j] - idx[256 b + j - 1] (d_0 = 0) in w_b bits, w_b the bit length of the
 * block's largest delta; the block's 256 slots fill 8 w_b uint32 words, slot j at bits
 * [j w_b, (j + 1) w_b), least significant bit first, unused slots 0.  word_off[b] (uint32, nb + 1
 * entries) is block b's first word; word_off[nb] is the stream's length in words.
 * sizes: nb = ceil(nnz / 256) and the longest stream, 256 nb words (nnz < 2^31). */
int stacr_index_stream_sizes(int64_t nnz, int64_t *blocks, int64_t *max_words);
/* idx: nnz int32 / int64 (idx_bytes 4 / 8), non-decreasing and non-negative.  base: int64[nb];
 * word_off: uint32[nb + 1]; words: uint32[max_words]; status: one uint32 on the device, set to the
 * OR of 1 (a decreasing pair), 2 (a gap of 2^32 or more) and 4 (a negative index); a nonzero status
 * means the stream does not hold the input (such deltas are stored as 0). */
int stacr_index_stream_encode(const void *idx, int idx_bytes, int64_t nnz, void *base, void *word_off, void *words,
                              void *status, void *stream);
/* The sorted indices back, as int32 or int64 (idx_bytes 4 / 8). */
int stacr_index_stream_decode(const void *base, const void *word_off, const void *words, int64_t nnz, void *idx,
                              int idx_bytes, void *stream);

/* ---------------------------------------------------------------- C1 checkpoint-boundary codec
 * pack_tensor (stacr/protocols/checkpointing.py:411-529) forms C = X Q in fp32 (the caller's GEMM,
 * as the reference's `flat_fp32 @ basis_fp32`); stacr_c1_observe then reads X once and reports
 * everything the reference inspects before it decides between a compressed record and a dense
 * fallback, and stacr_c1_store writes the record's coefficients; unpack_record (:531-545) is
 * stacr_c1_restore. */
#define STACR_DTYPE_I8 3 /* int8 coefficient codes (stacr_c1_store / stacr_c1_restore) */
#define STACR_C1_MAX_RANK 128
/* stats flags, per tensor (X, C, the reconstruction C Q^T, the residual X - C Q^T, the basis):
 * "holds a NaN" and "holds a value that is not NaN".  With the tensor's max below: non-finite =
 * NaN or max = inf; the reference's _safe_max_abs (:80-99) = NaN without a non-NaN value, FLT_MAX
 * with a NaN and an inf (torch.nan_to_num clamps the inf), else the max. */
#define STACR_C1_INPUT_NAN 1u
#define STACR_C1_COEFF_NAN 2u
#define STACR_C1_RECON_NAN 4u
#define STACR_C1_BASIS_NAN 8u
#define STACR_C1_INPUT_VALID 16u
#define STACR_C1_COEFF_VALID 32u
#define STACR_C1_RECON_VALID 64u
#define STACR_C1_RESIDUAL_VALID 128u
#define STACR_C1_BASIS_VALID 256u
#define STACR_C1_RESIDUAL_NAN 512u
typedef struct {
    double error;  /* sum over X of rnd32((x - p)^2), p = sum_j c_j q_j (fp32 chain), in fp64 */
    double denom;  /* sum of rnd32(x^2), in fp64 */
    float energy;  /* (float)error / max((float)denom, 1e-12) */
    float input_max_abs, coeff_max_abs, reconstruction_max_abs, residual_max_abs, basis_max_abs;
    /* (the largest |v| that is not NaN, inf included; 0 when there is none) */
    uint32_t flags;
    uint32_t reserved;
} StacrC1Stats;
int stacr_c1_workspace_bytes(int64_t rows, int64_t hidden, int rank, size_t *bytes);
/* x: rows x hidden (dtype); coeff: fp32 rows x rank; basis: hidden x rank (basis_dtype, widened to
 * fp32 as the reference's `basis.to(float32)`).  stats: one StacrC1Stats on the device; scales:
 * fp32[rank], s_j = (m_j finite and > 0 ? m_j : 1) / 127 with m_j = max |c_j| over the rows (NaN if
 * one is NaN).  Deterministic: the partial sums are combined in a fixed order. */
int stacr_c1_observe(const void *x, int dtype, int64_t rows, int64_t hidden, const float *coeff, const void *basis,
                     int basis_dtype, int rank, void *stats, float *scales, void *workspace, size_t workspace_bytes,
                     void *stream);
/* The record's coefficients: quantize -> int8 clamp(round half to even(c / s_j), -127, 127) (out_dtype
 * STACR_DTYPE_I8), else C rounded once to out_dtype (the basis dtype, :376-377). */
int stacr_c1_store(const float *coeff, int64_t rows, int rank, const float *scales, int quantize, void *out,
                   int out_dtype, void *stream);
/* out = sum_j c'_j q_j in fp32, rounded once to out_dtype; c' = code * s_j for coeff_dtype
 * STACR_DTYPE_I8, else the stored coefficient widened to fp32. */
int stacr_c1_restore(const void *coeff, int coeff_dtype, const float *scales, const void *basis, int basis_dtype,
                     int64_t rows, int64_t hidden, int rank, void *out, int out_dtype, void *stream);

/* int8 coefficients with one fp32 scale per row of C (rows x rank, dtype): m = max |c| over the
 * row (NaN if the row holds one), s = (m finite and > 0 ? m : 1) / 127, q = clamp(round half to even
 * (c / s), -127, 127), a NaN quotient coded 0.  codes: int8[rows * rank]; scales: float[rows]. */
int stacr_quantize_rows_int8(const void *coeff, int dtype, int64_t rows, int rank, void *codes, void *scales,
                             void *stream);
/* out = q * s in fp32, rounded once to out_dtype. */
int stacr_dequantize_rows_int8(const void *codes, const void *scales, int64_t rows, int rank, void *out,
                               int out_dtype, void *stream);

/*
 * Reduced QR of a tall fp32 matrix: replaces torch.linalg.qr(matrix, mode="reduced") in the basis
 * re-orthonormalization (stacr/oja.py:8-11 orthonormalize; stacr/adaptive.py:3368 after the
 * post-forward Oja step).  a: rows x cols, row-major fp32; q: rows x cols (row-major), r: cols x
 * cols upper triangular (row-major; NULL: not written).  LAPACK's Householder convention (as
 * torch's QR): R[j][j] = -sign(alpha_j) * norm, a reflector with tau = 0 where the column below the
 * diagonal is zero; the same result on every run.  One workgroup, the matrix in LDS:
 * STACR_ERR_UNSUPPORTED unless cols <= 16 and rows * cols <= 32768; cols <= rows.
 */
int stacr_qr(const float *a, int64_t rows, int cols, float *q, float *r, void *stream);

/*
 * The same reduced QR for any tall matrix of cols <= 16 (rows >= cols), e.g. the 8192 x 16 basis of a
 * wide layer (stacr_amd's wrapper takes it past 8192 elements, where it is the faster of the two):
 * replaces torch.linalg.qr(matrix, mode="reduced") at the same call sites (stacr/oja.py:8-11,
 * stacr/adaptive.py:3368).  Q and R as stacr_qr (LAPACK's signs), by
 * CholeskyQR in fp64 with the signs recovered from Q's top block; a matrix whose columns are within
 * 1e-5 of dependent (or whose sign decision is that close) takes LAPACK's Householder QR in one
 * workgroup instead.  Three launches; the workspace (workspace_bytes from
 * stacr_qr_tall_workspace_bytes, 8-byte aligned) holds the partial Gram matrices and the product.
 */
int stacr_qr_tall_workspace_bytes(int64_t rows, int cols, size_t *bytes);
int stacr_qr_tall(const float *a, int64_t rows, int cols, float *q, float *r, void *workspace,
                  size_t workspace_bytes, void *stream);

/*
 * Kernel timing (benchmarking aid; no counterpart in the reference).  Between begin and end,
 * every kernel this library launches is bracketed by HIP events on its stream, preceded by a
 * `sleep_us` device-side sleep so host enqueue gaps are not measured (up to max_launches
 * launches are recorded).  end synchronises the recorded events and returns, per kernel name in
 * first-launch order, the summed milliseconds and launch count (names: 64-byte slots).
 * A session is process wide: it records the launches of every thread (an autograd worker's
 * included).  Do not enable during stream capture.
 */
int stacr_profile_begin(int max_launches, double sleep_us);
int stacr_profile_end(int max_kernels, char *names, double *total_ms, int *launches, int *n_kernels);

#ifdef __cplusplus
}
#endif

#endif /* STACR_AMD_H */
