// C ABI entry points: argument validation, the reference's k rules, error reporting.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "internal.h"

namespace {

thread_local char g_err[512] = "";

// Python's round() of a double: nearest integer, ties to even (stacr/layers.py:25,33,51).
int64_t py_round(double v) { return (int64_t)nearbyint(v); }

// stacr/layers.py:33: k = max(1, min(n, round(budget * n)))
int64_t chunk_k(int64_t n, double budget)
{
    int64_t k = py_round(budget * (double)n);
    if (k > n) k = n;
    return k < 1 ? 1 : k;
}

bool valid_dtype(int dt) { return dt == STACR_DTYPE_F32 || dt == STACR_DTYPE_BF16 || dt == STACR_DTYPE_F16; }

struct KPlan {
    int64_t k_total = 0, k_full = 0, k_last = 0, k_sum = 0, k_saved = 0, chunk_rows = 1;
};

// k rules: stacr/layers.py:25-27 (chunk_topk total), :33 (per chunk), :38-40 (trim), :51-53 (global)
int plan_k(int64_t rows, int64_t feats, int mode, double budget, int64_t chunk_rows, KPlan *p)
{
    if (rows < 0 || feats < 0) return stacr_fail(STACR_ERR_INVALID, "negative shape (%lld x %lld)", (long long)rows, (long long)feats);
    if (mode != STACR_MODE_CHUNK_TOPK && mode != STACR_MODE_GLOBAL_TOPK)
        return stacr_fail(STACR_ERR_INVALID, "unknown residual mode %d", mode);
    if (!(budget >= 0.0 && budget <= 1.0)) return stacr_fail(STACR_ERR_INVALID, "budget %g outside [0, 1]", budget);
    if (mode == STACR_MODE_CHUNK_TOPK && chunk_rows < 1)
        return stacr_fail(STACR_ERR_INVALID, "chunk_rows must be positive");
    *p = KPlan{};
    const int64_t total = rows * feats;
    if (total == 0 || budget <= 0.0) return STACR_OK;
    p->k_total = py_round(budget * (double)total);
    if (p->k_total <= 0) { p->k_total = 0; return STACR_OK; }
    if (mode == STACR_MODE_GLOBAL_TOPK) {
        p->chunk_rows = rows;
        p->k_full = p->k_last = p->k_sum = p->k_saved = p->k_total;
        return STACR_OK;
    }
    const int64_t cr = chunk_rows < rows ? chunk_rows : rows;
    const int64_t n_chunks = (rows + cr - 1) / cr;
    const int64_t last_rows = rows - (n_chunks - 1) * cr;
    p->chunk_rows = cr;
    p->k_full = chunk_k(cr * feats, budget);
    p->k_last = chunk_k(last_rows * feats, budget);
    p->k_sum = (n_chunks - 1) * p->k_full + p->k_last;
    p->k_saved = p->k_sum > p->k_total ? p->k_total : p->k_sum;
    return STACR_OK;
}

}  // namespace

int stacr_fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int stacr_hip_check(hipError_t err, const char *what)
{
    if (err == hipSuccess) return STACR_OK;
    return stacr_fail(STACR_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

extern "C" {

int stacr_abi_version(void) { return STACR_ABI_VERSION; }

const char *stacr_last_error(void) { return g_err; }

int stacr_residual_plan(int64_t rows, int64_t feats, int mode, double budget, int64_t chunk_rows,
                        int64_t *k_total, int64_t *k_saved, int *index_bytes)
{
    KPlan p;
    const int rc = plan_k(rows, feats, mode, budget, chunk_rows, &p);
    if (rc) return rc;
    if (k_total) *k_total = p.k_total;
    if (k_saved) *k_saved = p.k_saved;
    if (index_bytes) *index_bytes = rows * feats < 2147483647LL ? 4 : 8;  // stacr/layers.py:41
    return STACR_OK;
}

static int fill_save_args(int64_t rows, int64_t feats, int rank, int dtype, int mode, double budget,
                          int64_t chunk_rows, int bits, StacrSaveArgs *a)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported activation dtype code %d", dtype);
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (bits != 0 && bits != 4 && bits != 8) return stacr_fail(STACR_ERR_INVALID, "residual_bits must be 0, 4, or 8");
    KPlan p;
    const int rc = plan_k(rows, feats, mode, budget, chunk_rows, &p);
    if (rc) return rc;
    if ((uint64_t)rows * (uint64_t)feats >= (1ull << 32))
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rows*feats = %lld exceeds 2^32 elements",
                          (long long)(rows * feats));
    *a = StacrSaveArgs{};
    a->dtype = dtype;
    a->rows = rows;
    a->feats = feats;
    a->rank = rank;
    a->mode = mode;
    a->chunk_rows = p.chunk_rows;
    a->k_total = p.k_total;
    a->k_full = p.k_full;
    a->k_last = p.k_last;
    a->k_sum = p.k_sum;
    a->bits = bits;
    return STACR_OK;
}

int stacr_save_workspace_bytes(int64_t rows, int64_t feats, int rank, int dtype, int mode, double budget,
                               int64_t chunk_rows, int bits, size_t *bytes)
{
    if (!bytes) return stacr_fail(STACR_ERR_INVALID, "bytes is NULL");
    StacrSaveArgs a;
    const int rc = fill_save_args(rows, feats, rank, dtype, mode, budget, chunk_rows, bits, &a);
    if (rc) return rc;
    *bytes = rows * feats ? stacr_save_ws_layout(a, nullptr) : 0;
    return STACR_OK;
}

static int save_impl(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank, int mode,
                     double budget, int64_t chunk_rows, int bits, void *coeff, void *idx, int index_bytes, void *data,
                     float *scale, void *workspace, size_t workspace_bytes, void *stream, void *census,
                     size_t census_bytes, int *census_written)
{
    if (census_written) *census_written = 0;
    StacrSaveArgs a;
    int rc = fill_save_args(rows, feats, rank, dtype, mode, budget, chunk_rows, bits, &a);
    if (rc) return rc;
    if (rows * feats == 0) return STACR_OK;
    if (!x || !q || !coeff) return stacr_fail(STACR_ERR_INVALID, "stacr_save: x, q and coeff must be non-NULL");
    if (a.k_total > 0) {
        if (!idx || !data || !scale) return stacr_fail(STACR_ERR_INVALID, "stacr_save: idx, data, scale must be non-NULL");
        const int want = rows * feats < 2147483647LL ? 4 : 8;
        if (index_bytes != want)
            return stacr_fail(STACR_ERR_INVALID, "stacr_save: index_bytes must be %d for %lld elements", want,
                              (long long)(rows * feats));
    }
    if (!workspace) return stacr_fail(STACR_ERR_INVALID, "stacr_save: workspace is NULL");
    a.x = x;
    a.q = q;
    a.coeff = coeff;
    a.idx = idx;
    a.index_bytes = index_bytes;
    a.data = data;
    a.scale = scale;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    a.stream = static_cast<hipStream_t>(stream);
    if (census) {
        if (census_bytes < (size_t)census_words(rows, feats) * 4)
            return stacr_fail(STACR_ERR_INVALID, "stacr_save_census: census has %zu bytes, needs %zu", census_bytes,
                              (size_t)census_words(rows, feats) * 4);
        a.census = static_cast<uint32_t *>(census);
        a.census_written = census_written;
    }
    return stacr_save_launch(a);
}

int stacr_save(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank, int mode,
               double budget, int64_t chunk_rows, int bits, void *coeff, void *idx, int index_bytes, void *data,
               float *scale, void *workspace, size_t workspace_bytes, void *stream)
{
    return save_impl(x, q, dtype, rows, feats, rank, mode, budget, chunk_rows, bits, coeff, idx, index_bytes, data,
                     scale, workspace, workspace_bytes, stream, nullptr, 0, nullptr);
}

int stacr_save_census_bytes(int64_t rows, int64_t feats, size_t *bytes)
{
    if (rows < 0 || feats < 0 || !bytes) return stacr_fail(STACR_ERR_INVALID, "stacr_save_census_bytes: bad argument");
    *bytes = (size_t)census_words(rows, feats) * 4;
    return STACR_OK;
}

int stacr_save_census(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank, int mode,
                      double budget, int64_t chunk_rows, int bits, void *coeff, void *idx, int index_bytes, void *data,
                      float *scale, void *workspace, size_t workspace_bytes, void *census, size_t census_bytes,
                      int *census_written, void *stream)
{
    if (!census || !census_written)
        return stacr_fail(STACR_ERR_INVALID, "stacr_save_census: census and census_written must be non-NULL");
    return save_impl(x, q, dtype, rows, feats, rank, mode, budget, chunk_rows, bits, coeff, idx, index_bytes, data,
                     scale, workspace, workspace_bytes, stream, census, census_bytes, census_written);
}

int stacr_select_residual(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                          int rank, int mode, double budget, int64_t chunk_rows, int bits, void *idx,
                          int index_bytes, void *data, float *scale, void *workspace, size_t workspace_bytes,
                          void *stream)
{
    StacrSaveArgs a;
    int rc = fill_save_args(rows, feats, rank, dtype, mode, budget, chunk_rows, bits, &a);
    if (rc) return rc;
    if (rows * feats == 0 || a.k_total == 0) return STACR_OK;
    if (!x || !q || !coeff || !idx || !data || !scale || !workspace)
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_residual: NULL pointer argument");
    const int want = rows * feats < 2147483647LL ? 4 : 8;
    if (index_bytes != want)
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_residual: index_bytes must be %d", want);
    a.x = x;
    a.q = q;
    a.coeff_in = coeff;
    a.coeff = nullptr;
    a.idx = idx;
    a.index_bytes = index_bytes;
    a.data = data;
    a.scale = scale;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    a.stream = static_cast<hipStream_t>(stream);
    return stacr_save_launch(a);
}

int stacr_quantize_values(const void *values, int dtype, int64_t n, int bits, void *data, float *scale,
                          void *workspace, size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported value dtype code %d", dtype);
    if (bits != 4 && bits != 8) return stacr_fail(STACR_ERR_INVALID, "stacr_quantize_values: bits must be 4 or 8");
    if (n < 0) return stacr_fail(STACR_ERR_INVALID, "negative length");
    if (n == 0) return STACR_OK;
    if (!values || !data || !scale || !workspace) return stacr_fail(STACR_ERR_INVALID, "NULL pointer argument");
    if (workspace_bytes < 4) return stacr_fail(STACR_ERR_WORKSPACE, "stacr_quantize_values needs 4 workspace bytes");
    return stacr_quantize_launch(values, dtype, n, bits, data, scale, workspace, static_cast<hipStream_t>(stream));
}

static int fill_grad_args(int64_t rows, int64_t d_out, int64_t d_in, int rank, int64_t nnz, StacrGradArgs *a)
{
    if (rows < 0 || d_out < 0 || d_in < 0 || nnz < 0) return stacr_fail(STACR_ERR_INVALID, "negative size");
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (nnz > rows * d_in) return stacr_fail(STACR_ERR_INVALID, "nnz exceeds rows*d_in");
    if (nnz >= (1ll << 31)) return stacr_fail(STACR_ERR_UNSUPPORTED, "nnz %lld >= 2^31", (long long)nnz);
    *a = StacrGradArgs{};
    a->rows = rows;
    a->d_out = d_out;
    a->d_in = d_in;
    a->rank = rank;
    a->nnz = nnz;
    return STACR_OK;
}

int stacr_weight_grad_workspace_bytes(int64_t rows, int64_t d_out, int64_t d_in, int rank, int64_t nnz, size_t *bytes)
{
    if (!bytes) return stacr_fail(STACR_ERR_INVALID, "bytes is NULL");
    StacrGradArgs a;
    const int rc = fill_grad_args(rows, d_out, d_in, rank, nnz, &a);
    if (rc) return rc;
    // the query does not know the dtypes, alignment or bias: enough for whichever path runs
    const size_t legacy = stacr_grad_ws_layout(a, nullptr), tiles = stacr_tiles_ws_bound(rows, d_out, d_in, nnz);
    *bytes = legacy > tiles ? legacy : tiles;
    return STACR_OK;
}

static int grad_impl(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff, const void *q,
                     int64_t d_in, int rank, const void *idx, int index_bytes, const void *data, const float *scale,
                     int bits, int val_dtype, int64_t nnz, int transposed, void *dw, int dw_dtype, void *dbias,
                     int dbias_dtype, void *workspace, size_t workspace_bytes, void *stream, const void *census)
{
    StacrGradArgs a;
    int rc = fill_grad_args(rows, d_out, d_in, rank, nnz, &a);
    if (rc) return rc;
    if (!valid_dtype(dtype) || !valid_dtype(dw_dtype) || (dbias && !valid_dtype(dbias_dtype)))
        return stacr_fail(STACR_ERR_INVALID, "unsupported dtype code");
    if (bits != 0 && bits != 4 && bits != 8) return stacr_fail(STACR_ERR_INVALID, "residual_bits must be 0, 4, or 8");
    if (nnz > 0) {
        if (!idx || !data || (bits && !scale)) return stacr_fail(STACR_ERR_INVALID, "sparse residual pointers are NULL");
        if (index_bytes != 4 && index_bytes != 8) return stacr_fail(STACR_ERR_INVALID, "index_bytes must be 4 or 8");
        if (bits == 0 && !valid_dtype(val_dtype)) return stacr_fail(STACR_ERR_INVALID, "bad value dtype");
    }
    if (d_out * d_in == 0) return STACR_OK;
    if (!dw || !q || (rows > 0 && (!g || !coeff)) || !workspace)
        return stacr_fail(STACR_ERR_INVALID, "stacr_weight_grad: NULL pointer argument");
    a.g = g;
    a.dtype = dtype;
    a.coeff = coeff;
    a.q = q;
    a.idx = idx;
    a.index_bytes = index_bytes;
    a.data = data;
    a.scale = scale;
    a.bits = bits;
    a.val_dtype = val_dtype;
    a.transposed = transposed ? 1 : 0;
    a.dw = dw;
    a.dw_dtype = dw_dtype;
    a.dbias = dbias;
    a.dbias_dtype = dbias_dtype;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    a.stream = static_cast<hipStream_t>(stream);
    a.census = static_cast<const uint32_t *>(census);
    return stacr_grad_launch(a);
}

int stacr_weight_grad(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff, const void *q,
                      int64_t d_in, int rank, const void *idx, int index_bytes, const void *data, const float *scale,
                      int bits, int val_dtype, int64_t nnz, int transposed, void *dw, int dw_dtype, void *dbias,
                      int dbias_dtype, void *workspace, size_t workspace_bytes, void *stream)
{
    return grad_impl(g, dtype, rows, d_out, coeff, q, d_in, rank, idx, index_bytes, data, scale, bits, val_dtype, nnz,
                     transposed, dw, dw_dtype, dbias, dbias_dtype, workspace, workspace_bytes, stream, nullptr);
}

int stacr_weight_grad_census(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff, const void *q,
                             int64_t d_in, int rank, const void *idx, int index_bytes, const void *data,
                             const float *scale, int bits, int val_dtype, int64_t nnz, int transposed, void *dw,
                             int dw_dtype, void *dbias, int dbias_dtype, const void *census, size_t census_bytes,
                             void *workspace, size_t workspace_bytes, void *stream)
{
    if (!census) return stacr_fail(STACR_ERR_INVALID, "stacr_weight_grad_census: census is NULL");
    if (rows < 0 || d_in < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_weight_grad_census: bad shape");
    const size_t need = (size_t)census_words(rows, d_in) * 4;
    if (census_bytes < need)
        return stacr_fail(STACR_ERR_INVALID, "stacr_weight_grad_census: census has %zu bytes, this problem's needs %zu",
                          census_bytes, need);
    return grad_impl(g, dtype, rows, d_out, coeff, q, d_in, rank, idx, index_bytes, data, scale, bits, val_dtype, nnz,
                     transposed, dw, dw_dtype, dbias, dbias_dtype, workspace, workspace_bytes, stream, census);
}

}  // extern "C"

// ------------------------------------------------------------------ adaptive engine
namespace {

struct AdaptivePlan {
    int64_t k = 0, k_full = 0, k_last = 0, k_sum = 0, k_saved = 0, chunk_rows = 1;
    int index_bytes = 4;
};

// stacr/adaptive.py:1357-1365,1492,1524-1530 and _choose_index_dtype (:138-159)
int plan_adaptive(int64_t rows, int64_t feats, double budget, int64_t chunk_rows, AdaptivePlan *p)
{
    if (rows < 0 || feats < 0) return stacr_fail(STACR_ERR_INVALID, "negative shape");
    if (!(budget >= 0.0 && budget <= 1.0)) return stacr_fail(STACR_ERR_INVALID, "residual_budget must be in [0, 1]");
    if (chunk_rows < 1) return stacr_fail(STACR_ERR_INVALID, "chunk_rows must be positive");
    *p = AdaptivePlan{};
    const int64_t total = rows * feats;
    p->index_bytes = total < 32768 ? 2 : (total <= (1ll << 31) ? 4 : 8);
    if (total == 0) return STACR_OK;
    int64_t k = (int64_t)((double)total * budget);  // Python int() of a positive float truncates
    if (k <= 0) return STACR_OK;
    k = stacr::hmin(k, total);
    const int64_t chunk = stacr::hmin(chunk_rows, rows);
    const int64_t pck = stacr::hmax<int64_t>(1, (k * chunk + rows - 1) / rows);
    const int64_t n_chunks = (rows + chunk - 1) / chunk;
    const int64_t last_rows = rows - (n_chunks - 1) * chunk;
    p->k = k;
    p->chunk_rows = chunk;
    p->k_full = stacr::hmin(pck, chunk * feats);
    p->k_last = stacr::hmin(pck, last_rows * feats);
    p->k_sum = p->k_full * (n_chunks - 1) + p->k_last;
    p->k_saved = stacr::hmin(p->k_sum, k);
    return STACR_OK;
}

int fill_adaptive_args(int64_t rows, int64_t feats, int rank, int dtype, double budget, int64_t chunk_rows,
                       StacrSaveArgs *a, AdaptivePlan *p)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported activation dtype code %d", dtype);
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    const int rc = plan_adaptive(rows, feats, budget, chunk_rows, p);
    if (rc) return rc;
    if ((uint64_t)rows * (uint64_t)feats >= (1ull << 32))
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rows*feats = %lld exceeds 2^32 elements", (long long)(rows * feats));
    *a = StacrSaveArgs{};
    a->dtype = dtype;
    a->rows = rows;
    a->feats = feats;
    a->rank = rank;
    a->mode = STACR_MODE_CHUNK_TOPK;
    a->chunk_rows = p->chunk_rows;
    a->k_total = p->k;
    a->k_full = p->k_full;
    a->k_last = p->k_last;
    a->k_sum = p->k_sum;
    a->bits = 0;
    return STACR_OK;
}

}  // namespace

int stacr_adaptive_residual_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows, int64_t *k,
                                 int64_t *k_saved, int *index_bytes)
{
    AdaptivePlan p;
    const int rc = plan_adaptive(rows, feats, budget, chunk_rows, &p);
    if (rc) return rc;
    if (k) *k = p.k;
    if (k_saved) *k_saved = p.k_saved;
    if (index_bytes) *index_bytes = p.index_bytes;
    return STACR_OK;
}

namespace {

// Workspace of an adaptive save: the save's own, then the energies' (the separate pass's partials, or
// the projection pass's per-workgroup partials, whichever is larger).
int adaptive_ws(const StacrSaveArgs &a, size_t *save, size_t *energy_off, size_t *total)
{
    *save = a.rows * a.feats ? stacr_save_ws_layout(a, nullptr) : 0;
    *energy_off = (*save + 255) & ~(size_t)255;
    const int64_t slots = a.rows * a.feats ? stacr_save_energy_slots(a) : 0;
    const size_t parts = ((size_t)slots * kEnergyStride * sizeof(float) + 255) & ~(size_t)255;
    *total = *energy_off + stacr::hmax(stacr_energy_ws(), parts + stacr_energy_fold_ws());
    return STACR_OK;
}

int fill_adaptive_y(int64_t rows, int64_t feats, int q_cols, int rank, int dtype, double budget, int64_t chunk_rows,
                    float *y, StacrSaveArgs *a, AdaptivePlan *p)
{
    int rc = fill_adaptive_args(rows, feats, rank, dtype, budget, chunk_rows, a, p);
    if (rc) return rc;
    if (q_cols < rank || q_cols > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_INVALID, "q_cols %d outside rank..%d", q_cols, STACR_MAX_RANK);
    a->q_ld = q_cols;
    a->y_cols = q_cols;
    a->y_out = y;
    return STACR_OK;
}

// a placeholder address marking "Y requested" for the planning queries (never written through)
float *const kYPlanned = reinterpret_cast<float *>(alignof(float));

int adaptive_save_impl(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int q_cols, int rank,
                       double budget, int64_t chunk_rows, const void *coeff_in, void *coeff, void *idx,
                       int index_bytes, void *values, float *energy, float *y, int *y_written, void *workspace,
                       size_t workspace_bytes, void *stream, const char *who)
{
    if (y_written) *y_written = 0;
    StacrSaveArgs a;
    AdaptivePlan p;
    int rc = fill_adaptive_y(rows, feats, q_cols, rank, dtype, budget, chunk_rows, y, &a, &p);
    if (rc) return rc;
    if (rows * feats == 0) return STACR_OK;
    if (!x || !q || (!coeff && !coeff_in) || !workspace)
        return stacr_fail(STACR_ERR_INVALID, "%s: x, q, coeff (or coeff_in) and workspace must be non-NULL", who);
    if (p.k > 0) {
        if (!idx || !values) return stacr_fail(STACR_ERR_INVALID, "%s: idx and values must be non-NULL", who);
        if (index_bytes != p.index_bytes)
            return stacr_fail(STACR_ERR_INVALID, "%s: index_bytes must be %d", who, p.index_bytes);
    }
    size_t save, off_energy, need;
    adaptive_ws(a, &save, &off_energy, &need);
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "%s: workspace has %zu bytes, needs %zu", who, workspace_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t slots = energy ? stacr_save_energy_slots(a) : 0;
    float *epart = reinterpret_cast<float *>(static_cast<char *>(workspace) + off_energy);
    int energy_fused = 0;
    a.x = x;
    a.q = q;
    a.coeff_in = coeff_in;
    a.coeff = coeff_in ? nullptr : coeff;
    a.idx = idx;
    a.index_bytes = index_bytes;
    a.data = values;
    a.scale = nullptr;
    a.workspace = workspace;
    a.workspace_bytes = save;
    a.stream = s;
    a.y_written = y_written;
    a.energy_part = slots ? epart : nullptr;
    a.energy_written = &energy_fused;
    rc = stacr_save_launch(a);
    if (rc) return rc;
    if (!energy) return STACR_OK;
    // the projection pass formed the energy partials (one read of X), else a pass of its own
    if (energy_fused) {
        char *fold_ws = reinterpret_cast<char *>(epart) + (((size_t)slots * kEnergyStride * sizeof(float) + 255) & ~(size_t)255);
        return stacr_energy_fold_launch(epart, slots, dtype, rows, rank, energy, fold_ws, s);
    }
    return stacr_energy_launch(x, coeff_in ? coeff_in : coeff, dtype, rows, feats, rank, energy, epart, s);
}

}  // namespace

int stacr_adaptive_save_workspace_bytes(int64_t rows, int64_t feats, int rank, int dtype, double budget,
                                        int64_t chunk_rows, size_t *bytes)
{
    return stacr_adaptive_save_y_workspace_bytes(rows, feats, rank, rank, dtype, budget, chunk_rows, bytes);
}

int stacr_adaptive_save_y_workspace_bytes(int64_t rows, int64_t feats, int q_cols, int rank, int dtype, double budget,
                                          int64_t chunk_rows, size_t *bytes)
{
    if (!bytes) return stacr_fail(STACR_ERR_INVALID, "bytes is NULL");
    StacrSaveArgs a;
    AdaptivePlan p;
    size_t save, off, need = 0;
    // with or without Y the plans can differ (Y over more columns takes the wide pass): the larger
    for (int with_y = 0; with_y < 2; ++with_y) {
        const int rc = fill_adaptive_y(rows, feats, q_cols, rank, dtype, budget, chunk_rows,
                                       with_y ? kYPlanned : nullptr, &a, &p);
        if (rc) return rc;
        size_t t;
        adaptive_ws(a, &save, &off, &t);
        need = stacr::hmax(need, t);
    }
    *bytes = need;
    return STACR_OK;
}

int stacr_adaptive_save(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int rank, double budget,
                        int64_t chunk_rows, const void *coeff_in, void *coeff, void *idx, int index_bytes, void *values,
                        float *energy, void *workspace, size_t workspace_bytes, void *stream)
{
    return adaptive_save_impl(x, q, dtype, rows, feats, rank, rank, budget, chunk_rows, coeff_in, coeff, idx,
                              index_bytes, values, energy, nullptr, nullptr, workspace, workspace_bytes, stream,
                              "stacr_adaptive_save");
}

int stacr_adaptive_save_y(const void *x, const void *q, int dtype, int64_t rows, int64_t feats, int q_cols, int rank,
                          double budget, int64_t chunk_rows, const void *coeff_in, void *coeff, void *idx,
                          int index_bytes, void *values, float *energy, float *y, int *y_written, void *workspace,
                          size_t workspace_bytes, void *stream)
{
    return adaptive_save_impl(x, q, dtype, rows, feats, q_cols, rank, budget, chunk_rows, coeff_in, coeff, idx,
                              index_bytes, values, energy, y, y_written, workspace, workspace_bytes, stream,
                              "stacr_adaptive_save_y");
}

int stacr_adaptive_quantize(const void *values, int dtype, int64_t n, int bits, void *data, void *scale,
                            void *workspace, size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported value dtype code %d", dtype);
    if (bits != 4 && bits != 8) return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_quantize: bits must be 4 or 8");
    if (n < 0) return stacr_fail(STACR_ERR_INVALID, "negative length");
    if (!scale || !workspace || (n > 0 && (!values || !data)))
        return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_quantize: NULL pointer argument");
    if (workspace_bytes < 4) return stacr_fail(STACR_ERR_WORKSPACE, "stacr_adaptive_quantize needs 4 workspace bytes");
    return stacr_aq_quantize_launch(values, dtype, n, bits, data, scale, workspace, static_cast<hipStream_t>(stream));
}

int stacr_adaptive_dequantize(const void *data, int bits, const void *scale, int64_t n, void *out, int out_dtype,
                              void *stream)
{
    if (bits != 4 && bits != 8) return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_dequantize: bits must be 4 or 8");
    if (!valid_dtype(out_dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported output dtype code %d", out_dtype);
    if (n < 0) return stacr_fail(STACR_ERR_INVALID, "negative length");
    if (n > 0 && (!data || !scale || !out)) return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_dequantize: NULL pointer");
    return stacr_aq_dequantize_launch(data, bits, scale, n, out, out_dtype, static_cast<hipStream_t>(stream));
}

static bool valid_int_bytes(int b) { return b == 2 || b == 4 || b == 8; }

int stacr_csr_encode(const void *idx, int idx_bytes, int64_t nnz, int64_t rows, int64_t n_cols, void *row_ptrs,
                     int ptr_bytes, void *cols, int col_bytes, void *stream)
{
    if (!valid_int_bytes(idx_bytes) || !valid_int_bytes(col_bytes) || (ptr_bytes != 4 && ptr_bytes != 8))
        return stacr_fail(STACR_ERR_INVALID, "stacr_csr_encode: bad integer width");
    if (nnz < 0 || rows < 0 || n_cols < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_csr_encode: bad size");
    if (!row_ptrs || (nnz > 0 && (!idx || !cols))) return stacr_fail(STACR_ERR_INVALID, "stacr_csr_encode: NULL pointer");
    return stacr_csr_encode_launch(idx, idx_bytes, nnz, rows, n_cols, row_ptrs, ptr_bytes, cols, col_bytes,
                                   static_cast<hipStream_t>(stream));
}

int stacr_csr_decode(const void *row_ptrs, int ptr_bytes, const void *cols, int col_bytes, int64_t rows,
                     int64_t n_cols, int64_t nnz, void *idx, int idx_bytes, void *stream)
{
    if (!valid_int_bytes(idx_bytes) || !valid_int_bytes(col_bytes) || (ptr_bytes != 4 && ptr_bytes != 8))
        return stacr_fail(STACR_ERR_INVALID, "stacr_csr_decode: bad integer width");
    if (nnz < 0 || rows < 1 || n_cols < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_csr_decode: bad size");
    if (nnz > 0 && (!row_ptrs || !cols || !idx)) return stacr_fail(STACR_ERR_INVALID, "stacr_csr_decode: NULL pointer");
    return stacr_csr_decode_launch(row_ptrs, ptr_bytes, cols, col_bytes, rows, n_cols, nnz, idx, idx_bytes,
                                   static_cast<hipStream_t>(stream));
}

int stacr_delta_max(const void *idx, int idx_bytes, int64_t nnz, void *max_delta, void *stream)
{
    if (!valid_int_bytes(idx_bytes)) return stacr_fail(STACR_ERR_INVALID, "stacr_delta_max: bad integer width");
    if (nnz < 0 || !max_delta || (nnz > 0 && !idx)) return stacr_fail(STACR_ERR_INVALID, "stacr_delta_max: bad argument");
    return stacr_delta_max_launch(idx, idx_bytes, nnz, max_delta, static_cast<hipStream_t>(stream));
}

int stacr_delta_encode(const void *idx, int idx_bytes, int64_t nnz, void *base, int base_bytes, void *deltas,
                       int delta_bytes, void *stream)
{
    if (!valid_int_bytes(idx_bytes) || !valid_int_bytes(delta_bytes) || (base_bytes != 4 && base_bytes != 8))
        return stacr_fail(STACR_ERR_INVALID, "stacr_delta_encode: bad integer width");
    if (nnz < 0 || (nnz > 0 && (!idx || !base)) || (nnz > 1 && !deltas))
        return stacr_fail(STACR_ERR_INVALID, "stacr_delta_encode: bad argument");
    return stacr_delta_encode_launch(idx, idx_bytes, nnz, base, base_bytes, deltas, delta_bytes,
                                     static_cast<hipStream_t>(stream));
}

int stacr_delta_decode_workspace_bytes(int64_t nnz, size_t *bytes)
{
    if (!bytes || nnz < 0) return stacr_fail(STACR_ERR_INVALID, "stacr_delta_decode_workspace_bytes: bad argument");
    *bytes = stacr_delta_decode_ws(nnz);
    return STACR_OK;
}

int stacr_delta_decode(const void *base, int base_bytes, const void *deltas, int delta_bytes, int64_t nnz, void *idx,
                       int idx_bytes, void *workspace, size_t workspace_bytes, void *stream)
{
    if (!valid_int_bytes(idx_bytes) || !valid_int_bytes(delta_bytes) || (base_bytes != 4 && base_bytes != 8))
        return stacr_fail(STACR_ERR_INVALID, "stacr_delta_decode: bad integer width");
    if (nnz < 0 || (nnz > 0 && (!base || !idx || !workspace)) || (nnz > 1 && !deltas))
        return stacr_fail(STACR_ERR_INVALID, "stacr_delta_decode: bad argument");
    if (workspace_bytes < stacr_delta_decode_ws(nnz))
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_delta_decode: workspace too small");
    return stacr_delta_decode_launch(base, base_bytes, deltas, delta_bytes, nnz, idx, idx_bytes, workspace,
                                     static_cast<hipStream_t>(stream));
}

int stacr_oja_workspace_bytes(int64_t rows, int64_t feats, int rank, size_t *bytes)
{
    if (!bytes || rows < 0 || feats < 0) return stacr_fail(STACR_ERR_INVALID, "stacr_oja_workspace_bytes: bad argument");
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    *bytes = stacr_oja_ws_bytes(rows, feats, rank);
    return STACR_OK;
}

int stacr_oja_step(const void *x, int dtype, int64_t rows, int64_t feats, const float *q, int rank, float lr,
                   float *update, float *out, void *workspace, size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported activation dtype code %d", dtype);
    if (rows < 0 || feats < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step: bad shape");
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (!q || !update || !out || !workspace || (rows > 0 && !x))
        return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step: NULL pointer argument");
    if (!isfinite(lr)) return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step: lr must be finite");
    const size_t need = stacr_oja_ws_bytes(rows, feats, rank);
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_oja_step: workspace has %zu bytes, needs %zu", workspace_bytes, need);
    return stacr_oja_launch(x, dtype, rows, feats, q, rank, lr, update, out, workspace, static_cast<hipStream_t>(stream));
}

int stacr_oja_step_given_y(const void *x, int dtype, int64_t rows, int64_t feats, const float *q, int rank,
                           const float *y, float lr, float *update, float *out, void *workspace,
                           size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "unsupported activation dtype code %d", dtype);
    if (rows < 0 || feats < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step_given_y: bad shape");
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (!q || !update || !out || !workspace || (rows > 0 && (!x || !y)))
        return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step_given_y: NULL pointer argument");
    if (!isfinite(lr)) return stacr_fail(STACR_ERR_INVALID, "stacr_oja_step_given_y: lr must be finite");
    if (!stacr_oja_given_y_ok(dtype, rows, feats, rank, x, y))
        return stacr_fail(STACR_ERR_UNSUPPORTED,
                          "stacr_oja_step_given_y: needs bf16 X (16-byte aligned, features a multiple of 8, at most "
                          "8192), rank <= 16, rows > 0, and Y 16-byte aligned with rows * rank a multiple of 4");
    const size_t need = stacr_oja_ws_bytes(rows, feats, rank);
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_oja_step_given_y: workspace has %zu bytes, needs %zu",
                          workspace_bytes, need);
    return stacr_oja_given_y_launch(x, rows, feats, q, rank, y, lr, update, out, workspace,
                                    static_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------ uniform / block_sparse / sampled
namespace {

int check_factors(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats, int rank,
                  const char *who)
{
    if (!valid_dtype(dtype)) return stacr_fail(STACR_ERR_INVALID, "%s: unsupported dtype code %d", who, dtype);
    if (rows < 0 || feats < 1) return stacr_fail(STACR_ERR_INVALID, "%s: bad shape", who);
    if (rank < 1 || rank > STACR_MAX_RANK)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rank %d outside 1..%d", rank, STACR_MAX_RANK);
    if (rows * feats >= (1ll << 32))
        return stacr_fail(STACR_ERR_UNSUPPORTED, "rows*feats = %lld exceeds 2^32 elements", (long long)(rows * feats));
    if (rows > 0 && (!x || !coeff || !q)) return stacr_fail(STACR_ERR_INVALID, "%s: NULL pointer argument", who);
    return STACR_OK;
}

int index_bytes_for(int64_t total) { return total < (1ll << 31) - 1 ? 4 : 8; }

}  // namespace

int stacr_select_uniform(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                         int rank, int64_t k, void *idx, int index_bytes, void *values, void *stream)
{
    int rc = check_factors(x, coeff, q, dtype, rows, feats, rank, "stacr_select_uniform");
    if (rc) return rc;
    if (k < 0 || k > rows * feats) return stacr_fail(STACR_ERR_INVALID, "stacr_select_uniform: k outside [0, rows*feats]");
    if (index_bytes != index_bytes_for(rows * feats))
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_uniform: index_bytes must be %d", index_bytes_for(rows * feats));
    if (k > 0 && (!idx || !values)) return stacr_fail(STACR_ERR_INVALID, "stacr_select_uniform: NULL output");
    return stacr_uniform_launch(x, coeff, q, dtype, rows, feats, rank, k, idx, index_bytes, values,
                                static_cast<hipStream_t>(stream));
}

int stacr_block_sparse_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows, int64_t block_size,
                            int64_t *count_full, int64_t *count_last, int64_t *entries, size_t *workspace_bytes)
{
    if (rows < 1 || feats < 1 || chunk_rows < 1 || block_size < 1 || feats % block_size)
        return stacr_fail(STACR_ERR_INVALID, "stacr_block_sparse_plan: needs rows, chunk_rows >= 1 and feats %% block_size == 0");
    if (!(budget > 0.0 && budget <= 1.0)) return stacr_fail(STACR_ERR_INVALID, "budget %g outside (0, 1]", budget);
    if (!count_full || !count_last || !entries || !workspace_bytes)
        return stacr_fail(STACR_ERR_INVALID, "stacr_block_sparse_plan: NULL output");
    const int64_t cr = chunk_rows < rows ? chunk_rows : rows;
    const int64_t n_seg = (rows + cr - 1) / cr;
    const int64_t last_rows = rows - (n_seg - 1) * cr;
    auto count_of = [&](int64_t seg_rows) {  // max(1, round(budget * blocks)) (stacr/layers.py:83)
        const int64_t blocks = seg_rows * feats / block_size;
        const int64_t c = py_round(budget * (double)blocks);
        return c < 1 ? (int64_t)1 : c;
    };
    *count_full = count_of(cr);
    *count_last = count_of(last_rows);
    *entries = ((n_seg - 1) * *count_full + *count_last) * block_size;
    *workspace_bytes = stacr_block_ws(rows, feats, block_size, n_seg, *count_full > *count_last ? *count_full : *count_last);
    return STACR_OK;
}

int stacr_select_block_sparse(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                              int rank, double budget, int64_t chunk_rows, int64_t block_size, void *idx,
                              int index_bytes, void *values, void *workspace, size_t workspace_bytes, void *stream)
{
    int rc = check_factors(x, coeff, q, dtype, rows, feats, rank, "stacr_select_block_sparse");
    if (rc) return rc;
    int64_t cf, cl, n_out;
    size_t need;
    rc = stacr_block_sparse_plan(rows, feats, budget, chunk_rows, block_size, &cf, &cl, &n_out, &need);
    if (rc) return rc;
    if (index_bytes != index_bytes_for(rows * feats))
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_block_sparse: index_bytes must be %d",
                          index_bytes_for(rows * feats));
    if (!idx || !values || !workspace) return stacr_fail(STACR_ERR_INVALID, "stacr_select_block_sparse: NULL pointer");
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_select_block_sparse: workspace has %zu bytes, needs %zu",
                          workspace_bytes, need);
    const int64_t cr = chunk_rows < rows ? chunk_rows : rows;
    return stacr_block_launch(x, coeff, q, dtype, rows, feats, rank, block_size, cr, cf, cl, idx, index_bytes, values,
                              workspace, static_cast<hipStream_t>(stream));
}

namespace {

// Counts of the adaptive block_sparse selector (stacr/adaptive.py:1788-1832): k = floor(total * b)
// entries, k_blocks = max(1, ceil(k / bs)), per chunk max(1, ceil(k_blocks * chunk / rows)) blocks
// (at most the chunk's own), the union cut to k_blocks.
struct AdaptiveBlockPlan {
    int64_t k_blocks = 0, chunk_rows = 0, count_full = 0, count_last = 0, n_cand = 0, n_final = 0;
    int index_bytes = 4;
};

int plan_adaptive_blocks(int64_t rows, int64_t feats, double budget, int64_t chunk_rows, int64_t bs,
                         AdaptiveBlockPlan *p)
{
    if (rows < 1 || feats < 1 || chunk_rows < 1 || bs < 1)
        return stacr_fail(STACR_ERR_INVALID, "adaptive block_sparse: needs rows, feats, chunk_rows, block_size >= 1");
    if (!(budget >= 0.0 && budget <= 1.0)) return stacr_fail(STACR_ERR_INVALID, "budget %g outside [0, 1]", budget);
    const int64_t total = rows * feats;
    p->index_bytes = total < 32768 ? 2 : (total <= (1ll << 31) ? 4 : 8);
    int64_t k = (int64_t)((double)total * budget);
    if (k > total) k = total;
    if (k <= 0) return STACR_OK;
    const int64_t bpr = (feats + bs - 1) / bs;
    p->k_blocks = (k + bs - 1) / bs;
    p->chunk_rows = chunk_rows < rows ? chunk_rows : rows;
    const int64_t n_seg = (rows + p->chunk_rows - 1) / p->chunk_rows;
    const int64_t last_rows = rows - (n_seg - 1) * p->chunk_rows;
    int64_t per = (p->k_blocks * p->chunk_rows + rows - 1) / rows;
    if (per < 1) per = 1;
    p->count_full = per < p->chunk_rows * bpr ? per : p->chunk_rows * bpr;
    p->count_last = per < last_rows * bpr ? per : last_rows * bpr;
    p->n_cand = (n_seg - 1) * p->count_full + p->count_last;
    p->n_final = p->n_cand < p->k_blocks ? p->n_cand : p->k_blocks;
    return STACR_OK;
}

}  // namespace

int stacr_adaptive_block_sparse_plan(int64_t rows, int64_t feats, double budget, int64_t chunk_rows,
                                     int64_t block_size, int64_t *k_blocks, int64_t *max_entries, int *index_bytes,
                                     size_t *workspace_bytes)
{
    AdaptiveBlockPlan p;
    const int rc = plan_adaptive_blocks(rows, feats, budget, chunk_rows, block_size, &p);
    if (rc) return rc;
    if (k_blocks) *k_blocks = p.k_blocks;
    if (max_entries) *max_entries = p.n_final * block_size;
    if (index_bytes) *index_bytes = p.index_bytes;
    if (workspace_bytes)
        *workspace_bytes = p.k_blocks ? stacr_adaptive_block_ws(rows, feats, block_size, p.n_cand, p.k_blocks) : 0;
    return STACR_OK;
}

int stacr_adaptive_select_block_sparse(const void *x, const void *coeff, const void *q, int dtype, int64_t rows,
                                       int64_t feats, int rank, double budget, int64_t chunk_rows, int64_t block_size,
                                       void *idx, int index_bytes, void *values, int64_t *count, void *workspace,
                                       size_t workspace_bytes, void *stream)
{
    int rc = check_factors(x, coeff, q, dtype, rows, feats, rank, "stacr_adaptive_select_block_sparse");
    if (rc) return rc;
    AdaptiveBlockPlan p;
    rc = plan_adaptive_blocks(rows, feats, budget, chunk_rows, block_size, &p);
    if (rc) return rc;
    if (index_bytes != p.index_bytes)
        return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_select_block_sparse: index_bytes must be %d", p.index_bytes);
    if (!count) return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_select_block_sparse: NULL count");
    if (!p.k_blocks) return stacr_fill_int_launch(count, 8, 1, 0, static_cast<hipStream_t>(stream));
    if (!idx || !values || !workspace)
        return stacr_fail(STACR_ERR_INVALID, "stacr_adaptive_select_block_sparse: NULL pointer argument");
    const size_t need = stacr_adaptive_block_ws(rows, feats, block_size, p.n_cand, p.k_blocks);
    if (workspace_bytes < need)
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_adaptive_select_block_sparse: workspace has %zu bytes, needs %zu",
                          workspace_bytes, need);
    return stacr_adaptive_block_launch(x, coeff, q, dtype, rows, feats, rank, block_size, p.chunk_rows, p.count_full,
                                       p.count_last, p.k_blocks, idx, index_bytes, values, count, workspace,
                                       static_cast<hipStream_t>(stream));
}

int stacr_sample_magnitudes(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                            int rank, const int64_t *positions, int64_t n, void *out, void *stream)
{
    int rc = check_factors(x, coeff, q, dtype, rows, feats, rank, "stacr_sample_magnitudes");
    if (rc) return rc;
    if (n < 0 || (n > 0 && (!positions || !out))) return stacr_fail(STACR_ERR_INVALID, "stacr_sample_magnitudes: bad sample");
    return stacr_sample_launch(x, coeff, q, dtype, rows, feats, rank, positions, n, out, static_cast<hipStream_t>(stream));
}

int stacr_threshold_workspace_bytes(int64_t rows, int64_t feats, size_t *bytes)
{
    if (!bytes || rows < 0 || feats < 1) return stacr_fail(STACR_ERR_INVALID, "stacr_threshold_workspace_bytes: bad argument");
    *bytes = stacr_threshold_ws(rows, feats);
    return STACR_OK;
}

int stacr_select_threshold(const void *x, const void *coeff, const void *q, int dtype, int64_t rows, int64_t feats,
                           int rank, const float *threshold, int64_t cap, void *idx, int index_bytes, void *values,
                           int64_t *count, void *workspace, size_t workspace_bytes, void *stream)
{
    int rc = check_factors(x, coeff, q, dtype, rows, feats, rank, "stacr_select_threshold");
    if (rc) return rc;
    if (cap < 0 || cap > rows * feats) return stacr_fail(STACR_ERR_INVALID, "stacr_select_threshold: cap outside [0, rows*feats]");
    if (index_bytes != index_bytes_for(rows * feats))
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_threshold: index_bytes must be %d", index_bytes_for(rows * feats));
    if (!threshold || !count || !workspace || (cap > 0 && (!idx || !values)))
        return stacr_fail(STACR_ERR_INVALID, "stacr_select_threshold: NULL pointer argument");
    if (workspace_bytes < stacr_threshold_ws(rows, feats))
        return stacr_fail(STACR_ERR_WORKSPACE, "stacr_select_threshold: workspace too small");
    return stacr_threshold_launch(x, coeff, q, dtype, rows, feats, rank, threshold, cap, idx, index_bytes, values,
                                  count, workspace, static_cast<hipStream_t>(stream));
}
