// stacr_weight_grad_noalloc: stacr_weight_grad for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
// backward's plan workspace (entry counts, matrix-core operands, light-entry records and block
// headers; or, for the general kernels, bucketed entries, pieces and round headers) lives in a
// file-scope device array instead of a caller buffer.  Each GPU the library runs on holds its own
// copy of the array until the process ends; the address of a device's copy is looked up once, on
// the entry point's first call with that device current, and every later call on the device
// reuses it.  Calls that overlap on one GPU share that scratch and race; nothing in it needs to
// start at zero (the count and plan kernels write every word the weight-gradient kernel uses).
#include <mutex>

#include "internal.h"

namespace {

__device__ __align__(256) unsigned char scratch[STACR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch copy (looked up once per device).
int scratch_for_current_device(void **out)
{
    int dev = 0;
    int rc = stacr_hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices)
        return stacr_fail(STACR_ERR_UNSUPPORTED, "stacr_weight_grad_noalloc: device %d outside 0..%d", dev,
                          kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        rc = stacr_hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (rc) return rc;
        if (!ptr) return stacr_fail(STACR_ERR_HIP, "stacr_weight_grad_noalloc: scratch address is NULL");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return STACR_OK;
}

}  // namespace

extern "C" int stacr_weight_grad_noalloc(const void *g, int dtype, int64_t rows, int64_t d_out, const void *coeff,
                                         const void *q, int64_t d_in, int rank, const void *idx, int index_bytes,
                                         const void *data, const float *scale, int bits, int val_dtype, int64_t nnz,
                                         int transposed, void *dw, int dw_dtype, void *dbias, int dbias_dtype,
                                         void *stream)
{
    size_t need = 0;
    int rc = stacr_weight_grad_workspace_bytes(rows, d_out, d_in, rank, nnz, &need);
    if (rc) return rc;
    if (need > (size_t)STACR_NOALLOC_SCRATCH_BYTES)
        return stacr_fail(STACR_ERR_UNSUPPORTED,
                          "stacr_weight_grad_noalloc: this problem needs %zu workspace bytes, above the %zu-byte "
                          "static scratch; call stacr_weight_grad with a caller workspace",
                          need, (size_t)STACR_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    rc = scratch_for_current_device(&ws);
    if (rc) return rc;
    return stacr_weight_grad(g, dtype, rows, d_out, coeff, q, d_in, rank, idx, index_bytes, data, scale, bits,
                             val_dtype, nnz, transposed, dw, dw_dtype, dbias, dbias_dtype, ws,
                             (size_t)STACR_NOALLOC_SCRATCH_BYTES, stream);
}
