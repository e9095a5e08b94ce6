/* le_gemm_noalloc: the small-M GEMM for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * le_gemm needs a workspace (the activations as fp16 planes and per-super-block sum records). Here
 * that workspace is a file-scope device array, `scratch`, of LE_GEMM_SCRATCH_BYTES. Every GPU the
 * library runs on holds its own copy of it until the process ends. Its device address is looked up
 * once per device with hipGetSymbolAddress when a context is created on that device (le_init calls
 * le_scratch_attach), and that address, never the array's host-side name, is what the kernels
 * receive.
 *
 * Sharing: every call on one GPU uses that GPU's array and leaves the last call's contents in it.
 * The GEMM pre-pass writes every workspace byte the main pass reads, and the main pass every
 * K-slice partial result the summing pass reads, so nothing has to start at zero. The whole array
 * is offered as workspace, so shapes whose K slices' partial results fit in it are summed
 * reproducibly, as le_gemm does with le_gemm_workspace_size_rows bytes. Calls that overlap on one GPU (two streams, two host threads) race on the array; callers
 * serialize them.
 *
 * This file is compiled by hipcc (it declares device memory) and linked into lible_qmm.so.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/le_qmm.h"

static __device__ __align__(256) unsigned char scratch[LE_GEMM_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices]; /* device address of `scratch` on each device, or null */
}  // namespace

/* Looks up the address of `scratch` on `device` (which must be current) once. Returns LE_OK or
 * LE_ERR_HIP. Called by le_init. */
int le_scratch_attach(int device) {
    if (device < 0 || device >= kMaxDevices) return LE_ERR_ARG;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return LE_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return LE_ERR_HIP;
    }
    g_ptr[device] = p;
    return LE_OK;
}

/* Host-side helpers of le_qmm.cpp (the context lives there). */
int le_ctx_device(const le_ctx *ctx);
int le_ctx_fail(le_ctx *ctx, int code, const char *msg);

extern "C" int le_gemm_noalloc(le_ctx *ctx, int ty, const void *w, const float *x, int m, float *y, int rows,
                               int cols, le_stream_t stream) {
    if (!ctx) return LE_ERR_ARG;
    const size_t need = le_gemm_workspace_size(ty, m, cols);
    if (need > (size_t)LE_GEMM_SCRATCH_BYTES) {
        char buf[160];
        snprintf(buf, sizeof buf, "le_gemm_noalloc: m=%d x cols=%d needs %zu workspace bytes, above the %zu-byte scratch", m,
                 cols, need, (size_t)LE_GEMM_SCRATCH_BYTES);
        return le_ctx_fail(ctx, LE_ERR_WORKSPACE, buf);
    }
    const int dev = le_ctx_device(ctx);
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (dev >= 0 && dev < kMaxDevices) p = g_ptr[dev];
    }
    if (!p) return le_ctx_fail(ctx, LE_ERR_HIP, "le_gemm_noalloc: scratch address unknown on this device");
    return le_gemm(ctx, ty, w, x, m, y, rows, cols, need ? p : nullptr, need ? (size_t)LE_GEMM_SCRATCH_BYTES : 0, stream);
}
