// tbq_noalloc.hip -- tbq_moe_forward_noalloc: the MoE layer with its
// workspace in a file-scope device array instead of caller or library
// memory, for callers that cannot allocate (code under HIP graph capture,
// serving loops that forbid hipMalloc).  Nothing here allocates: no
// hipMalloc/hipFree and no allocating library call on any path.
//
// `scratch` is one array per GPU, held until the process ends.  In host code
// its name is only a host-side stand-in; the device address comes from
// hipGetSymbolAddress, looked up once per device (with that device current)
// on the entry point's first call there, and that pointer is what the
// kernels get.  The workspace layout is tbq_moe_forward's: its first 256 KiB
// are the router's per-token arrival counters, which must be zero before a
// call and which every call leaves at zero; the set-up clears them once with
// a fill kernel on the caller's stream (stream-ordered before the call's own
// kernels, and capturable, unlike a memset node).  Every call on a GPU
// shares that GPU's array: calls that overlap on one GPU (other streams,
// other threads) race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>

#include "../../include/tbq.h"

namespace {

constexpr size_t SCRATCH_BYTES = (size_t)TBQ_NOALLOC_SCRATCH_BYTES;
constexpr size_t COUNTER_BYTES = 256 * 1024;   // tbq_moe_forward's counter area
constexpr int MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

std::mutex g_mu;
void *g_ptr[MAX_DEVICES] = {};

__global__ __launch_bounds__(256) void k_zero_u32(unsigned *__restrict__ p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// The device address of this GPU's `scratch`, set up on first use.  NULL on
// failure (the HIP error is in *err).
void *device_scratch(hipStream_t st, hipError_t *err) {
    int dev = 0;
    if ((*err = hipGetDevice(&dev)) != hipSuccess) return nullptr;
    if (dev < 0 || dev >= MAX_DEVICES) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[dev]) return g_ptr[dev];
    void *p = nullptr;
    if ((*err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess || !p) return nullptr;
    const int n = (int)(COUNTER_BYTES / 4);
    hipLaunchKernelGGL(k_zero_u32, dim3(n / 256), dim3(256), 0, st, (unsigned *)p, n);
    if ((*err = hipGetLastError()) != hipSuccess) return nullptr;
    g_ptr[dev] = p;
    return p;
}

}  // namespace

extern "C" int tbq_host_fail(const char *msg);

extern "C" int tbq_moe_forward_noalloc(const tbq_moe_layer *L, int T, const float *xn, const float *resid,
                                       float *out, int *sel_idx, float *sel_w, int mode, void *stream) {
    if (!L || T <= 0) return tbq_host_fail("tbq_moe_forward_noalloc: null layer or T <= 0");
    const size_t need = tbq_moe_workspace_size(L, T, mode);
    if (need > SCRATCH_BYTES) {
        char msg[200];
        snprintf(msg, sizeof msg,
                 "tbq_moe_forward_noalloc: T=%d in mode %d needs a %zu-byte workspace, above the static %zu bytes",
                 T, mode, need, SCRATCH_BYTES);
        return tbq_host_fail(msg);
    }
    if (!tbq_init()) return 0;
    hipError_t err = hipSuccess;
    void *ws = device_scratch(reinterpret_cast<hipStream_t>(stream), &err);
    if (!ws) {
        char msg[200];
        snprintf(msg, sizeof msg, "tbq_moe_forward_noalloc: scratch set-up: %s", hipGetErrorString(err));
        return tbq_host_fail(msg);
    }
    return tbq_moe_forward(L, T, xn, resid, out, sel_idx, sel_w, ws, SCRATCH_BYTES, mode, stream);
}
