// exl3_noalloc.hip -- the allocation-free form of exl3_gemv_mr.
//
// exl3_gemv_mr_noalloc runs the same fused GEMV kernels as exl3_gemv_mr, with their workspace
// (completion counters + split-K partial sums) in `scratch`, a file-scope device array of
// EXL3_NOALLOC_SCRATCH_BYTES that every GPU holds for the life of the process.  It is for callers
// that cannot allocate device memory: code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc.  The entry point calls no hipMalloc / hipFree and no
// allocating library routine.
//
// Host code never passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in, not a device address): the first call on a device, with that device current, looks
// up the device's own copy with hipGetSymbolAddress and keeps the pointer per device.
//
// Sharing: every call on one GPU uses that GPU's one array.  The counters (the first
// EXL3_GEMV_COUNTER_BYTES) must be zero when a call starts: the array is cleared once per device
// at set-up, and every call leaves them zero again.  Calls that overlap on one GPU (concurrent
// streams, or two graphs replayed at once) race on the array and must be serialized by the caller.
#include "../../include/exl3_mi355x.h"

#include <hip/hip_runtime.h>

#include <mutex>

static __device__ __align__(256) unsigned char scratch[EXL3_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
void* g_scratch[MAX_DEVICES];
std::mutex g_mu;

// zero `words` 32-bit words (the completion counters), grid-stride
__global__ void __launch_bounds__(256) clear_words_kernel(uint32_t* __restrict__ p, int words)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < words; i += gridDim.x * 256) p[i] = 0u;
}

// The current device's copy of `scratch` (set up on first use: symbol lookup, counters cleared on
// `stream`).  nullptr on failure.
void* scratch_of_current_device(hipStream_t stream)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev]) return g_scratch[dev];
    void* ptr = nullptr;
    // The first call may come while `stream` captures a graph in the global mode, which refuses
    // runtime calls outside the capture: this thread relaxes it for the lookup (no stream work),
    // then restores it.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return nullptr;
    const hipError_t found = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess || found != hipSuccess || !ptr) return nullptr;
    // a fill kernel rather than hipMemsetAsync: the first call may be under graph capture
    constexpr int words = EXL3_GEMV_COUNTER_BYTES / 4;
    hipLaunchKernelGGL(clear_words_kernel, dim3(words / 256 / 16), dim3(256), 0, stream, (uint32_t*) ptr, words);
    if (hipGetLastError() != hipSuccess) return nullptr;
    g_scratch[dev] = ptr;
    return ptr;
}

}  // namespace

extern "C" {

int exl3_gemv_mr_noalloc(const void* x, int64_t ldx, const void* trellis, void* y, int64_t ldy, const void* suh,
                         const void* svh, int m, int k, int n, int K, int mcg, int mul1, void* stream)
{
    if (!x || !trellis || !y || !suh || !svh) return EXL3_EINVAL;
    const size_t need = exl3_gemv_workspace_size(m, k, n, K, 1);
    if (need == 0)   // not a GEMV shape: exl3_gemv_mr's own status (declined or invalid), nothing launched
        return exl3_gemv_mr(x, ldx, trellis, y, ldy, suh, nullptr, svh, m, k, n, K, mcg, mul1, nullptr, 0, stream);
    if (need > (size_t) EXL3_NOALLOC_SCRATCH_BYTES) return EXL3_EWORKSPACE;
    void* ws = scratch_of_current_device((hipStream_t) stream);
    if (!ws) return EXL3_ELAUNCH;
    // A_had = NULL: every workgroup rotates its own input slices (the same output, bitwise)
    return exl3_gemv_mr(x, ldx, trellis, y, ldy, suh, nullptr, svh, m, k, n, K, mcg, mul1, ws,
                        (size_t) EXL3_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
