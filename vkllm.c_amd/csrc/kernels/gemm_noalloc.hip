// The prompt-step GEMM for callers that cannot allocate device memory (code under stream capture, serving loops
// that forbid hipMalloc): vkllm_hip_gemm with its split-K workspace taken from a fixed array of the library instead
// of a caller buffer.
//
// `scratch` is a file-scope device array of kNoAllocWorkElems floats (32 MiB). Every GPU the library runs on holds
// its own copy until the process ends. Host code never names the array in a kernel argument or copy (on the host
// the name is not a device address): vkllm_context_new calls noalloc_scratch_init with the context's device
// current, which looks the array's address up with hipGetSymbolAddress once per device, and the entry point passes
// that address to the kernels. The split-K partial tiles are written whole before the reduce reads them, so the
// array needs no clearing between calls; calls that overlap on one GPU (two contexts' streams at once) race on it.
// Contexts may be created from several threads at once: the per-device address is looked up under a lock and
// published with release/acquire atomics.
#include <atomic>
#include <mutex>

#include "runtime.h"

namespace
{
constexpr size_t kNoAllocWorkElems = (size_t)8 << 20;
__device__ __align__(256) float scratch[kNoAllocWorkElems];
std::atomic<float *> g_scratch[VKLLM_MAX_PHY_DEVS]; // scratch's device address per device (noalloc_scratch_init)
std::mutex g_scratch_lock;
} // namespace

namespace vk
{
hipError_t noalloc_scratch_init(int dev)
{
    if (dev < 0 || dev >= VKLLM_MAX_PHY_DEVS)
        return hipErrorInvalidDevice;
    if (g_scratch[dev].load(std::memory_order_acquire))
        return hipSuccess;
    std::lock_guard<std::mutex> hold(g_scratch_lock);
    if (g_scratch[dev].load(std::memory_order_relaxed))
        return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return e;
    g_scratch[dev].store((float *)p, std::memory_order_release);
    return hipSuccess;
}
} // namespace vk

extern "C" vkllm_err_t vkllm_hip_gemm_noalloc(struct vkllm_context *ctx, int epi, const uint16_t *A,
                                              const uint16_t *B, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                                              uint32_t ldc, uint32_t split, uint64_t work_elems)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && A && B && C && M > 0 && N > 0 && K >= 8 && K % 8 == 0);
    _CHECK_ARGS(epi == vk::GEMM_PLAIN || epi == vk::GEMM_SILU_HI || epi == vk::GEMM_RESID || epi == vk::GEMM_SWIGLU);
    _CHECK_ARGS(epi == vk::GEMM_SWIGLU ? (K % 64 == 0 && N % 64 == 0 && split * 2 == N && ldc >= split && ldc % 8 == 0)
                                       : ldc >= N);
    _CHECK_ARGS(((uintptr_t)A | (uintptr_t)B) % 16 == 0);
    _CHECK_ARGS(epi != vk::GEMM_SWIGLU || (uintptr_t)C % 16 == 0);
    if (work_elems > kNoAllocWorkElems)
    {
        log_error("vkllm_hip_gemm_noalloc: work_elems %llu exceeds the library's scratch of %llu floats",
                  (unsigned long long)work_elems, (unsigned long long)kNoAllocWorkElems);
        return VKLLM_ERR_ARGS;
    }
    const int dev = ctx->device->device_id;
    float *const work = dev >= 0 && dev < VKLLM_MAX_PHY_DEVS ? g_scratch[dev].load(std::memory_order_acquire) : nullptr;
    if (!work)
    {
        log_error("vkllm_hip_gemm_noalloc: no scratch address for device %d", dev);
        return VKLLM_ERR_VULKAN;
    }
    const hipError_t e = vk::launch_gemm(ctx->device->stream, epi, A, B, C, M, N, K, ldc, split,
                                         ctx->device->cu_count, work, (size_t)work_elems);
    if (e != hipSuccess)
        return hip_fail(e, "vkllm_hip_gemm_noalloc", __FILE__, __LINE__);
    return VKLLM_ERR_OK;
}
