// Device figures that bench.py reports beside the roofline fractions, measured with kernels that do nothing else:
//   vkllm_hip_probe_stream_read: the HBM read rate of a plain streaming kernel (16-byte non-temporal loads, each byte
//     read once, nothing written), over windows of a buffer four times the GPU's 256 MB memory-side cache, so no
//     window is found in it. The decode GEMVs stream their weights the same way, with their arithmetic on top.
//   vkllm_hip_probe_launch_gap: the time per launch of a chain of empty kernels on the context's stream, each
//     depending on the one before (stream order), replayed from a captured graph as the decode step is: the cost of
//     one kernel boundary that a decode step pays between its products.
// Neither has a counterpart in the reference; they are measurement entry points, like vkllm_hip_time_ops.
#include <algorithm>
#include <vector>

#include "device_common.h"
#include "runtime.h"

namespace
{
constexpr int kProbeUnroll = 8;               // 16-byte loads in flight per thread
constexpr uint32_t kProbeBlocks = 1024;       // workgroups of 256 threads
constexpr uint64_t kProbeBuffer = 1ull << 30; // bytes: four times the memory-side cache

// workgroup b reads vectors [b per, (b + 1) per) (per a multiple of 256 kProbeUnroll); the XOR of everything read is
// stored only when it equals a constant, which keeps the loads from being removed
__global__ __launch_bounds__(256) void probe_read_kernel(const vk::u32x4 *p, uint64_t per, uint32_t *sink)
{
    const vk::u32x4 *b = p + blockIdx.x * per;
    uint32_t acc = 0;
    for (uint64_t i = threadIdx.x; i < per; i += 256 * kProbeUnroll)
    {
        vk::u32x4 v[kProbeUnroll];
#pragma unroll
        for (int k = 0; k < kProbeUnroll; ++k)
            v[k] = __builtin_nontemporal_load(b + i + 256 * k);
#pragma unroll
        for (int k = 0; k < kProbeUnroll; ++k)
            acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
    }
    if (acc == 0x9e3779b9u)
        sink[blockIdx.x] = acc;
}

__global__ void probe_empty_kernel(uint32_t *sink)
{
    if (threadIdx.x == 0xffffffffu)
        sink[0] = 1;
}

struct Probe
{
    void *buf = nullptr;
    uint32_t *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    ~Probe()
    {
        if (e0)
            (void)hipEventDestroy(e0);
        if (e1)
            (void)hipEventDestroy(e1);
        if (buf)
            (void)hipFree(buf);
        if (sink)
            (void)hipFree(sink);
    }
};

float elapsed_ms(hipEvent_t a, hipEvent_t b)
{
    float ms = 0.f;
    return hipEventElapsedTime(&ms, a, b) == hipSuccess ? ms : -1.f;
}
} // namespace

#define PROBE_TRY(x)                                                                                                  \
    do                                                                                                                \
    {                                                                                                                 \
        hipError_t e_ = (x);                                                                                          \
        if (e_ != hipSuccess)                                                                                         \
            return hip_fail(e_, #x, __FILE__, __LINE__);                                                              \
    } while (0)

extern "C" vkllm_err_t vkllm_hip_probe_stream_read(struct vkllm_context *ctx, uint64_t window_bytes, uint32_t reps,
                                                   double *gbps_median, double *gbps_best)
{
    DeviceScope device_scope(ctx);
    constexpr uint64_t quantum = (uint64_t)kProbeBlocks * 256 * kProbeUnroll * 16; // 32 MiB
    _CHECK_ARGS(ctx && gbps_median && gbps_best && reps > 0 && reps <= 1024);
    _CHECK_ARGS(window_bytes >= quantum && window_bytes % quantum == 0 && window_bytes <= kProbeBuffer);
    hipStream_t st = ctx->device->stream;
    Probe p;
    PROBE_TRY(hipMalloc(&p.buf, kProbeBuffer));
    PROBE_TRY(hipMalloc(&p.sink, kProbeBlocks * sizeof(uint32_t)));
    PROBE_TRY(hipMemsetAsync(p.buf, 0x5a, kProbeBuffer, st));
    PROBE_TRY(hipEventCreate(&p.e0));
    PROBE_TRY(hipEventCreate(&p.e1));
    const uint64_t windows = kProbeBuffer / window_bytes, per = window_bytes / 16 / kProbeBlocks;
    std::vector<float> ms;
    for (uint32_t r = 0; r <= reps; ++r) // the first pass is untimed
    {
        const vk::u32x4 *w = (const vk::u32x4 *)((const char *)p.buf + (r % windows) * window_bytes);
        PROBE_TRY(hipEventRecord(p.e0, st));
        probe_read_kernel<<<kProbeBlocks, 256, 0, st>>>(w, per, p.sink);
        PROBE_TRY(hipGetLastError());
        PROBE_TRY(hipEventRecord(p.e1, st));
        PROBE_TRY(hipEventSynchronize(p.e1));
        if (r > 0)
            ms.push_back(elapsed_ms(p.e0, p.e1));
    }
    std::sort(ms.begin(), ms.end());
    _CHECK_ARGS(ms.front() > 0.f);
    *gbps_median = (double)window_bytes / (ms[ms.size() / 2] * 1e-3) / 1e9;
    *gbps_best = (double)window_bytes / (ms.front() * 1e-3) / 1e9;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_probe_launch_gap(struct vkllm_context *ctx, uint32_t launches, uint32_t blocks,
                                                  double *us_per_launch)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx && us_per_launch && launches > 0 && launches <= 4096 && blocks > 0 && blocks <= 65536);
    hipStream_t st = ctx->device->stream;
    Probe p;
    PROBE_TRY(hipMalloc(&p.sink, sizeof(uint32_t)));
    PROBE_TRY(hipEventCreate(&p.e0));
    PROBE_TRY(hipEventCreate(&p.e1));
    // the chain is captured into a graph and replayed, as the decode step is, so the host's launch rate is not what
    // is timed
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    PROBE_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    for (uint32_t i = 0; i < launches; ++i)
        probe_empty_kernel<<<blocks, 256, 0, st>>>(p.sink);
    const hipError_t launched = hipGetLastError();
    const hipError_t ended = hipStreamEndCapture(st, &graph);
    hipError_t e = launched != hipSuccess ? launched : ended;
    if (e == hipSuccess)
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    float ms = -1.f;
    if (e == hipSuccess)
        e = hipGraphLaunch(exec, st); // untimed first replay
    if (e == hipSuccess)
        e = hipEventRecord(p.e0, st);
    if (e == hipSuccess)
        e = hipGraphLaunch(exec, st);
    if (e == hipSuccess)
        e = hipEventRecord(p.e1, st);
    if (e == hipSuccess)
        e = hipEventSynchronize(p.e1);
    if (e == hipSuccess)
        ms = elapsed_ms(p.e0, p.e1);
    if (exec)
        (void)hipGraphExecDestroy(exec);
    if (graph)
        (void)hipGraphDestroy(graph);
    PROBE_TRY(e);
    _CHECK_ARGS(ms > 0.f);
    *us_per_launch = (double)ms * 1e3 / launches;
    return VKLLM_ERR_OK;
}
