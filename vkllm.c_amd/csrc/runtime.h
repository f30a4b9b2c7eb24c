// Internal runtime of libvkllm: the HIP device behind a vkllm_context, the device-memory pool, tensor views for
// kernels, the kernel registry and timing, and the entry points shared between the C API files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "vkllm/vkllm_commands.h"
#include "vkllm/vkllm_common.h"
#include "vkllm/vkllm_context.h"
#include "vkllm/vkllm_dtypes.h"
#include "vkllm/vkllm_errors.h"
#include "vkllm/vkllm_graph.h"
#include "vkllm/vkllm_hip.h"
#include "vkllm/vkllm_ops.h"
#include "vkllm/vkllm_pipeline.h"
#include "vkllm/vkllm_tensor.h"
#include "kernels/kernels.h"

// Kernel families (registry slots). One vkllm_pipeline per slot.
enum KernelId
{
    KID_COPY = 0,
    KID_BIN,
    KID_EMBEDDING,
    KID_RMSNORM,
    KID_GEMV,
    KID_GEMM,
    KID_ROPE,
    KID_SOFTMAX,
    KID_FFN,
    KID_UPDATE_ROWS,
    KID_ARG_MAX,
    // fused token-step kernels
    KID_F_EMBED,
    KID_F_QKV,
    KID_F_ATTN_SCORES,
    KID_F_ATTN_PV,
    KID_F_O_RESID,
    KID_F_GATEUP,
    KID_F_DOWN_RESID,
    KID_F_LOGITS,
    KID_F_ARGMAX,
    KID_F_RMSNORM,
    KID_F_GEMM,
    KID_F_ROPE_KV,
    KID_F_ATTN_PREFILL,
    KID_F_SWIGLU,
    KID_F_ATTN_SMALL,
    KID_F_ATTN_O,
    KID_F_ATTN_LONG,
    KID_COUNT
};

struct vkllm_pipeline_table
{
    vkllm_pipeline entries[KID_COUNT];
};

struct vkllm_gpu_device
{
    int device_id = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t props{};
    int cu_count = 0;
    // size-class pool for tensor memory; blocks go back to the free list of their class on free
    std::unordered_map<size_t, std::vector<void *>> free_blocks;
    std::vector<void *> all_blocks;
    size_t pooled_bytes = 0;
    // pinned host blocks (mirrors of mapped tensors), same size classes
    std::unordered_map<size_t, std::vector<void *>> pinned_free;
    std::vector<void *> pinned_all;
    // recycled tensor structs (a token step builds and frees one per graph node)
    std::vector<void *> node_free;
    int scope_depth = 0; // entry points of this device's context on the call stack (DeviceScope)
    int exec_mode = VKLLM_EXEC_FUSED;
    int graph_replay = 1;
    int timing = 0;
    // timing mode: one event pair per launch, resolved into the pipelines' counters at synchronisation points
    struct TimingRec
    {
        vkllm_pipeline *pipeline;
        hipEvent_t begin, end;
        vkllm_pipeline *node; // optional: a graph node's record, whose last_ns also receives the launch's duration
    };
    // the node record the next timed launch adds its duration to (set by the fused executor, taken by timing_end)
    vkllm_pipeline *timing_node = nullptr;
    std::vector<TimingRec> timing_pending;
    std::vector<hipEvent_t> event_pool;
    // split-K partial tiles of the MATMUL op's matrix-core path, allocated at its first use (op_gemm_workspace)
    float *op_work = nullptr;
    size_t op_work_elems = 0;
};

// ---- errors ----
vkllm_err_t hip_fail(hipError_t e, const char *what, const char *file, int line);
#define HIP_TRY(_expr)                                                                                              \
    do                                                                                                              \
    {                                                                                                               \
        hipError_t _he = (_expr);                                                                                   \
        if (_he != hipSuccess)                                                                                      \
            return hip_fail(_he, #_expr, __FILE__, __LINE__);                                                       \
    } while (0)

// Makes the context's device current for one entry point and gives the caller's back on return. Allocations,
// function attributes and occupancy queries act on the current device, and one thread may hold contexts on several
// devices. Only the outermost entry point of a call checks (one hipGetDevice when the device is already current):
// the library's own calls into its entry points (a graph build creates hundreds of tensors) run on the same context,
// whose nesting depth the device record keeps (a context is used by one thread at a time).
struct DeviceScope
{
    vkllm_gpu_device *dev = nullptr; // the device record whose depth this scope counts
    int prev = -1;                   // the caller's device, when this scope switched away from it
    explicit DeviceScope(const vkllm_context *ctx)
    {
        if (!ctx || !ctx->device)
            return;
        dev = ctx->device;
        if (dev->scope_depth++ > 0)
            return;
        int cur = 0;
        if (hipGetDevice(&cur) == hipSuccess && cur != dev->device_id && hipSetDevice(dev->device_id) == hipSuccess)
            prev = cur;
    }
    // before an entry point frees the device record: stop counting on it (the caller's device still comes back)
    void release()
    {
        dev = nullptr;
    }
    ~DeviceScope()
    {
        if (dev)
            --dev->scope_depth;
        if (prev >= 0)
            (void)hipSetDevice(prev);
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;
};

// ---- memory ----
size_t pool_class(size_t bytes);
void *pool_alloc(vkllm_gpu_device *dev, size_t bytes);
void pool_free(vkllm_gpu_device *dev, void *p, size_t bytes);
void pool_release_all(vkllm_gpu_device *dev);
void *pinned_alloc(vkllm_gpu_device *dev, size_t bytes);
void pinned_free(vkllm_gpu_device *dev, void *p, size_t bytes);
void node_pool_release(vkllm_gpu_device *dev);

// Device address of a tensor's element [0,0,0,0]; follows views to their base and allocates the base's memory
// on first use. nullptr on allocation failure.
void *tensor_dev(vkllm_context *ctx, vkllm_tensor *t);
// The tensor owning the memory a view aliases.
vkllm_tensor *tensor_base(vkllm_tensor *t);
uint32_t dtype_bytes(vkllm_dtype_t dt);
vk::TView tview(vkllm_context *ctx, vkllm_tensor *t);

// ---- kernel registry and timing ----
vkllm_pipeline *pipeline_of(vkllm_context *ctx, KernelId id);
// Records the timing events around the launches made by `fn` when timing is enabled.
template <typename F> hipError_t timed(vkllm_context *ctx, vkllm_pipeline *p, F &&fn);
void timing_begin(vkllm_context *ctx, vkllm_pipeline *p);
void timing_end(vkllm_context *ctx, vkllm_pipeline *p);
// Waits for the recorded launches and adds their durations to their pipelines' last_ns/total_ns/launches.
hipError_t timing_flush(vkllm_context *ctx);

template <typename F> hipError_t timed(vkllm_context *ctx, vkllm_pipeline *p, F &&fn)
{
    timing_begin(ctx, p);
    hipError_t e = fn();
    timing_end(ctx, p);
    return e;
}

// ---- commands ----
// After a kernel wrote `t` on `cmds`' stream: mark it valid and queue a host-mirror refresh for mapped tensors.
void commands_note_write(vkllm_commands *cmds, vkllm_tensor *t);

// ---- graph execution (node-by-node) ----
vkllm_err_t op_init(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t);
vkllm_err_t op_run(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t);
vkllm_err_t op_post_run(vkllm_context *ctx, vkllm_commands *cmds, vkllm_tensor *t);

// ---- fused token-step plans (fused.cpp) ----
struct vkllm_models_llama2;
void *fused_plan_new(vkllm_models_llama2 *model, vkllm_tensor *input_toks, uint32_t offset);
void fused_plan_free(void *plan);
vkllm_err_t fused_plan_init(vkllm_context *ctx, vkllm_graph *graph);
vkllm_err_t fused_plan_run(vkllm_context *ctx, vkllm_graph *graph);
// true once the plan ran as fused kernels (which read none of the graph's node tensors)
bool fused_plan_ran(const void *plan);
// drops a single-token step launched ahead for the plan's model (before node-by-node execution of its graph)
vkllm_err_t fused_plan_discard_ahead(vkllm_context *ctx, vkllm_graph *graph);
void fused_model_release(vkllm_context *ctx, vkllm_models_llama2 *model);
