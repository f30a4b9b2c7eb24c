// Context, device, memory pool, kernel registry, timing, strings and logging.
// Replaces src/core/vkllm_context.c, src/core/vkllm_gpu_device.c (device selection), src/core/vkllm_pipeline.c
// (kernel table + per-pipeline timing), src/core/vkllm_errors.c, src/core/vkllm_dtypes.c, src/core/vkllm_ops.c.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "runtime.h"
#include "vkllm/vkllm_hashmap.h"
#include "vkllm/vkllm_models_llama2.h"

extern "C" void vkllm_log(int level, const char *file, int line, const char *fmt, ...)
{
    static int quiet = -1;
    if (quiet < 0)
    {
        const char *q = getenv("VKLLM_QUIET");
        quiet = q && *q && *q != '0';
    }
    if (level == VKLLM_LOG_INFO && quiet)
        return;
    const char *base = strrchr(file, '/');
    fprintf(stderr, "[vkllm] %s %s:%d: ", level == VKLLM_LOG_ERROR ? "ERROR" : "INFO", base ? base + 1 : file,
            line);
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
}

vkllm_err_t hip_fail(hipError_t e, const char *what, const char *file, int line)
{
    vkllm_log(VKLLM_LOG_ERROR, file, line, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
    return e == hipErrorOutOfMemory ? VKLLM_ERR_ALLOC : VKLLM_ERR_VULKAN;
}

// ------------------------------------------------------------------------------------------------------------
// strings: src/core/vkllm_errors.c, src/core/vkllm_dtypes.c, src/core/vkllm_ops.c

extern "C" const char *vkllm_err_s(vkllm_err_t err)
{
    switch (err)
    {
    case VKLLM_ERR_OK:
        return "VKLLM_ERR_OK";
    case VKLLM_ERR_ALLOC:
        return "VKLLM_ERR_ALLOC";
    case VKLLM_ERR_VULKAN:
        return "VKLLM_ERR_VULKAN";
    case VKLLM_ERR_DEV_NOT_FOUND:
        return "VKLLM_ERR_DEV_NOT_FOUND";
    case VKLLM_ERR_PIPELINE_NOT_FOUND:
        return "VKLLM_ERR_PIPELINE_NOT_FOUND";
    case VKLLM_ERR_ARGS:
        return "VKLLM_ERR_ARGS";
    default:
        return "VKLLM_ERR_UNKNOWN";
    }
}

extern "C" const char *vkllm_dtype_s(vkllm_dtype_t dtype)
{
    switch (dtype)
    {
    case vkllm_dtype_float32:
        return "float32";
    case vkllm_dtype_float16:
        return "float16";
    case vkllm_dtype_int8:
        return "int8";
    case vkllm_dtype_uint32:
        return "uint32";
    default:
        return "vkllm_dtype_start";
    }
}

extern "C" vkllm_err_t vkllm_get_dtype_info(vkllm_dtype_t dtype, struct vkllm_dtype_info *info)
{
    uint32_t b = dtype_bytes(dtype);
    if (!info || b == 0)
        return VKLLM_ERR_ARGS;
    info->dtype = dtype;
    info->bytes = b;
    info->items_per_block = 1;
    info->bytes_per_block = b;
    return VKLLM_ERR_OK;
}

extern "C" const char *vkllm_op_s(const vkllm_op_t op)
{
    static const char *names[] = {"VKLLM_OP_NONE",      "VKLLM_OP_COPY",    "VKLLM_OP_BIN",
                                  "VKLLM_OP_EMBEDDING", "VKLLM_OP_RMSNORM", "VKLLM_OP_MATMUL",
                                  "VKLLM_OP_ROPE",      "VKLLM_OP_SOFTMAX", "VKLLM_OP_FFN_UP_AND_GATE",
                                  "VKLLM_OP_UPDATE_ROWS", "VKLLM_OP_ARG_MAX", "VKLLM_OP_REF"};
    if ((int)op < 0 || (int)op >= (int)(sizeof(names) / sizeof(names[0])))
        return "VKLLM_OP_COUNTS";
    return names[op];
}

uint32_t dtype_bytes(vkllm_dtype_t dt)
{
    switch (dt)
    {
    case vkllm_dtype_float32:
    case vkllm_dtype_uint32:
        return 4;
    case vkllm_dtype_float16:
        return 2;
    case vkllm_dtype_int8:
        return 1;
    default:
        return 0;
    }
}

// ------------------------------------------------------------------------------------------------------------
// memory pool: blocks are kept per size class (1/8 power-of-two granularity, 256 B minimum) and reused

size_t pool_class(size_t bytes)
{
    if (bytes <= 256)
        return 256;
    size_t p = 1;
    while (p < bytes)
        p <<= 1;
    size_t step = p >= 2048 ? p / 8 : 256;
    return (bytes + step - 1) / step * step;
}

void *pool_alloc(vkllm_gpu_device *dev, size_t bytes)
{
    size_t c = pool_class(bytes);
    auto it = dev->free_blocks.find(c);
    if (it != dev->free_blocks.end() && !it->second.empty())
    {
        void *p = it->second.back();
        it->second.pop_back();
        return p;
    }
    void *p = nullptr;
    if (hipMalloc(&p, c) != hipSuccess)
    {
        (void)hipGetLastError();
        return nullptr;
    }
    dev->all_blocks.push_back(p);
    dev->pooled_bytes += c;
    return p;
}

void pool_free(vkllm_gpu_device *dev, void *p, size_t bytes)
{
    if (p)
        dev->free_blocks[pool_class(bytes)].push_back(p);
}

void *pinned_alloc(vkllm_gpu_device *dev, size_t bytes)
{
    size_t c = pool_class(bytes);
    auto it = dev->pinned_free.find(c);
    if (it != dev->pinned_free.end() && !it->second.empty())
    {
        void *p = it->second.back();
        it->second.pop_back();
        return p;
    }
    void *p = nullptr;
    if (hipHostMalloc(&p, c, hipHostMallocDefault) != hipSuccess)
    {
        (void)hipGetLastError();
        return nullptr;
    }
    dev->pinned_all.push_back(p);
    return p;
}

void pinned_free(vkllm_gpu_device *dev, void *p, size_t bytes)
{
    if (p)
        dev->pinned_free[pool_class(bytes)].push_back(p);
}

void pool_release_all(vkllm_gpu_device *dev)
{
    for (void *p : dev->all_blocks)
        (void)hipFree(p);
    dev->all_blocks.clear();
    dev->free_blocks.clear();
    dev->pooled_bytes = 0;
    for (void *p : dev->pinned_all)
        (void)hipHostFree(p);
    dev->pinned_all.clear();
    dev->pinned_free.clear();
}

// ------------------------------------------------------------------------------------------------------------
// kernel registry and timing (src/core/vkllm_pipeline.c:168-331)

static const char *kernel_names[KID_COUNT] = {
    "copy",          "bin",           "embedding",       "rmsnorm",       "gemv",          "gemm",
    "rope",          "softmax",       "ffn_up_and_gate", "update_rows",   "arg_max",       "fused_embed",
    "fused_qkv_rope", "fused_attn_scores", "fused_attn_pv", "fused_o_resid", "fused_gateup", "fused_down_resid",
    "fused_logits",  "fused_argmax",  "fused_rmsnorm",   "fused_gemm",    "fused_rope_kv", "fused_attn_prefill",
    "fused_swiglu",   "fused_attn_small", "fused_attn_o",    "fused_attn_long"};

vkllm_pipeline *pipeline_of(vkllm_context *ctx, KernelId id)
{
    return &ctx->pipelines->entries[id];
}

static hipEvent_t pooled_event(vkllm_gpu_device *dev)
{
    if (!dev->event_pool.empty())
    {
        hipEvent_t e = dev->event_pool.back();
        dev->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

void timing_begin(vkllm_context *ctx, vkllm_pipeline *p)
{
    vkllm_gpu_device *dev = ctx->device;
    if (!dev->timing)
        return;
    hipEvent_t b = pooled_event(dev);
    p->ev_begin = b;
    if (b)
        (void)hipEventRecord(b, dev->stream);
}

void timing_end(vkllm_context *ctx, vkllm_pipeline *p)
{
    vkllm_gpu_device *dev = ctx->device;
    vkllm_pipeline *node = dev->timing_node; // applies to this launch only
    dev->timing_node = nullptr;
    if (!dev->timing || !p->ev_begin)
        return;
    hipEvent_t e = pooled_event(dev);
    if (!e)
        return;
    (void)hipEventRecord(e, dev->stream);
    dev->timing_pending.push_back({p, (hipEvent_t)p->ev_begin, e, node});
    p->ev_begin = nullptr;
    p->pending = 1;
    // bound the number of events in flight; the flush waits for the oldest launches only
    if (dev->timing_pending.size() >= 4096)
        (void)timing_flush(ctx);
}

hipError_t timing_flush(vkllm_context *ctx)
{
    vkllm_gpu_device *dev = ctx->device;
    hipError_t rc = hipSuccess;
    for (auto &r : dev->timing_pending)
    {
        float ms = 0.f;
        hipError_t e = hipEventSynchronize(r.end);
        if (e == hipSuccess)
            e = hipEventElapsedTime(&ms, r.begin, r.end);
        if (e == hipSuccess)
        {
            const uint64_t ns = (uint64_t)((double)ms * 1e6);
            r.pipeline->last_ns = ns;
            r.pipeline->total_ns += ns;
            r.pipeline->launches += 1;
            if (r.node)
            {
                // a node's last_ns is the sum over the launches of the step that computed it
                r.node->last_ns += ns;
                r.node->total_ns += ns;
                r.node->launches += 1;
            }
        }
        else if (rc == hipSuccess)
            rc = e;
        r.pipeline->pending = 0;
        dev->event_pool.push_back(r.begin);
        dev->event_pool.push_back(r.end);
    }
    dev->timing_pending.clear();
    return rc;
}

extern "C" vkllm_err_t vkllm_pipeline_query_exec_time(struct vkllm_context *context, struct vkllm_pipeline *pipeline,
                                                      uint64_t *cost)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && pipeline && cost);
    _CHECK_ARGS(context->device->timing);
    HIP_TRY(timing_flush(context));
    *cost = pipeline->last_ns;
    return VKLLM_ERR_OK;
}

extern "C" int vkllm_hip_kernel_family_count(void)
{
    return KID_COUNT;
}

extern "C" vkllm_err_t vkllm_hip_kernel_stats(struct vkllm_context *context, int index, const char **name,
                                              uint64_t *launches, uint64_t *total_ns)
{
    _CHECK_ARGS(context && index >= 0 && index < KID_COUNT);
    HIP_TRY(timing_flush(context));
    const vkllm_pipeline &p = context->pipelines->entries[index];
    if (name)
        *name = p.name;
    if (launches)
        *launches = p.launches;
    if (total_ns)
        *total_ns = p.total_ns;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_reset_kernel_stats(struct vkllm_context *context)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context);
    HIP_TRY(timing_flush(context));
    for (int i = 0; i < KID_COUNT; ++i)
    {
        context->pipelines->entries[i].last_ns = 0;
        context->pipelines->entries[i].total_ns = 0;
        context->pipelines->entries[i].launches = 0;
    }
    return VKLLM_ERR_OK;
}

// ------------------------------------------------------------------------------------------------------------
// context (src/core/vkllm_context.c:8-35)

static int env_flag(const char *name, int dflt)
{
    const char *v = getenv(name);
    if (!v || !*v)
        return dflt;
    return *v != '0';
}

extern "C" vkllm_err_t vkllm_context_new(uint32_t dev, struct vkllm_context **context)
{
    _CHECK_ARGS(context);
    *context = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    {
        (void)hipGetLastError();
        log_error("no HIP device available");
        return VKLLM_ERR_DEV_NOT_FOUND;
    }
    if ((int)dev >= count)
    {
        log_error("device %u not found (%d visible)", dev, count);
        return VKLLM_ERR_DEV_NOT_FOUND;
    }
    // the device is current while the context is set up; the caller's comes back on return, as after every entry
    // point that takes the context
    struct RestoreDevice
    {
        int d = -1;
        ~RestoreDevice()
        {
            if (d >= 0)
                (void)hipSetDevice(d);
        }
    } restore;
    if (hipGetDevice(&restore.d) != hipSuccess)
        restore.d = -1;
    HIP_TRY(hipSetDevice((int)dev));
    // the allocation-free GEMM's scratch array: its address on this device, looked up once with the device current
    {
        const hipError_t e = vk::noalloc_scratch_init((int)dev);
        if (e != hipSuccess)
            return hip_fail(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
    }
    // host waits on the stream spin rather than sleep: a token step is milliseconds long and waking a sleeping
    // waiter adds tens of microseconds to every step (VKLLM_SPIN_WAIT=0 keeps HIP's default scheduling)
    if (env_flag("VKLLM_SPIN_WAIT", 1) && hipSetDeviceFlags(hipDeviceScheduleSpin) != hipSuccess)
        (void)hipGetLastError(); // flags are fixed once the device is in use; keep what it has
    auto *ctx = (vkllm_context *)calloc(1, sizeof(vkllm_context));
    if (!ctx)
        return VKLLM_ERR_ALLOC;
    ctx->appname = "vkllm";
    ctx->device = new vkllm_gpu_device();
    ctx->device->device_id = (int)dev;
    ctx->pipelines = (vkllm_pipeline_table *)calloc(1, sizeof(vkllm_pipeline_table));
    for (int i = 0; i < KID_COUNT; ++i)
    {
        ctx->pipelines->entries[i].name = kernel_names[i];
        ctx->pipelines->entries[i].kernel_id = i;
    }
    vkllm_err_t rc = vkllm_hashmap_new(&ctx->stats.node_time_cost, 1024);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_context_free(ctx);
        return rc;
    }
    if (hipGetDeviceProperties(&ctx->device->props, (int)dev) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->device->stream, hipStreamNonBlocking) != hipSuccess)
    {
        (void)hipGetLastError();
        vkllm_context_free(ctx);
        return VKLLM_ERR_VULKAN;
    }
    ctx->device->cu_count = ctx->device->props.multiProcessorCount;
    const char *mode = getenv("VKLLM_EXEC");
    ctx->device->exec_mode = (mode && strcmp(mode, "nodes") == 0) ? VKLLM_EXEC_NODES : VKLLM_EXEC_FUSED;
    ctx->device->graph_replay = env_flag("VKLLM_GRAPH", 1);
    ctx->device->timing = env_flag("VKLLM_TIMING", 0);
    *context = ctx;
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_context_free(struct vkllm_context *ctx)
{
    DeviceScope device_scope(ctx);
    if (!ctx)
        return;
    if (ctx->device)
    {
        if (ctx->device->stream)
            (void)hipStreamSynchronize(ctx->device->stream);
        if (ctx->pipelines)
            (void)timing_flush(ctx);
        for (hipEvent_t e : ctx->device->event_pool)
            (void)hipEventDestroy(e);
        if (ctx->device->op_work)
            (void)hipFree(ctx->device->op_work);
        pool_release_all(ctx->device);
        node_pool_release(ctx->device);
        if (ctx->device->stream)
            (void)hipStreamDestroy(ctx->device->stream);
        device_scope.release();
        delete ctx->device;
    }
    free(ctx->pipelines);
    if (ctx->stats.node_time_cost)
        vkllm_hashmap_free(ctx->stats.node_time_cost);
    free(ctx);
}

// ------------------------------------------------------------------------------------------------------------
// extensions (vkllm_hip.h)

extern "C" vkllm_err_t vkllm_hip_set_exec_mode(struct vkllm_context *ctx, int mode)
{
    _CHECK_ARGS(ctx && (mode == VKLLM_EXEC_FUSED || mode == VKLLM_EXEC_NODES));
    ctx->device->exec_mode = mode;
    return VKLLM_ERR_OK;
}

extern "C" int vkllm_hip_get_exec_mode(struct vkllm_context *ctx)
{
    DeviceScope device_scope(ctx);
    return ctx ? ctx->device->exec_mode : -1;
}

extern "C" vkllm_err_t vkllm_hip_set_graph_replay(struct vkllm_context *ctx, int enable)
{
    _CHECK_ARGS(ctx);
    ctx->device->graph_replay = enable ? 1 : 0;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_set_timing(struct vkllm_context *ctx, int enable)
{
    _CHECK_ARGS(ctx);
    ctx->device->timing = enable ? 1 : 0;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_synchronize(struct vkllm_context *ctx)
{
    DeviceScope device_scope(ctx);
    _CHECK_ARGS(ctx);
    HIP_TRY(hipStreamSynchronize(ctx->device->stream));
    HIP_TRY(timing_flush(ctx));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_hip_context_stream(struct vkllm_context *ctx, void **stream)
{
    _CHECK_ARGS(ctx && stream);
    *stream = (void *)ctx->device->stream;
    return VKLLM_ERR_OK;
}

extern "C" const char *vkllm_hip_device_arch(struct vkllm_context *ctx)
{
    DeviceScope device_scope(ctx);
    return ctx ? ctx->device->props.gcnArchName : "";
}

extern "C" int vkllm_hip_abi_layout(const char **names, uint64_t *values, int n)
{
#define E(_name, _val) {_name, (uint64_t)(_val)}
    static const struct
    {
        const char *name;
        uint64_t value;
    } table[] = {
        E("sizeof(vkllm_tensor)", sizeof(vkllm_tensor)),
        E("vkllm_tensor.dtype", offsetof(vkllm_tensor, dtype)),
        E("vkllm_tensor.shapes", offsetof(vkllm_tensor, shapes)),
        E("vkllm_tensor.strides", offsetof(vkllm_tensor, strides)),
        E("vkllm_tensor.bytes", offsetof(vkllm_tensor, bytes)),
        E("vkllm_tensor.data.dev", offsetof(vkllm_tensor, data.dev)),
        E("vkllm_tensor.data.host", offsetof(vkllm_tensor, data.host)),
        E("vkllm_tensor.data.mapped", offsetof(vkllm_tensor, data.mapped)),
        E("vkllm_tensor.op", offsetof(vkllm_tensor, op)),
        E("vkllm_tensor.pipeline", offsetof(vkllm_tensor, pipeline)),
        E("vkllm_tensor.srcs", offsetof(vkllm_tensor, srcs)),
        E("vkllm_tensor.params", offsetof(vkllm_tensor, params)),
        E("sizeof(vkllm_graph)", sizeof(vkllm_graph)),
        E("vkllm_graph.output_node", offsetof(vkllm_graph, output_node)),
        E("vkllm_graph.commands", offsetof(vkllm_graph, commands)),
        E("sizeof(vkllm_models_llama2)", sizeof(vkllm_models_llama2)),
        E("vkllm_models_llama2.weights", offsetof(vkllm_models_llama2, weights)),
        E("sizeof(vkllm_context)", sizeof(vkllm_context)),
        E("vkllm_context.stats", offsetof(vkllm_context, stats)),
        E("sizeof(vkllm_pipeline)", sizeof(vkllm_pipeline)),
    };
#undef E
    int total = (int)(sizeof(table) / sizeof(table[0]));
    int k = 0;
    for (; k < total && k < n; ++k)
    {
        if (names)
            names[k] = table[k].name;
        if (values)
            values[k] = table[k].value;
    }
    return names || values ? k : total;
}
