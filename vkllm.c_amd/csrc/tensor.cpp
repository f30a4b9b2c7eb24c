// Tensors: HBM storage (pooled, allocated on first use for op outputs), pinned host mirrors for mapped tensors,
// and the reference's view operations. Replaces src/core/vkllm_tensor.c:13-335.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "runtime.h"

// dst = src + suffix, truncated to n - 1 bytes (views are made for every node of every step; no formatted print)
static void name_with_suffix(char *dst, size_t n, const char *src, const char *suffix)
{
    const size_t ls = strnlen(src, n - 1);
    memcpy(dst, src, ls);
    const size_t lx = strnlen(suffix, n - 1 - ls);
    memcpy(dst + ls, suffix, lx);
    dst[ls + lx] = '\0';
}

// contiguous byte strides, W innermost (src/core/vkllm_tensor.c:13-31)
static void calc_strides(const uint32_t *shapes, vkllm_dtype_t dtype, uint32_t *strides)
{
    uint32_t eb = dtype_bytes(dtype);
    strides[3] = eb;
    strides[2] = shapes[3] * eb;
    strides[1] = shapes[2] * strides[2];
    strides[0] = shapes[1] * strides[1];
}

// Tensor structs are recycled per device: a decode step builds and frees one per graph node (741 at 32 layers),
// and a calloc/free pair per node costs more than building it. Each struct sits behind a header that records its
// params capacity; structs of the common capacity go back to the device's free list, others to free().
namespace
{
constexpr size_t kNodeParamsCap = 64;
constexpr size_t kNodeFreeMax = 1u << 14;
struct alignas(16) NodeHdr
{
    size_t params_cap;
};
} // namespace

static vkllm_tensor *node_alloc(vkllm_gpu_device *dev, size_t params_bytes)
{
    const size_t cap = params_bytes <= kNodeParamsCap ? kNodeParamsCap : params_bytes;
    const size_t total = sizeof(NodeHdr) + sizeof(vkllm_tensor) + cap;
    NodeHdr *h = nullptr;
    if (cap == kNodeParamsCap && dev && !dev->node_free.empty())
    {
        h = (NodeHdr *)dev->node_free.back();
        dev->node_free.pop_back();
        memset(h, 0, total);
    }
    else if (!(h = (NodeHdr *)calloc(1, total)))
        return nullptr;
    h->params_cap = cap;
    return (vkllm_tensor *)(h + 1);
}

static void node_release(vkllm_gpu_device *dev, vkllm_tensor *t)
{
    NodeHdr *h = (NodeHdr *)t - 1;
    if (h->params_cap == kNodeParamsCap && dev && dev->node_free.size() < kNodeFreeMax)
    {
        try
        {
            dev->node_free.push_back(h);
            return;
        }
        catch (...)
        {
        }
    }
    free(h);
}

void node_pool_release(vkllm_gpu_device *dev)
{
    for (void *p : dev->node_free)
        free(p);
    dev->node_free.clear();
}

vkllm_tensor *tensor_base(vkllm_tensor *t)
{
    while (t && t->data.is_ref && t->srcs[0])
        t = t->srcs[0];
    return t;
}

void *tensor_dev(vkllm_context *ctx, vkllm_tensor *t)
{
    vkllm_tensor *b = tensor_base(t);
    if (!b)
        return nullptr;
    if (!b->data.dev && !b->data.is_ref && !b->data.borrowed)
        b->data.dev = pool_alloc(ctx->device, b->bytes);
    return b->data.dev;
}

vk::TView tview(vkllm_context *ctx, vkllm_tensor *t)
{
    vk::TView v;
    v.p = tensor_dev(ctx, t);
    uint32_t eb = dtype_bytes(t->dtype);
    for (int i = 0; i < 4; ++i)
    {
        v.n[i] = t->shapes[i];
        v.s[i] = eb ? t->strides[i] / eb : 0;
    }
    v.dt = (int32_t)t->dtype;
    return v;
}

extern "C" vkllm_err_t vkllm_tensor_new(struct vkllm_context *context, const char *name, const uint32_t *shapes,
                                        vkllm_dtype_t dtype, vkllm_op_t op, struct vkllm_tensor **srcs,
                                        const uint32_t n_srcs, const void *params, size_t params_bytes, bool mapped,
                                        struct vkllm_tensor **p)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && p);
    if (!shapes)
    {
        log_error("shape is empty. shapes is NULL");
        return VKLLM_ERR_ARGS;
    }
    for (int i = 0; i < 4; ++i)
        if (shapes[i] == 0)
        {
            log_error("shape is empty. shapes[%d] is 0", i);
            return VKLLM_ERR_ARGS;
        }
    if (dtype_bytes(dtype) == 0)
    {
        log_error("unknown dtype %d", (int)dtype);
        return VKLLM_ERR_ARGS;
    }
    _CHECK_ARGS(n_srcs <= VKLLM_MAX_SRCS);
    uint64_t total = (uint64_t)shapes[0] * shapes[1] * shapes[2] * shapes[3] * dtype_bytes(dtype);
    uint64_t aligned = (total + 255) / 256 * 256;
    if (aligned > 0xffffffffull)
    {
        log_error("tensor %s is %llu bytes; the byte count and strides are 32-bit", name ? name : "",
                  (unsigned long long)total);
        return VKLLM_ERR_ARGS;
    }
    auto *t = node_alloc(context->device, params_bytes);
    if (!t)
        return VKLLM_ERR_ALLOC;
    if (name)
        memcpy((char *)t->name, name, strnlen(name, sizeof(t->name) - 1)); // the zeroed struct holds the terminator
    t->dtype = dtype;
    memcpy(t->shapes, shapes, sizeof(t->shapes));
    calc_strides(shapes, dtype, t->strides);
    t->bytes = (uint32_t)aligned;
    t->device = context->device;
    t->op = op;
    for (uint32_t i = 0; i < n_srcs; ++i)
        t->srcs[i] = srcs ? srcs[i] : nullptr;
    if (params && params_bytes)
        memcpy(t->params, params, params_bytes);
    t->data.mapped = mapped;
    if (mapped)
    {
        t->data.host = pinned_alloc(context->device, t->bytes);
        if (!t->data.host)
        {
            node_release(context->device, t);
            return VKLLM_ERR_ALLOC;
        }
        memset(t->data.host, 0, t->bytes);
    }
    // inputs, constants, caches and mapped tensors are backed now; other op outputs on first use
    if (mapped || op == VKLLM_OP_NONE || op == VKLLM_OP_UPDATE_ROWS)
    {
        if (!tensor_dev(context, t))
        {
            pinned_free(context->device, t->data.host, t->bytes);
            node_release(context->device, t);
            return VKLLM_ERR_ALLOC;
        }
    }
    context->stats.tensor_alloc_counts += 1;
    *p = t;
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_tensor_free(struct vkllm_context *context, struct vkllm_tensor *t)
{
    DeviceScope device_scope(context);
    if (!t)
        return;
    if (!t->data.is_ref)
    {
        if (t->data.dev && !t->data.borrowed)
            pool_free(context->device, t->data.dev, t->bytes);
        if (t->data.host)
            pinned_free(context->device, t->data.host, t->bytes);
    }
    node_release(context->device, t);
    context->stats.tensor_free_counts += 1;
}

extern "C" vkllm_err_t vkllm_tensor_flush_cache(struct vkllm_context *context, struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && tensor);
    if (!tensor->data.mapped)
    {
        log_error("can only flush mapped buffer.");
        return VKLLM_ERR_ARGS;
    }
    vkllm_tensor *b = tensor_base(tensor);
    void *dev = tensor_dev(context, b);
    if (!dev)
        return VKLLM_ERR_ALLOC;
    HIP_TRY(hipMemcpyAsync(dev, b->data.host, b->bytes, hipMemcpyHostToDevice, context->device->stream));
    b->data.valid = true;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_invalid_cache(struct vkllm_context *context, struct vkllm_tensor *tensor)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && tensor);
    if (!tensor->data.mapped)
    {
        log_error("can only invalid mapped buffer.");
        return VKLLM_ERR_ARGS;
    }
    vkllm_tensor *b = tensor_base(tensor);
    void *dev = tensor_dev(context, b);
    if (!dev)
        return VKLLM_ERR_ALLOC;
    // the host mirror is brought up to date only when the device holds newer contents; a mirror that is current (a
    // fused step writes its arg-max ids there once they are final) needs no wait, so work queued behind it (a step
    // launched ahead) keeps running while the caller reads
    if (b->data.valid && !b->data.host_current)
    {
        HIP_TRY(hipMemcpyAsync(b->data.host, dev, b->bytes, hipMemcpyDeviceToHost, context->device->stream));
        HIP_TRY(hipStreamSynchronize(context->device->stream));
        b->data.host_current = true;
    }
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_new_staging(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                                struct vkllm_tensor **staging)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && tensor && staging);
    return vkllm_tensor_new(context, "", tensor->shapes, tensor->dtype, VKLLM_OP_NONE, nullptr, 0, nullptr, 0, true,
                            staging);
}

extern "C" vkllm_err_t vkllm_tensor_reshape(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                            const uint32_t *shapes)
{
    _CHECK_ARGS(context && tensor && shapes);
    _CHECK_ARGS((uint64_t)tensor->shapes[0] * tensor->shapes[1] * tensor->shapes[2] * tensor->shapes[3] ==
                (uint64_t)shapes[0] * shapes[1] * shapes[2] * shapes[3]);
    memcpy(tensor->shapes, shapes, sizeof(tensor->shapes));
    calc_strides(shapes, tensor->dtype, tensor->strides);
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_permute(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                            const uint32_t *axis)
{
    _CHECK_ARGS(context && tensor && axis);
    _CHECK_ARGS(axis[0] < 4 && axis[1] < 4 && axis[2] < 4 && axis[3] < 4);
    uint32_t sh[4], st[4];
    memcpy(sh, tensor->shapes, sizeof(sh));
    memcpy(st, tensor->strides, sizeof(st));
    for (int i = 0; i < 4; ++i)
    {
        tensor->shapes[i] = sh[axis[i]];
        tensor->strides[i] = st[axis[i]];
    }
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_copy_ref(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                             struct vkllm_tensor **p)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && tensor && p);
    auto *t = node_alloc(context->device, 0);
    if (!t)
        return VKLLM_ERR_ALLOC;
    name_with_suffix((char *)t->name, sizeof(t->name), tensor->name, "_ref");
    t->dtype = tensor->dtype;
    memcpy(t->shapes, tensor->shapes, sizeof(t->shapes));
    memcpy(t->strides, tensor->strides, sizeof(t->strides));
    t->bytes = tensor->bytes;
    t->device = tensor->device;
    t->data.dev = nullptr; // resolved through srcs[0] when used
    t->data.host = tensor->data.host;
    t->data.mapped = tensor->data.mapped;
    t->data.is_ref = true;
    t->op = VKLLM_OP_REF;
    t->srcs[0] = tensor;
    context->stats.tensor_alloc_counts += 1;
    *p = t;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_slice0(struct vkllm_context *context, struct vkllm_tensor *tensor,
                                           uint32_t extents[4], struct vkllm_tensor **slice)
{
    _CHECK_ARGS(context && tensor && extents && slice);
    for (int i = 0; i < 4; ++i)
        _CHECK_ARGS(extents[i] <= tensor->shapes[i] && extents[i] > 0);
    _CHECK(vkllm_tensor_copy_ref(context, tensor, slice));
    vkllm_tensor *t = *slice;
    name_with_suffix((char *)t->name, sizeof(t->name), tensor->name, "_slice0");
    memcpy(t->shapes, extents, sizeof(t->shapes));
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_tensor_s(struct vkllm_context *context, struct vkllm_tensor *tensor, char *buf,
                                      size_t len)
{
    _CHECK_ARGS(context && tensor && buf && len > 0);
    int n = snprintf(buf, len, "%s<%s>[%u, %u, %u, %u]", tensor->name, vkllm_dtype_s(tensor->dtype),
                     tensor->shapes[0], tensor->shapes[1], tensor->shapes[2], tensor->shapes[3]);
    if (n < 0 || (size_t)n >= len)
        return VKLLM_ERR_ARGS;
    return VKLLM_ERR_OK;
}
