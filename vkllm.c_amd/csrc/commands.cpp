// Command batches on the context's HIP stream. Replaces src/core/vkllm_commands.c:96-369.
// HIP streams execute in order as work is enqueued, so there is no command buffer to record: ops launch their
// kernels when run, uploads and downloads are stream-ordered copies, and wait_exec is a stream synchronisation
// followed by the host-side work the reference defers to that point (mapped-tensor readback, deferred tasks).
#include <cstdlib>
#include <cstring>

#include "runtime.h"

extern "C" vkllm_err_t vkllm_commands_new(struct vkllm_context *context, struct vkllm_commands **commands)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands);
    auto *c = (vkllm_commands *)calloc(1, sizeof(vkllm_commands));
    if (!c)
        return VKLLM_ERR_ALLOC;
    c->device = context->device;
    c->stream = context->device->stream;
    if (vkllm_array_commands_task_new(&c->defer_tasks, 16) != VKLLM_ERR_OK ||
        vkllm_array_ptr_new(&c->written_mapped, 16) != VKLLM_ERR_OK)
    {
        vkllm_array_commands_task_free(c->defer_tasks);
        free(c);
        return VKLLM_ERR_ALLOC;
    }
    *commands = c;
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_commands_free(struct vkllm_context *context, struct vkllm_commands *commands)
{
    DeviceScope device_scope(context);
    if (!commands)
        return;
    vkllm_array_commands_task_free(commands->defer_tasks);
    vkllm_array_ptr_free(commands->written_mapped);
    free(commands);
}

extern "C" vkllm_err_t vkllm_commands_begin(struct vkllm_context *context, struct vkllm_commands *commands)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands);
    commands->recording = true;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_commands_end(struct vkllm_context *context, struct vkllm_commands *commands)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands);
    commands->recording = false;
    return VKLLM_ERR_OK;
}

void commands_note_write(vkllm_commands *cmds, vkllm_tensor *t)
{
    vkllm_tensor *b = tensor_base(t);
    b->data.valid = true;
    b->data.host_current = false;
    if (!b->data.mapped || !cmds)
        return;
    for (size_t i = 0; i < cmds->written_mapped->used_n; ++i)
        if (cmds->written_mapped->data[i] == b)
            return;
    vkllm_array_ptr_append(cmds->written_mapped, b);
}

extern "C" vkllm_err_t vkllm_commands_upload(struct vkllm_context *context, struct vkllm_commands *commands,
                                             struct vkllm_tensor *tensor, const uint8_t *data, size_t bytes)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor && data);
    _CHECK_ARGS(bytes <= tensor->bytes);
    vkllm_tensor *b = tensor_base(tensor);
    if (tensor->data.mapped && b->data.host)
    {
        memcpy(b->data.host, data, bytes);
        return vkllm_tensor_flush_cache(context, tensor);
    }
    void *dev = tensor_dev(context, tensor);
    if (!dev)
        return VKLLM_ERR_ALLOC;
    // pageable source: complete the copy before returning so the caller may reuse `data`
    HIP_TRY(hipMemcpyAsync(dev, data, bytes, hipMemcpyHostToDevice, context->device->stream));
    HIP_TRY(hipStreamSynchronize(context->device->stream));
    b->data.valid = true;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_commands_download(struct vkllm_context *context, struct vkllm_commands *commands,
                                               struct vkllm_tensor *tensor, uint8_t *data, size_t bytes)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands && tensor && data);
    _CHECK_ARGS(bytes <= tensor->bytes);
    vkllm_tensor *b = tensor_base(tensor);
    if (b->data.host_current && b->data.host)
    {
        HIP_TRY(hipStreamSynchronize(context->device->stream));
        memcpy(data, b->data.host, bytes);
        return VKLLM_ERR_OK;
    }
    if (!b->data.valid)
    {
        log_error("tensor %s has no device contents (never written, or an intermediate of a fused step; set "
                  "VKLLM_EXEC=nodes to materialise intermediates)",
                  tensor->name);
        return VKLLM_ERR_ARGS;
    }
    void *dev = tensor_dev(context, tensor);
    if (!dev)
        return VKLLM_ERR_ALLOC;
    HIP_TRY(hipMemcpyAsync(data, dev, bytes, hipMemcpyDeviceToHost, context->device->stream));
    HIP_TRY(hipStreamSynchronize(context->device->stream));
    return VKLLM_ERR_OK;
}

extern "C" void vkllm_commands_sync_tensor(struct vkllm_context *context, struct vkllm_commands *commands,
                                           struct vkllm_tensor *tensor, uint32_t dst_access, uint32_t dst_stage)
{
    DeviceScope device_scope(context);
    __UNUSED(context);
    __UNUSED(commands);
    __UNUSED(tensor);
    __UNUSED(dst_access);
    __UNUSED(dst_stage);
}

extern "C" vkllm_err_t vkllm_commands_submit(struct vkllm_context *context, struct vkllm_commands *commands)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands);
    HIP_TRY(hipGetLastError());
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_commands_wait_exec(struct vkllm_context *context, struct vkllm_commands *commands)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && commands);
    hipStream_t st = context->device->stream;
    for (size_t i = 0; i < commands->written_mapped->used_n; ++i)
    {
        auto *t = (vkllm_tensor *)commands->written_mapped->data[i];
        HIP_TRY(hipMemcpyAsync(t->data.host, t->data.dev, t->bytes, hipMemcpyDeviceToHost, st));
    }
    HIP_TRY(hipStreamSynchronize(st));
    HIP_TRY(timing_flush(context));
    commands->written_mapped->used_n = 0;
    vkllm_err_t rc = VKLLM_ERR_OK;
    for (size_t i = 0; i < commands->defer_tasks->used_n; ++i)
    {
        vkllm_commands_task *task = &commands->defer_tasks->data[i];
        vkllm_err_t r = task->func(task);
        if (r != VKLLM_ERR_OK)
            rc = r;
    }
    commands->defer_tasks->used_n = 0;
    return rc;
}
