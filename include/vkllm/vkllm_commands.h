/* Command batches on the context's HIP stream. Replaces src/core/vkllm_commands.h:36-52.
 * Work is enqueued on the stream as ops run (HIP streams execute eagerly), so begin/end/submit only mark the
 * batch; wait_exec synchronises the stream, refreshes the host mirrors of mapped tensors written in the batch,
 * and runs deferred host tasks. */
#ifndef VKLLM_COMMANDS_H
#define VKLLM_COMMANDS_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_array.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_gpu_device;
struct vkllm_tensor;
struct vkllm_context;

struct vkllm_commands_task
{
    vkllm_err_t (*func)(void *);
    struct vkllm_context *context;
    void *priv;
};

VKLLM_DEF_ARRAY(commands_task, struct vkllm_commands_task)

struct vkllm_commands
{
    struct vkllm_gpu_device *device;
    void *stream; /* hipStream_t */
    bool recording;
    struct vkllm_array_commands_task *defer_tasks;
    struct vkllm_array_ptr *written_mapped; /* mapped tensors written on the device in this batch */
};

/* src/core/vkllm_commands.c:96-122 */
extern vkllm_err_t vkllm_commands_new(struct vkllm_context *context, struct vkllm_commands **commands);
extern void vkllm_commands_free(struct vkllm_context *context, struct vkllm_commands *commands);
extern vkllm_err_t vkllm_commands_begin(struct vkllm_context *context, struct vkllm_commands *commands);
extern vkllm_err_t vkllm_commands_end(struct vkllm_context *context, struct vkllm_commands *commands);
/* src/core/vkllm_commands.c:172-211: bytes > tensor->bytes -> VKLLM_ERR_ARGS; mapped: host mirror + flush */
extern vkllm_err_t vkllm_commands_upload(struct vkllm_context *context, struct vkllm_commands *commands,
                                         struct vkllm_tensor *tensor, const uint8_t *data, size_t bytes);
/* src/core/vkllm_commands.c:236-269: data is complete when vkllm_commands_wait_exec returns */
extern vkllm_err_t vkllm_commands_download(struct vkllm_context *context, struct vkllm_commands *commands,
                                           struct vkllm_tensor *tensor, uint8_t *data, size_t bytes);
/* src/core/vkllm_commands.h:44-46; stream order already provides the dependency, so this is a no-op */
extern void vkllm_commands_sync_tensor(struct vkllm_context *context, struct vkllm_commands *commands,
                                       struct vkllm_tensor *tensor, uint32_t dst_access, uint32_t dst_stage);
/* src/core/vkllm_commands.c:328-359 */
extern vkllm_err_t vkllm_commands_submit(struct vkllm_context *context, struct vkllm_commands *commands);
extern vkllm_err_t vkllm_commands_wait_exec(struct vkllm_context *context, struct vkllm_commands *commands);

#ifdef __cplusplus
}
#endif
#endif
