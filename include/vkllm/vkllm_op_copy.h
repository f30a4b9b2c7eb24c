/* VKLLM_OP_COPY. Replaces src/core/vkllm_op_copy.h (same functions and params struct). */
#ifndef VKLLM_OP_COPY_H
#define VKLLM_OP_COPY_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif
/* srcs[0] -> tensor, strided gather into the tensor's layout */
extern vkllm_err_t vkllm_op_copy_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_copy_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_copy_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
