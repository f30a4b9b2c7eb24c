/* VKLLM_OP_ARG_MAX. Replaces src/core/vkllm_op_arg_max.h (same functions and params struct). */
#ifndef VKLLM_OP_ARG_MAX_H
#define VKLLM_OP_ARG_MAX_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif
/* srcs[0] [B,C,H,W] -> uint32 [B,C,H,1] */
extern vkllm_err_t vkllm_op_arg_max_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_arg_max_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_arg_max_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
