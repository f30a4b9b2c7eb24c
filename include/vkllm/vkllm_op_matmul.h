/* VKLLM_OP_MATMUL. Replaces src/core/vkllm_op_matmul.h:12-23 (same functions and params struct). */
#ifndef VKLLM_OP_MATMUL_H
#define VKLLM_OP_MATMUL_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_op_matmul_params
{
    float scale;
    int32_t act; /* 1 = SiLU */
};
extern vkllm_err_t vkllm_op_matmul_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_matmul_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_matmul_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
