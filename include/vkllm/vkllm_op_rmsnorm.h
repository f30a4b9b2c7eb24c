/* VKLLM_OP_RMSNORM. Replaces src/core/vkllm_op_rmsnorm.h:14-25 (same functions and params struct). */
#ifndef VKLLM_OP_RMSNORM_H
#define VKLLM_OP_RMSNORM_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_op_rmsnorm_params
{
    float power; /* carried but unused, as in the reference */
    float eps;
};
extern vkllm_err_t vkllm_op_rmsnorm_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_rmsnorm_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_rmsnorm_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
