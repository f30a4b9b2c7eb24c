/* VKLLM_OP_SOFTMAX. Replaces src/core/vkllm_op_softmax.h:12-22 (same functions and params struct). */
#ifndef VKLLM_OP_SOFTMAX_H
#define VKLLM_OP_SOFTMAX_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_op_softmax_params
{
    int32_t seq_mask;  /* > 0: causal mask, entries i > h + offsets are excluded and written as 0 */
    uint32_t offsets;
};
extern vkllm_err_t vkllm_op_softmax_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_softmax_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_softmax_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
