/* VKLLM_OP_ROPE. Replaces src/core/vkllm_op_rope.h:12-23 (same functions and params struct). */
#ifndef VKLLM_OP_ROPE_H
#define VKLLM_OP_ROPE_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_op_rope_params
{
    uint32_t offset; /* position of row 0 */
    float base;      /* frequency base (theta) */
    bool neox_style; /* rotate (w, w+D/2) instead of (2w, 2w+1) */
};
extern vkllm_err_t vkllm_op_rope_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_rope_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_rope_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
