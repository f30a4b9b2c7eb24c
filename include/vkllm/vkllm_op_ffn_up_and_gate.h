/* VKLLM_OP_FFN_UP_AND_GATE. Replaces src/core/vkllm_op_ffn_up_and_gate.h (same functions and params struct). */
#ifndef VKLLM_OP_FFN_UP_AND_GATE_H
#define VKLLM_OP_FFN_UP_AND_GATE_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif
/* srcs {x, W_up, W_gate}: out = (x.W_up^T) * silu(x.W_gate^T) */
extern vkllm_err_t vkllm_op_ffn_up_and_gate_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_ffn_up_and_gate_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_ffn_up_and_gate_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
