/* VKLLM_OP_EMBEDDING. Replaces src/core/vkllm_op_embedding.h (same functions and params struct). */
#ifndef VKLLM_OP_EMBEDDING_H
#define VKLLM_OP_EMBEDDING_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif
/* params: one uint32_t unk token; srcs[0] uint32 ids [1,C,H,W], srcs[1] table [1,1,V,D] */
extern vkllm_err_t vkllm_op_embedding_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_embedding_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_embedding_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
