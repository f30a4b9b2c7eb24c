/* VKLLM_OP_UPDATE_ROWS. Replaces src/core/vkllm_op_update_rows.h:12-21 (same functions and params struct). */
#ifndef VKLLM_OP_UPDATE_ROWS_H
#define VKLLM_OP_UPDATE_ROWS_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_commands.h"
#include "vkllm_context.h"
#include "vkllm_tensor.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_op_update_rows_params
{
    uint32_t offset_rows;
};
extern vkllm_err_t vkllm_op_update_rows_init(struct vkllm_context *context, struct vkllm_commands *commands,
                                    struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_update_rows_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                   struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_op_update_rows_post_run(struct vkllm_context *context, struct vkllm_commands *commands,
                                        struct vkllm_tensor *tensor);

#ifdef __cplusplus
}
#endif
#endif
