/* Operator tags. Replaces src/core/vkllm_ops.h:8-25 (same values). */
#ifndef VKLLM_OPS_H
#define VKLLM_OPS_H
#ifdef __cplusplus
extern "C" {
#endif

typedef enum
{
    VKLLM_OP_NONE = 0,
    VKLLM_OP_COPY = 1,
    VKLLM_OP_BIN = 2,
    VKLLM_OP_EMBEDDING = 3,
    VKLLM_OP_RMSNORM = 4,
    VKLLM_OP_MATMUL = 5,
    VKLLM_OP_ROPE = 6,
    VKLLM_OP_SOFTMAX = 7,
    VKLLM_OP_FFN_UP_AND_GATE = 8,
    VKLLM_OP_UPDATE_ROWS = 9,
    VKLLM_OP_ARG_MAX = 10,
    VKLLM_OP_REF = 11,
    VKLLM_OP_COUNTS = 12,
} vkllm_op_t;

/* "VKLLM_OP_NONE" ... "VKLLM_OP_REF" */
extern const char *vkllm_op_s(const vkllm_op_t op);

#ifdef __cplusplus
}
#endif
#endif
