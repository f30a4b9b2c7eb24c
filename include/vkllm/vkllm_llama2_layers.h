/* LLaMA-2 sub-graph builders. Replaces src/models/vkllm_llama2_layers.h:11-49 (same structs and functions). */
#ifndef VKLLM_LLAMA2_LAYERS_H
#define VKLLM_LLAMA2_LAYERS_H
#include <stdint.h>
#include "vkllm_errors.h"
#include "vkllm_op_rope.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_context;
struct vkllm_graph;
struct vkllm_tensor;
struct vkllm_kvcache;

struct vkllm_llama2_self_attn_layer_params
{
    struct vkllm_tensor *WK, *WQ, *WV, *WO;
    struct vkllm_tensor *norm_weight;
    float norm_power;
    float norm_eps;
    float freq_base;
    uint32_t offsets;
    uint32_t num_head;
};

struct vkllm_llama2_ffn_layer_params
{
    struct vkllm_tensor *WU, *WG, *WD;
    struct vkllm_tensor *norm_weight;
    float norm_power;
    float norm_eps;
};

struct vkllm_llama2_transformer_block_params
{
    struct vkllm_llama2_ffn_layer_params ffn;
    struct vkllm_llama2_self_attn_layer_params attn;
};

/* src/models/vkllm_llama2_layers.c:98-340 */
extern vkllm_err_t vkllm_llama2_build_self_attn_layer(struct vkllm_context *context, struct vkllm_graph *graph,
                                                      struct vkllm_kvcache *kvcache, struct vkllm_tensor *input,
                                                      struct vkllm_llama2_self_attn_layer_params params,
                                                      uint32_t block_idx);
/* src/models/vkllm_llama2_layers.c:13-96 */
extern vkllm_err_t vkllm_llama2_build_ffn_layer(struct vkllm_context *context, struct vkllm_graph *graph,
                                                struct vkllm_tensor *input, struct vkllm_llama2_ffn_layer_params params,
                                                uint32_t block_idx);
/* src/models/vkllm_llama2_layers.c:342-354 */
extern vkllm_err_t vkllm_llama2_build_transformer_block(struct vkllm_context *context, struct vkllm_graph *graph,
                                                        struct vkllm_kvcache *kvcache, struct vkllm_tensor *input,
                                                        struct vkllm_llama2_transformer_block_params params,
                                                        uint32_t block_idx);

#ifdef __cplusplus
}
#endif
#endif
