/* Computation graphs. Replaces src/core/vkllm_graph.h:11-29 (same functions and fields; extern "C" added).
 * init/run/post_run visit the nodes reachable from output_node in post-order, as the reference does
 * (src/core/vkllm_graph.c:58-307). A graph built by vkllm_models_llama2_build_graph additionally carries a
 * fused execution plan (`plan`): run then executes the whole token step as fused gfx950 kernels (a captured
 * hipGraph for decode) instead of node by node. */
#ifndef VKLLM_GRAPH_H
#define VKLLM_GRAPH_H
#include "vkllm_array.h"
#ifdef __cplusplus
extern "C" {
#endif

struct vkllm_tensor;
struct vkllm_context;
struct vkllm_commands;

VKLLM_DEF_ARRAY(tensor, struct vkllm_tensor *)

struct vkllm_graph
{
    struct vkllm_array_tensor *nodes;
    struct vkllm_array_tensor *input_nodes;
    struct vkllm_tensor *output_node;
    struct vkllm_commands *commands;
    void *plan; /* fused execution plan, NULL for hand-built graphs */
};

extern vkllm_err_t vkllm_graph_new(struct vkllm_context *context, struct vkllm_graph **graph);
extern vkllm_err_t vkllm_graph_add_input(struct vkllm_context *context, struct vkllm_graph *graph,
                                         struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_graph_set_output(struct vkllm_context *context, struct vkllm_graph *graph,
                                          struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_graph_add_node(struct vkllm_context *context, struct vkllm_graph *graph,
                                        struct vkllm_tensor *tensor);
extern vkllm_err_t vkllm_graph_init(struct vkllm_context *context, struct vkllm_graph *graph);
/* synchronous: results (and the host mirror of a mapped output) are ready on return */
extern vkllm_err_t vkllm_graph_run(struct vkllm_context *context, struct vkllm_graph *graph);
extern vkllm_err_t vkllm_graph_post_run(struct vkllm_context *context, struct vkllm_graph *graph);
/* frees every node added to the graph, inputs included (src/core/vkllm_graph.c:354-369) */
extern vkllm_err_t vkllm_graph_free(struct vkllm_context *context, struct vkllm_graph *graph);

#ifdef __cplusplus
}
#endif
#endif
