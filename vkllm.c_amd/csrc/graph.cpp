// Graphs: node lists, post-order execution from the output node, and dispatch to a fused plan when the graph
// was built by vkllm_models_llama2_build_graph. Replaces src/core/vkllm_graph.c:19-369.
#include <cstdlib>
#include <unordered_set>

#include "runtime.h"

extern "C" vkllm_err_t vkllm_graph_new(struct vkllm_context *context, struct vkllm_graph **graph)
{
    _CHECK_ARGS(context && graph);
    auto *g = (vkllm_graph *)calloc(1, sizeof(vkllm_graph));
    if (!g)
        return VKLLM_ERR_ALLOC;
    vkllm_err_t rc = vkllm_array_tensor_new(&g->input_nodes, 8);
    if (rc == VKLLM_ERR_OK)
        rc = vkllm_array_tensor_new(&g->nodes, 128);
    if (rc == VKLLM_ERR_OK)
        rc = vkllm_commands_new(context, &g->commands);
    if (rc != VKLLM_ERR_OK)
    {
        vkllm_array_tensor_free(g->input_nodes);
        vkllm_array_tensor_free(g->nodes);
        free(g);
        return rc;
    }
    *graph = g;
    return VKLLM_ERR_OK;
}

extern "C" vkllm_err_t vkllm_graph_add_input(struct vkllm_context *context, struct vkllm_graph *graph,
                                             struct vkllm_tensor *tensor)
{
    _CHECK_ARGS(context && graph && tensor);
    _CHECK(vkllm_array_tensor_append(graph->input_nodes, tensor));
    return vkllm_graph_add_node(context, graph, tensor);
}

extern "C" vkllm_err_t vkllm_graph_add_node(struct vkllm_context *context, struct vkllm_graph *graph,
                                            struct vkllm_tensor *tensor)
{
    _CHECK_ARGS(context && graph && tensor);
    return vkllm_array_tensor_append(graph->nodes, tensor);
}

extern "C" vkllm_err_t vkllm_graph_set_output(struct vkllm_context *context, struct vkllm_graph *graph,
                                              struct vkllm_tensor *tensor)
{
    _CHECK_ARGS(context && graph && tensor);
    graph->output_node = tensor;
    return VKLLM_ERR_OK;
}

// Post-order over srcs from `root`, each node once. Iterative so deep graphs (13B: ~1000 nodes) cannot overflow
// the stack.
template <typename F> static vkllm_err_t visit_post_order(vkllm_tensor *root, F &&fn)
{
    std::unordered_set<vkllm_tensor *> done;
    struct Frame
    {
        vkllm_tensor *t;
        int next;
    };
    std::vector<Frame> stack;
    std::unordered_set<vkllm_tensor *> on_stack;
    stack.push_back({root, 0});
    on_stack.insert(root);
    while (!stack.empty())
    {
        Frame &f = stack.back();
        if (f.next < VKLLM_MAX_SRCS)
        {
            vkllm_tensor *s = f.t->srcs[f.next++];
            if (s && !done.count(s))
            {
                if (on_stack.count(s))
                {
                    log_error("graph has a cycle through %s", s->name);
                    return VKLLM_ERR_ARGS;
                }
                stack.push_back({s, 0});
                on_stack.insert(s);
            }
            continue;
        }
        vkllm_tensor *t = f.t;
        stack.pop_back();
        on_stack.erase(t);
        done.insert(t);
        vkllm_err_t rc = fn(t);
        if (rc != VKLLM_ERR_OK)
            return rc;
    }
    return VKLLM_ERR_OK;
}

static bool use_fused(vkllm_context *ctx, vkllm_graph *g)
{
    return g->plan && ctx->device->exec_mode == VKLLM_EXEC_FUSED;
}

extern "C" vkllm_err_t vkllm_graph_init(struct vkllm_context *context, struct vkllm_graph *graph)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && graph->output_node && graph->commands);
    // a fused step runs none of the node kernels: its plan validates what the fused kernels need instead
    if (use_fused(context, graph))
        return fused_plan_init(context, graph);
    return visit_post_order(graph->output_node,
                            [&](vkllm_tensor *t) { return op_init(context, graph->commands, t); });
}

extern "C" vkllm_err_t vkllm_graph_run(struct vkllm_context *context, struct vkllm_graph *graph)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && graph->output_node && graph->commands);
    if (use_fused(context, graph))
        return fused_plan_run(context, graph);
    if (graph->plan) // node by node over a model whose fused steps may have launched one ahead
        _CHECK(fused_plan_discard_ahead(context, graph));
    _CHECK(vkllm_commands_begin(context, graph->commands));
    vkllm_err_t rc =
        visit_post_order(graph->output_node, [&](vkllm_tensor *t) { return op_run(context, graph->commands, t); });
    _CHECK(vkllm_commands_end(context, graph->commands));
    _CHECK(vkllm_commands_submit(context, graph->commands));
    vkllm_err_t wrc = vkllm_commands_wait_exec(context, graph->commands);
    return rc != VKLLM_ERR_OK ? rc : wrc;
}

extern "C" vkllm_err_t vkllm_graph_post_run(struct vkllm_context *context, struct vkllm_graph *graph)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph && graph->output_node && graph->commands);
    // a fused step ran none of the node kernels, so there is no per-node post-run work
    if (use_fused(context, graph))
        return VKLLM_ERR_OK;
    return visit_post_order(graph->output_node,
                            [&](vkllm_tensor *t) { return op_post_run(context, graph->commands, t); });
}

extern "C" vkllm_err_t vkllm_graph_free(struct vkllm_context *context, struct vkllm_graph *graph)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && graph);
    // queued node kernels may still read these tensors. A fused step's kernels read none of them (only the model's
    // buffers), so after one the next step, if it was launched ahead, keeps running while the graph is freed.
    if (!(graph->plan && fused_plan_ran(graph->plan)))
        (void)hipStreamSynchronize(context->device->stream);
    for (size_t i = 0; i < graph->nodes->used_n; ++i)
        vkllm_tensor_free(context, graph->nodes->data[i]);
    vkllm_array_tensor_free(graph->nodes);
    vkllm_array_tensor_free(graph->input_nodes);
    vkllm_commands_free(context, graph->commands);
    if (graph->plan)
        fused_plan_free(graph->plan);
    free(graph);
    return VKLLM_ERR_OK;
}
