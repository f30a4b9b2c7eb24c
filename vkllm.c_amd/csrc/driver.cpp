// The reference driver's token loop (tests/vkllm_test_infer_gguf.c:181-272) as a library call, so a host can time
// the public API's per-token sequence without an interpreter in the loop.
#include <chrono>
#include <cstring>

#include "runtime.h"
#include "vkllm/vkllm_models_llama2.h"

static uint64_t now_ns()
{
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

extern "C" vkllm_err_t vkllm_hip_token_loop(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                            const uint32_t *prompt, uint32_t prompt_len, uint32_t offset0,
                                            uint32_t n_steps, uint32_t *ids, uint64_t *step_ns, uint64_t *phase_ns)
{
    DeviceScope device_scope(context);
    _CHECK_ARGS(context && model && prompt && prompt_len > 0 && ids);
    if (phase_ns)
        memset(phase_ns, 0, 4 * sizeof(uint64_t));
    uint32_t offset = offset0, next = 0;
    for (uint32_t i = 0; i < n_steps; ++i)
    {
        const uint32_t S = i == 0 ? prompt_len : 1;
        const uint32_t *toks = i == 0 ? prompt : &next;
        const uint64_t t0 = now_ns();
        struct vkllm_tensor *input_toks = nullptr;
        const uint32_t shapes[] = {1, 1, 1, S};
        _CHECK(vkllm_tensor_new(context, "input_toks", shapes, vkllm_dtype_uint32, VKLLM_OP_NONE, nullptr, 0, nullptr,
                                0, true, &input_toks));
        struct vkllm_graph *graph = nullptr;
        vkllm_err_t rc = vkllm_graph_new(context, &graph);
        if (rc != VKLLM_ERR_OK)
        {
            vkllm_tensor_free(context, input_toks);
            return rc;
        }
        // build_graph adopts input_toks into the graph and frees the graph itself on failure
        _CHECK(vkllm_models_llama2_build_graph(context, model, input_toks, graph, offset));
        const uint64_t t1 = now_ns();
        rc = vkllm_graph_init(context, graph);
        if (rc == VKLLM_ERR_OK)
            rc = vkllm_commands_upload(context, graph->commands, input_toks, (const uint8_t *)toks,
                                       sizeof(uint32_t) * S);
        const uint64_t t2 = now_ns();
        if (rc == VKLLM_ERR_OK)
            rc = vkllm_graph_run(context, graph);
        if (rc == VKLLM_ERR_OK)
            rc = vkllm_graph_post_run(context, graph);
        const uint64_t t3 = now_ns();
        if (rc == VKLLM_ERR_OK)
            rc = vkllm_tensor_invalid_cache(context, graph->output_node);
        if (rc == VKLLM_ERR_OK)
        {
            const struct vkllm_tensor *out = graph->output_node;
            next = ((const uint32_t *)out->data.host)[S - 1];
            ids[i] = next;
        }
        vkllm_graph_free(context, graph);
        const uint64_t t4 = now_ns();
        if (rc != VKLLM_ERR_OK)
            return rc;
        if (step_ns)
            step_ns[i] = t4 - t0;
        if (phase_ns && i > 0)
        {
            phase_ns[0] += t1 - t0;
            phase_ns[1] += t2 - t1;
            phase_ns[2] += t3 - t2;
            phase_ns[3] += t4 - t3;
        }
        offset += S;
    }
    return VKLLM_ERR_OK;
}
