"""Parity at the kernel shapes the long workloads run, at their real widths, against the oracle.

* LLaMA-2-13B widths (dim 5120, 40 heads of 128, FFN 13824), one layer, vocabulary 1000: the 2048-token prompt step
  of the 13B workload, every row, then teacher-forced decode. That step runs the 128 x 320 residual tiles of the Wo and
  down products, the [Wu;Wg] product in full 256 x 256 rounds plus its split-K tail, and 40-head causal attention over
  2048 positions.
* LLaMA-2-7B widths (dim 4096, 32 heads of 128, FFN 11008), one layer, vocabulary 1000, a 4096-position cache: a
  4000-token prompt in four chunks, then teacher-forced decode through position 4095 on the one-launch long-cache
  attention (32 heads x 16 chunks of 256 positions at the end, 512 blocks resident at once), the cache the 7B
  long-context workload decodes to.

Reference path: src/models/vkllm_llama2_layers.c:98-354 (the layer), :223-257 with src/shaders/vkllm_softmax.comp:42-96
(the attention), tests/vkllm_test_infer_gguf.c:181-272 (the loop). Bar (one layer, so fp16 weights with fp32 sums):
logits within 2e-2 of the oracle on every row and step; ids equal, except at a one-ulp tie in the oracle's logits (fp32 summation
order alone decides such a row).
"""
import numpy as np
import pytest

from helpers import forced_decode, prompt_rows

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def _models(oracle, vk, ctx, shape, seed):
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=seed)
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    return cfg, ref, vk.Model(ctx, config=vcfg, seed=seed)


@pytest.mark.timeout(600)  # the oracle's 2048-token step at the 13B widths runs on the host's cores
def test_13b_widths_2048_token_prompt(ctx, vk, oracle):
    shape = dict(n_layer=1, dim=5120, n_head=40, ffn=13824, vocab=1000, ctx=2176)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=61)
    try:
        prompt = oracle.prompt_tokens(62, 2048, cfg.vocab)
        want_ids, ties = prompt_rows(ref, model, prompt, 0, "13b 2048", LOGIT_TOL)
        assert ties <= 2048 // 100
        _, ties, _ = forced_decode(ref, model, want_ids[-1], 2048, 8, "13b 2048", LOGIT_TOL)
        assert ties <= 1
    finally:
        ref.close()
        model.close()


@pytest.mark.timeout(600)  # the oracle's 4000-token prompt at the 7B widths runs on the host's cores
def test_7b_widths_decode_to_4096_positions(ctx, vk, oracle):
    shape = dict(n_layer=1, dim=4096, n_head=32, ffn=11008, vocab=1000, ctx=4096)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=71)
    try:
        prompt = oracle.prompt_tokens(72, 4000, cfg.vocab)
        offset, ties = 0, 0
        for n in (1024, 1024, 1024, 928):
            want_ids, t = prompt_rows(ref, model, prompt[offset:offset + n], offset, "7b 4096", LOGIT_TOL)
            ties += t
            offset += n
        assert ties <= 4000 // 100
        # decode with the captured graphs replayed, then the last 8 positions launched directly with timing on, whose
        # kernel counts show that every one of them took the one-launch long-cache attention
        last = 8
        n = shape["ctx"] - offset - last
        _, ties, tok = forced_decode(ref, model, want_ids[-1], offset, n, "7b 4096", LOGIT_TOL)
        ctx.set_timing(True)
        ctx.reset_kernel_stats()
        try:
            _, t2, _ = forced_decode(ref, model, tok, offset + n, last, "7b 4096 timed", LOGIT_TOL)
            stats = ctx.kernel_stats()
        finally:
            ctx.set_timing(False)
        assert ties + t2 <= 2
        print(f"[7b 4096] attention launches: {({k: v[0] for k, v in stats.items() if 'attn' in k})}", flush=True)
        assert stats.get("fused_attn_long", (0, 0))[0] == last
        assert stats.get("fused_attn_scores", (0, 0))[0] == 0 and stats.get("fused_attn_small", (0, 0))[0] == 0
    finally:
        ref.close()
        model.close()
