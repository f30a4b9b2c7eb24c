"""Vocabularies whose size is not a multiple of 4 (LLaMA-2 variants ship 32001 tokens), against the oracle.

The short-prompt vocabulary product stores four logits of a row as one 8-byte vector, so with such a vocabulary the
prompt step's logits take the tile GEMM instead, while the other products of the step stay on the streamed path;
the decode step's vocabulary GEMV and its arg max cover a last row that does not fill a unit. Reference path:
src/models/vkllm_models_llama2.c:488-602 (the output projection and arg max of the graph),
tests/vkllm_test_infer_gguf.c:181-272 (the loop). Bar: logits within 2e-2 of the oracle on every prompt row and
decode step; ids equal, except at a one-ulp tie in the oracle's logits.
"""
import numpy as np
import pytest

from helpers import assert_prefill_ids, fp16_ulp

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


@pytest.mark.parametrize("vocab", [1001, 1003, 32001])
def test_prompt_and_decode_with_a_vocabulary_not_a_multiple_of_4(ctx, vk, oracle, vocab):
    # dim 256 in heads of 64 and FFN 512 take the streamed short-prompt products
    shape = dict(n_layer=2, dim=256, n_head=4, ffn=512, vocab=vocab, ctx=128)
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=81)
    model = vk.Model(ctx, config=vk.llama_config(2, 256, 4, 512, vocab, 128), seed=81)
    try:
        prompt = oracle.prompt_tokens(82, 100, vocab)
        print(f"[vocab {vocab}] prompt of {len(prompt)} tokens", flush=True)
        want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
        ids = model.step(prompt, 0)
        logits = model.last_logits(len(prompt)).astype(np.float32)
        assert logits.shape == (len(prompt), vocab)
        err = float(np.max(np.abs(logits - want_logits.astype(np.float32))))
        print(f"[vocab {vocab}] prompt rows: max|dlogit| {err:.3g}", flush=True)
        assert err <= LOGIT_TOL
        assert assert_prefill_ids(ids, want_ids, want_logits, f"vocab {vocab}") <= 2
        tok, worst = int(want_ids[-1]), 0.0
        for pos in range(len(prompt), len(prompt) + 12):
            toks = np.array([tok], np.uint32)
            w_ids, w_logits, _ = ref.step(toks, pos, want_logits=True)
            g_ids = model.step(toks, pos)
            g_logits = model.last_logits(1).astype(np.float32)
            e = float(np.max(np.abs(g_logits - w_logits.astype(np.float32))))
            worst = max(worst, e)
            assert e <= LOGIT_TOL, f"vocab {vocab} position {pos}: max|dlogit| {e}"
            a, b = int(g_ids[0]), int(w_ids[0])
            if a != b:
                row = w_logits[0].astype(np.float32)
                assert row[b] - row[a] <= float(fp16_ulp(row[b])), f"vocab {vocab} position {pos}: id {a} vs {b}"
            tok = b
        print(f"[vocab {vocab}] decode: max|dlogit| {worst:.3g}", flush=True)
    finally:
        ref.close()
        model.close()
