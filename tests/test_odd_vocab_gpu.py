"""Vocabularies whose size is not a multiple of 4 (LLaMA-2 variants ship 32001 tokens), against the oracle.

The short-prompt vocabulary product stores four logits of a row as one 8-byte vector, so with such a vocabulary the
prompt step's logits take the tile GEMM instead, while the other products of the step stay on the streamed path;
the decode step's vocabulary GEMV and its arg max cover a last row that does not fill a unit. Small vocabularies
(fewer rows than one wave takes) and vocabularies past 65536 ids are run as well. Reference path:
src/models/vkllm_models_llama2.c:488-602 (the output projection and arg max of the graph),
tests/vkllm_test_infer_gguf.c:181-272 (the loop). Bar: logits within 2e-2 of the oracle on every prompt row and
decode step; ids equal, except at a one-ulp tie in the oracle's logits.
"""
import pytest

from helpers import forced_decode, prompt_rows

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


# not multiples of 4, and the edges of the vocabulary GEMV and its arg max: a vocabulary smaller than one wave's rows
# (52, 50) and one past 65536 ids (70004, 70001)
@pytest.mark.parametrize("vocab", [1001, 1003, 32001, 52, 50, 70004, 70001])
def test_prompt_and_decode_at_vocabulary_edges(ctx, vk, oracle, vocab):
    # dim 256 in heads of 64 and FFN 512 take the streamed short-prompt products
    shape = dict(n_layer=2, dim=256, n_head=4, ffn=512, vocab=vocab, ctx=128)
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=81)
    model = vk.Model(ctx, config=vk.llama_config(2, 256, 4, 512, vocab, 128), seed=81)
    try:
        prompt = oracle.prompt_tokens(82, 100, vocab)
        want_ids, ties = prompt_rows(ref, model, prompt, 0, f"vocab {vocab}", LOGIT_TOL)
        assert model.last_logits(len(prompt)).shape == (len(prompt), vocab)
        assert ties <= 2
        _, ties, _ = forced_decode(ref, model, want_ids[-1], len(prompt), 12, f"vocab {vocab}", LOGIT_TOL)
        assert ties <= 1
    finally:
        ref.close()
        model.close()
