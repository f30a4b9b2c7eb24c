"""Model geometries and prompt lengths that select different kernel paths, each against the oracle.

Each case builds a small random-init model on both sides (seeded, identical weights), runs its prompt as one or more
prompt steps (every row's logits compared), then teacher-forced decode steps. The cases cover the switches of the
token step (src/models/vkllm_llama2_layers.c:98-354 and the loop of tests/vkllm_test_infer_gguf.c:181-272 restated
in vkllm.c_amd/csrc/fused.cpp):
  * prompt length: one token (the decode kernels at position 0), two tokens, up to 32 tokens (the streamed QKV
    product split over K with the RoPE reduce), 33-128 tokens (the QKV product split over tokens), 129 tokens (the
    tile GEMMs), and prompts in chunks at nonzero offsets;
  * head size 8, 16, 32, 48 (no RoPE epilogue, no streamed products), 64, 128 and 256 (the transposed P.V when the
    cache holds exactly head_dim positions, in a prompt step and in a decode step), and head counts that are not
    multiples of 8; head size 256 past the short-cache bound (768 positions there) takes the two-kernel attention;
  * FFN widths that are multiples of 32, of 16 only (no fused SwiGLU epilogue on the tile GEMM), of 8 only (no
    streamed products), and of 4 only (node-by-node execution through the VKLLM_OP_* kernels);
  * vocabularies that are not multiples of 4.
Bar: logits within 2e-2 of the oracle on every prompt row and decode step (two layers, fp16 weights, fp32 sums);
ids equal, except at a one-ulp tie in the oracle's logits (fp32 summation order alone decides such a row). Node-by-
node execution exposes only the graph's output (the arg-max ids), so that case compares ids.
"""
import numpy as np
import pytest

from helpers import assert_prefill_ids, forced_decode, fp16_ulp, prompt_rows

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def _shape(dim, n_head, ffn, vocab=1000, ctx=160, n_layer=2):
    return dict(n_layer=n_layer, dim=dim, n_head=n_head, ffn=ffn, vocab=vocab, ctx=ctx)


# id: (shape, prompt chunks, decode steps)
CASES = {
    "hd64-prompt1": (_shape(256, 4, 512), [1], 6),
    "hd64-prompt2": (_shape(256, 4, 512), [2], 6),
    "hd64-prompt31": (_shape(256, 4, 512), [31], 4),
    "hd64-prompt32": (_shape(256, 4, 512), [32], 4),
    "hd64-prompt33": (_shape(256, 4, 512), [33], 4),
    "hd64-prompt128": (_shape(256, 4, 512), [128], 4),
    "hd64-prompt129": (_shape(256, 4, 512), [129], 4),
    "hd64-chunks40-50-60": (_shape(256, 4, 512), [40, 50, 60], 4),
    "hd64-3heads-vocab777": (_shape(192, 3, 384, vocab=777), [70], 6),
    "hd64-5heads": (_shape(320, 5, 640), [100], 4),
    "hd32-3heads": (_shape(96, 3, 256, vocab=500), [40], 6),
    "hd48-6heads": (_shape(288, 6, 768), [20], 6),
    "hd128-3heads-through-kv128": (_shape(384, 3, 1024), [50], 90),
    # head_dim 256: a first prompt of exactly 256 positions (the transposed P.V in the prompt step), a second chunk at
    # offset 256, then decode past the short-cache bound of 768 positions on the two-kernel attention
    "hd256-2heads-past-768": (_shape(512, 2, 1024, ctx=800), [256, 504], 20),
    # head_dim 16 and 8: decode through kv == head_dim, and a prompt of exactly head_dim positions
    "hd16-4heads-through-kv16": (_shape(64, 4, 128, vocab=300), [10], 12),
    "hd8-8heads-prompt8": (_shape(64, 8, 128, vocab=300), [8], 6),
    "ffn528-prompt60": (_shape(256, 4, 528), [60], 4),
    "ffn528-prompt150": (_shape(256, 4, 528), [150], 4),
    "ffn520-prompt60": (_shape(256, 4, 520), [60], 4),
    "ffn516-nodes": (_shape(256, 4, 516), [30], 4),
}
# node-by-node execution (an FFN width that is not a multiple of 8 leaves the fused step): ids only
IDS_ONLY = {"ffn516-nodes"}


def _ids_only(ref, model, prompt, n_decode, what):
    want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
    assert assert_prefill_ids(model.step(prompt, 0), want_ids, want_logits, what) <= 2
    tok = int(want_ids[-1])
    for pos in range(len(prompt), len(prompt) + n_decode):
        toks = np.array([tok], np.uint32)
        w_ids, w_logits, _ = ref.step(toks, pos, want_logits=True)
        a, b = int(model.step(toks, pos)[0]), int(w_ids[0])
        if a != b:
            row = w_logits[0].astype(np.float32)
            assert row[b] - row[a] <= float(fp16_ulp(row[b])), f"{what} position {pos}: id {a} vs {b}"
        tok = b
    print(f"[{what}] ids of {len(prompt)} prompt rows and {n_decode} decode steps checked", flush=True)


@pytest.mark.parametrize("name", sorted(CASES))
def test_shape_against_oracle(ctx, vk, oracle, name):
    shape, chunks, n_decode = CASES[name]
    assert sum(chunks) + n_decode <= shape["ctx"]
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=91)
    model = vk.Model(ctx, config=vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"],
                                                 shape["vocab"], shape["ctx"]), seed=91)
    try:
        prompt = oracle.prompt_tokens(92, sum(chunks), shape["vocab"])
        if name in IDS_ONLY:
            _ids_only(ref, model, prompt, n_decode, name)
            return
        offset, ties = 0, 0
        for n in chunks:
            want_ids, t = prompt_rows(ref, model, prompt[offset:offset + n], offset, name, LOGIT_TOL)
            ties += t
            offset += n
        assert ties <= 2
        _, t, _ = forced_decode(ref, model, want_ids[-1], offset, n_decode, name, LOGIT_TOL)
        assert t <= 1
    finally:
        ref.close()
        model.close()


def test_decode_to_the_last_cache_position_then_past_it(ctx, vk, oracle):
    """Decode up to the cache's last position (no step is launched ahead past it) against the oracle; a step at the
    position after it, or a prompt that would run past it, is refused with VKLLM_ERR_ARGS and leaves the model usable
    (the reference's build_graph bounds the cache view the same way, src/models/vkllm_kvcache.c:12-124)."""
    shape = _shape(256, 4, 512, ctx=48)
    ref = oracle.Model(cfg=oracle.make_cfg(**shape), seed=93)
    model = vk.Model(ctx, config=vk.llama_config(2, 256, 4, 512, 1000, 48), seed=93)
    try:
        prompt = oracle.prompt_tokens(94, 20, 1000)
        want_ids, _ = prompt_rows(ref, model, prompt, 0, "to ctx", LOGIT_TOL)
        _, _, tok = forced_decode(ref, model, want_ids[-1], 20, 28, "to ctx", LOGIT_TOL)  # positions 20..47
        for toks, at in (([tok], 48), ([tok, tok], 47), ([1] * 30, 20)):
            with pytest.raises(vk.VkllmError) as e:
                model.step(np.array(toks, np.uint32), at)
            assert e.value.code == vk.ERR_ARGS, e.value
        # still usable: the last position again, as the oracle computes it
        forced_decode(ref, model, tok, 47, 1, "to ctx again", LOGIT_TOL)
    finally:
        ref.close()
        model.close()
