"""Parity at the lengths that define the long workloads, at a small width with the real head size (128):

* a 4096-position KV cache decoded from position 1000 through 4095, the LLaMA-2-7B long-context workload's cache
  (1024-token prompt, decode to 4096). Attention switches from the one-kernel short-cache path to the long-cache
  path at 1024 positions and then runs 16 chunks of 256 positions per head;
* a 2048-token prompt, the LLaMA-2-13B workload's prompt length, prefilled whole and in three chunks, then decoded.

Against the oracle (src/models/vkllm_llama2_layers.c:223-257 for the attention, tests/vkllm_test_infer_gguf.c:181-272
for the loop). Long decodes are teacher-forced: every step feeds the oracle's previous id, so one near-tie cannot
send the two streams apart for the rest of the run. Bar: logits within 2e-2 at every step; each step's id equal to
the oracle's, except where the oracle's logits of the two ids are within one fp16 ulp (fp32 summation order alone
decides such a tie; the count is printed and must stay under 1% of the steps).
"""
import numpy as np
import pytest

from helpers import assert_prefill_ids, fp16_ulp

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def _models(oracle, vk, ctx, shape, seed):
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=seed)
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    return cfg, ref, vk.Model(ctx, config=vcfg, seed=seed)


def _forced_decode(ref, model, first_tok, offset, n):
    """n single-token steps from position `offset`, each fed the oracle's previous id. Returns the worst logit
    difference and the number of steps whose ids differed at a one-ulp tie."""
    tok, worst, ties = int(first_tok), 0.0, 0
    for i in range(n):
        toks = np.array([tok], np.uint32)
        want_ids, want_logits, _ = ref.step(toks, offset + i, want_logits=True)
        ids = model.step(toks, offset + i)
        logits = model.last_logits(1)
        err = float(np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))))
        worst = max(worst, err)
        assert err <= LOGIT_TOL, f"position {offset + i}: max|dlogit| {err}"
        a, b = int(ids[0]), int(want_ids[0])
        if a != b:
            row = want_logits[0].astype(np.float32)
            assert row[b] - row[a] <= float(fp16_ulp(row[b])), \
                f"position {offset + i}: id {a} vs oracle {b}, not a one-ulp tie"
            ties += 1
        tok = b
    return worst, ties


def test_decode_through_4096_positions(ctx, vk, oracle):
    shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=4096)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=23)
    try:
        prompt = oracle.prompt_tokens(24, 1000, cfg.vocab)
        want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
        ids = model.step(prompt, 0)
        logits = model.last_logits(len(prompt))
        assert np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))) <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, "1000-token prompt")
        n = shape["ctx"] - len(prompt)
        print(f"[long] decoding positions {len(prompt)}..{shape['ctx'] - 1}", flush=True)
        worst, ties = _forced_decode(ref, model, want_ids[-1], len(prompt), n)
        print(f"[long] {n} steps: max|dlogit| {worst:.3g}, {ties} one-ulp ties")
        assert ties <= n // 100
    finally:
        ref.close()
        model.close()


@pytest.mark.parametrize("chunks", [[2048], [700, 900, 448]], ids=["whole", "chunked"])
def test_prompt_2048_tokens(ctx, vk, oracle, chunks):
    shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=2176)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=25)
    try:
        prompt = oracle.prompt_tokens(26, 2048, cfg.vocab)
        offset = 0
        for n in chunks:
            part = prompt[offset:offset + n]
            print(f"[prompt] rows {offset}..{offset + n - 1}", flush=True)
            want_ids, want_logits, _ = ref.step(part, offset, want_logits=True)
            ids = model.step(part, offset)
            logits = model.last_logits(n)
            err = float(np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))))
            print(f"[prompt] max|dlogit| {err:.3g}")
            assert err <= LOGIT_TOL
            assert_prefill_ids(ids, want_ids, want_logits, f"{n}-row chunk at {offset}")
            offset += n
        worst, ties = _forced_decode(ref, model, want_ids[-1], offset, 16)
        assert ties == 0
    finally:
        ref.close()
        model.close()


def test_long_cache_decode_at_7b_widths(ctx, vk, oracle):
    """The 7B widths (dim 4096, 32 heads of 128, FFN 11008; one layer, vocabulary 1000): a 1030-token prompt (256 x 256
    tiles with a ragged last row block, the down product split over K), then decode past the 1024-position
    switch-over on the one-launch long-cache attention (32 heads x 5 chunks, every chunk block resident) with the
    oracle's ids fed back."""
    shape = dict(n_layer=1, dim=4096, n_head=32, ffn=11008, vocab=1000, ctx=1100)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=51)
    try:
        prompt = oracle.prompt_tokens(52, 1030, cfg.vocab)
        want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
        ids = model.step(prompt, 0)
        err = float(np.max(np.abs(model.last_logits(len(prompt)).astype(np.float32) -
                                  want_logits.astype(np.float32))))
        print(f"[7b long] 1030-token prompt: max|dlogit| {err:.3g}", flush=True)
        assert err <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, "1030-token prompt")
        worst, ties = _forced_decode(ref, model, want_ids[-1], len(prompt), 6)
        print(f"[7b long] decode max|dlogit| {worst:.3g}, {ties} one-ulp ties")
        assert ties <= 1
    finally:
        ref.close()
        model.close()
