"""The C token loop that bench.py times (vkllm_hip_token_loop, the reference driver's loop of
tests/vkllm_test_infer_gguf.c:181-272 in C) against the oracle and the committed fixture, and the decode step's
recovery when a bounded wait between workgroups gives up.

Bar: identical greedy ids; logits within 2e-2 where they are compared.
"""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LOGIT_TOL = 2e-2


def test_c_token_loop_matches_oracle_and_fixture(ctx, vk, oracle, tiny_gguf):
    """The tiny workload (16-token prompt from seed 1, 64 greedy steps) through vkllm_hip_token_loop."""
    with open(os.path.join(GOLDEN, "tiny_token_loop.json")) as f:
        want = json.load(f)
    ref = oracle.Model(tiny_gguf)
    try:
        want_ids, _ = ref.token_loop(np.array(want["prompt"], np.uint32), len(want["ids"]))
    finally:
        ref.close()
    assert want_ids.tolist() == want["ids"]
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        ids, step_ns, phase_ns = model.loop(np.array(want["prompt"], np.uint32), len(want["ids"]))
    finally:
        model.close()
    assert ids.tolist() == want["ids"]
    assert np.all(step_ns > 0) and np.all(phase_ns > 0)


def test_c_token_loop_from_nonzero_offset(ctx, vk, oracle):
    """A first prompt prefilled at offset 0, then the C loop started at offset0 = its length with a second prompt:
    the loop's positions continue the cache. Against the oracle's chained steps."""
    shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=256)
    cfg = oracle.make_cfg(**shape)
    first = oracle.prompt_tokens(31, 40, cfg.vocab)
    second = oracle.prompt_tokens(32, 9, cfg.vocab)
    n = 30
    ref = oracle.Model(cfg=cfg, seed=17)
    try:
        ref.step(first, 0)
        toks, offset, want = second, len(first), []
        for _ in range(n):
            out, _, _ = ref.step(toks, offset)
            want.append(int(out[-1]))
            offset += len(toks)
            toks = np.array([want[-1]], np.uint32)
    finally:
        ref.close()
    model = vk.Model(ctx, config=vk.llama_config(**_vk_shape(shape)), seed=17)
    try:
        model.step(first, 0)
        ids, _, _ = model.loop(second, n, offset=len(first))
    finally:
        model.close()
    assert ids.tolist() == want


def _vk_shape(shape):
    return dict(n_layer=shape["n_layer"], dim=shape["dim"], n_head=shape["n_head"], ffn=shape["ffn"],
                vocab=shape["vocab"], ctx=shape["ctx"])


@pytest.mark.parametrize("path", ["long", "attn_o", "persist"])
def test_decode_recovers_when_a_wait_gives_up(ctx, vk, oracle, monkeypatch, capfd, path):
    """VKLLM_SPIN_LIMIT=0 makes every bounded wait give up at once, without polling, so each kernel still exits
    normally: the one-kernel long-cache attention (1100-token prompt, chunks of 256 positions), the attention +
    Wo launch (VKLLM_ATTN_O=1, a short cache) or the persistent step's grid barriers (VKLLM_PERSIST=1, a short
    cache). The step must notice, clear the counters, switch to the kernels that never wait and run again: ids equal
    to the oracle's, logits within 2e-2, and every later step on the waiting-free path."""
    monkeypatch.setenv("VKLLM_SPIN_LIMIT", "0")
    if path in ("attn_o", "persist"):
        monkeypatch.setenv("VKLLM_PERSIST", "1" if path == "persist" else "0")
        if path == "attn_o":
            monkeypatch.setenv("VKLLM_ATTN_O", "1")
        shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=96)
        prompt_len = 20
    else:
        shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=2048)
        prompt_len = 1100
    cfg = oracle.make_cfg(**shape)
    prompt = oracle.prompt_tokens(33, prompt_len, cfg.vocab)
    ref = oracle.Model(cfg=cfg, seed=19)
    try:
        want_ids, want_logits = ref.token_loop(prompt, 6, want_logits=True)
    finally:
        ref.close()
    model = vk.Model(ctx, config=vk.llama_config(**_vk_shape(shape)), seed=19)
    try:
        ids, logits = model.token_loop(prompt, 6, want_logits=True)
    finally:
        model.close()
    log = capfd.readouterr().err
    err = float(np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))))
    print(f"[{path}] max|dlogit| {err:.3g}")
    # the first decode step's waits gave up once; the rerun and every later step used kernels that do not wait
    assert log.count("gave up") == 1, log
    assert ids.tolist() == want_ids.tolist()
    assert err <= LOGIT_TOL
