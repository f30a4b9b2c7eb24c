"""Launch-ahead of single-token steps: after a decode step at position p the library enqueues the step at p + 1 with
the first step's device-side arg max as its token, before the host has read that id. A next call with that token at
p + 1 (the reference driver's greedy loop, tests/vkllm_test_infer_gguf.c:255-269) only waits for it; any other call
discards it. These tests drive both paths against the oracle, which simply runs the calls it is given, and check that
the switch VKLLM_LAUNCH_AHEAD=0 changes no result.
"""
import numpy as np
import pytest

from helpers import fp16_ulp

pytestmark = pytest.mark.gpu

SHAPE = dict(n_layer=4, dim=256, n_head=4, ffn=512, vocab=1000, ctx=96)


def _pair(oracle, vk, ctx, seed):
    cfg = oracle.make_cfg(**SHAPE)
    ref = oracle.Model(cfg=cfg, seed=seed)
    vcfg = vk.llama_config(SHAPE["n_layer"], SHAPE["dim"], SHAPE["n_head"], SHAPE["ffn"], SHAPE["vocab"],
                           SHAPE["ctx"])
    return cfg, ref, vk.Model(ctx, config=vcfg, seed=seed)


def _check(ref, model, toks, offset, what):
    toks = np.asarray(toks, np.uint32)
    want_ids, want_logits, _ = ref.step(toks, offset, want_logits=True)
    ids = model.step(toks, offset)
    logits = model.last_logits(len(toks)).astype(np.float32)
    err = float(np.max(np.abs(logits[-1] - want_logits[-1].astype(np.float32))))
    assert err <= 2e-2, f"{what}: max|dlogit| {err}"
    a, b = int(ids[-1]), int(want_ids[-1])
    if a != b:
        row = want_logits[-1].astype(np.float32)
        assert row[b] - row[a] <= float(fp16_ulp(row[b])), f"{what}: id {a} vs oracle {b}"
    return b


def test_calls_that_match_and_calls_that_do_not(ctx, vk, oracle):
    """Greedy steps (the step launched ahead is taken), a forced other token at the next position, a step repeated at
    the same position with another token, a jump back to an earlier position, and a prompt step in between: every
    step's logits and id against the oracle running the same calls."""
    cfg, ref, model = _pair(oracle, vk, ctx, seed=81)
    try:
        prompt = oracle.prompt_tokens(82, 10, cfg.vocab)
        nxt = _check(ref, model, prompt, 0, "prompt")
        pos = len(prompt)
        script = []
        for _ in range(6):  # greedy: each call matches the step launched ahead
            script.append(("greedy", None, pos))
            pos += 1
        script.append(("forced", 7, pos))              # another token at the launched-ahead position
        script.append(("greedy", None, pos + 1))
        script.append(("same position", 11, pos + 1))  # the position just computed, again, with another token
        script.append(("greedy", None, pos + 2))
        script.append(("jump back", 3, pos - 2))       # an earlier position
        script.append(("greedy", None, pos - 1))
        for what, tok, at in script:
            t = nxt if tok is None else tok
            print(f"[ahead] {what}: token {t} at {at}", flush=True)
            nxt = _check(ref, model, [t], at, what)
        # a prompt continuing the sequence, then greedy again
        cont = oracle.prompt_tokens(83, 5, cfg.vocab)
        nxt = _check(ref, model, cont, pos, "prompt continuation")
        for i in range(3):
            nxt = _check(ref, model, [nxt], pos + 5 + i, "greedy after the prompt")
    finally:
        ref.close()
        model.close()


def test_switch_changes_no_result(ctx, vk, oracle, monkeypatch):
    """The C token loop (the reference driver's loop) with launch-ahead on and off: identical ids and last logits
    (bit for bit), and the oracle's stream wherever the oracle's margin decides it."""
    cfg = oracle.make_cfg(**SHAPE)
    prompt = oracle.prompt_tokens(84, 12, cfg.vocab)
    ref = oracle.Model(cfg=cfg, seed=85)
    try:
        want_ids, want_logits = ref.token_loop(prompt, 40, want_logits=True)
    finally:
        ref.close()
    vcfg = vk.llama_config(SHAPE["n_layer"], SHAPE["dim"], SHAPE["n_head"], SHAPE["ffn"], SHAPE["vocab"],
                           SHAPE["ctx"])
    out = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("VKLLM_LAUNCH_AHEAD", flag)  # read when the model's first step sets up its state
        model = vk.Model(ctx, config=vcfg, seed=85)
        try:
            ids = model.loop(prompt, 40)[0]
            out[flag] = (ids, model.last_logits(1))
        finally:
            model.close()
    on, off = out["1"][0].tolist(), out["0"][0].tolist()
    assert on == off, f"launch-ahead on {on} / off {off}"
    assert np.array_equal(out["1"][1].view(np.uint16), out["0"][1].view(np.uint16))
    # against the oracle's free-running stream, up to its first step whose top-1/top-2 margin is within the 2e-2
    # logits tolerance (such a step is decided by summation order, and the streams may part there)
    for i, (a, b) in enumerate(zip(on, want_ids.tolist())):
        top2 = np.sort(want_logits[i].astype(np.float32))[-2:]
        if top2[1] - top2[0] <= 2e-2:
            print(f"step {i}: oracle margin {top2[1] - top2[0]:.4f}; streams compared up to it")
            break
        assert a == b, f"step {i}: id {a} vs oracle {b} at margin {top2[1] - top2[0]:.4f}"


def test_two_models_interleaved(ctx, vk, oracle):
    """Two models of different widths on one context, their greedy steps interleaved: each model's step launched
    ahead runs (stream order) while the other model's call is served, and is taken when its own next call matches.
    Every step of both against its own oracle."""
    cfg_a, ref_a, model_a = _pair(oracle, vk, ctx, seed=85)
    cfg_b = oracle.make_cfg(n_layer=2, dim=192, n_head=3, ffn=384, vocab=777, ctx=64)
    ref_b = oracle.Model(cfg=cfg_b, seed=86)
    model_b = vk.Model(ctx, config=vk.llama_config(2, 192, 3, 384, 777, 64), seed=86)
    try:
        nxt_a = _check(ref_a, model_a, oracle.prompt_tokens(87, 12, cfg_a.vocab), 0, "prompt a")
        nxt_b = _check(ref_b, model_b, oracle.prompt_tokens(88, 9, cfg_b.vocab), 0, "prompt b")
        pos_a, pos_b = 12, 9
        for i in range(10):
            nxt_a = _check(ref_a, model_a, [nxt_a], pos_a, f"a at {pos_a}")
            nxt_b = _check(ref_b, model_b, [nxt_b], pos_b, f"b at {pos_b}")
            pos_a, pos_b = pos_a + 1, pos_b + 1
            if i % 3 == 2:  # now and then two steps of one model in a row
                nxt_a = _check(ref_a, model_a, [nxt_a], pos_a, f"a again at {pos_a}")
                pos_a += 1
        print("[ahead] two models interleaved: every step matched its oracle", flush=True)
    finally:
        ref_a.close()
        ref_b.close()
        model_a.close()
        model_b.close()
