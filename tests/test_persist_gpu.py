"""The persistent single-token step: every layer's products, the attention and the vocabulary product with its arg max
in one launch, phases separated by grid barriers (VKLLM_PERSIST=1, for short caches; by default the separate decode
kernels run). Reference path: src/models/vkllm_llama2_layers.c:98-354 (the layer),
src/models/vkllm_models_llama2.c:560-602 (output norm, logits, arg max), tests/vkllm_test_infer_gguf.c:181-272 (the
loop).

Each case runs the same calls on the oracle: a prompt, then teacher-forced single-token steps through a bucket edge
(64 / 65 or 128 / 129 positions) and kv == head_dim (the transposed P.V) and, for the small shape, through the last
short-cache positions into the long-cache path. Bar as for every decode step: logits within 2e-2 of the oracle, ids
equal except at a one-ulp tie in the oracle's logits. That the steps ran as the persistent launch is checked through
its timing family, which only accepts a last step that did.
"""
import numpy as np
import pytest

from helpers import fp16_ulp

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2

# name: shape, prompt length, decode steps after the prompt, positions of further single steps (prompted up to them)
CASES = {
    "small": (dict(n_layer=3, dim=256, n_head=4, ffn=512, vocab=1000, ctx=1100), 60, 8, [(1018, 9)]),
    "small_ffn1024": (dict(n_layer=2, dim=512, n_head=8, ffn=1024, vocab=1000, ctx=160), 60, 8, []),
    "7b": (dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=1000, ctx=256), 120, 12, []),
    "13b": (dict(n_layer=1, dim=5120, n_head=40, ffn=13824, vocab=1000, ctx=256), 120, 12, []),
}


def _step(ref, model, toks, offset, what):
    toks = np.asarray(toks, np.uint32)
    want_ids, want_logits, _ = ref.step(toks, offset, want_logits=True)
    ids = model.step(toks, offset)
    logits = model.last_logits(len(toks)).astype(np.float32)
    err = float(np.max(np.abs(logits - want_logits.astype(np.float32))))
    assert err <= LOGIT_TOL, f"{what} at {offset}: max|dlogit| {err}"
    a, b = int(ids[-1]), int(want_ids[-1])
    if a != b:
        row = want_logits[-1].astype(np.float32)
        assert row[b] - row[a] <= float(fp16_ulp(row[b])), f"{what} at {offset}: id {a} vs oracle {b}"
    return b, err


def _decode(ref, model, tok, offset, n, what):
    worst = 0.0
    for i in range(n):
        tok, err = _step(ref, model, [tok], offset + i, what)
        worst = max(worst, err)
    print(f"[{what}] decode {offset}..{offset + n - 1}: max|dlogit| {worst:.3g}", flush=True)
    return tok


def _persistent(model):
    """True when the model's last single-token step ran as the persistent launch (its timing family accepts it)."""
    try:
        model.time_kernel("decode_persist", 1)
        return True
    except RuntimeError:
        return False


@pytest.fixture(autouse=True)
def persistent(monkeypatch):
    monkeypatch.setenv("VKLLM_PERSIST", "1")  # read when a model's first step sets up its state


@pytest.mark.parametrize("name", list(CASES))
def test_persistent_step_against_oracle(ctx, vk, oracle, name):
    shape, prompt_len, n_dec, later = CASES[name]
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=101)
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=101)
    hd = shape["dim"] // shape["n_head"]
    try:
        print(f"[{name}] start", flush=True)
        tok, _ = _step(ref, model, oracle.prompt_tokens(102, prompt_len, cfg.vocab), 0, name + " prompt")
        tok = _decode(ref, model, tok, prompt_len, n_dec, name)  # across the 64-position bucket edges
        assert _persistent(model), f"{name}: the last step did not run as the persistent launch"
        pos = prompt_len + n_dec
        assert prompt_len <= hd - 1 < pos  # the decode steps pass kv == head_dim
        for at, n in later:
            tok, _ = _step(ref, model, oracle.prompt_tokens(104, at - pos, cfg.vocab), pos, name + " prompt")
            # the last short-cache buckets (kv up to 1024), then the long-cache path (separate kernels)
            tok = _decode(ref, model, tok, at, n, name + " to the long-cache path")
            assert not _persistent(model), f"{name}: kv {at + n} should take the long-cache kernels"
            pos = at + n
    finally:
        ref.close()
        model.close()


def test_switch_changes_no_id(ctx, vk, oracle, monkeypatch):
    """The C token loop at the 7B widths (2 layers, vocabulary 32000) with the persistent step on and off
    (VKLLM_PERSIST=0): logits within 2e-2 of each other and of the oracle, and the oracle's ids. (The two are not
    bit-identical: the persistent step's attention sums P.V over 16 dim slices of 256 threads per head, the separate
    kernel over 8 of 512.)"""
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=96)
    cfg = oracle.make_cfg(**shape)
    prompt = oracle.prompt_tokens(105, 16, cfg.vocab)
    ref = oracle.Model(cfg=cfg, seed=106)
    try:
        want_ids, want_logits = ref.token_loop(prompt, 24, want_logits=True)
    finally:
        ref.close()
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    out = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("VKLLM_PERSIST", flag)
        model = vk.Model(ctx, config=vcfg, seed=106)
        try:
            out[flag] = model.token_loop(prompt, 24, want_logits=True)
            assert _persistent(model) == (flag == "1")
        finally:
            model.close()
    (ids_on, lg_on), (ids_off, lg_off) = out["1"], out["0"]
    d_on = float(np.max(np.abs(lg_on.astype(np.float32) - want_logits.astype(np.float32))))
    d_off = float(np.max(np.abs(lg_off.astype(np.float32) - want_logits.astype(np.float32))))
    d_pair = float(np.max(np.abs(lg_on.astype(np.float32) - lg_off.astype(np.float32))))
    print(f"max|dlogit| persistent {d_on:.3g}, separate {d_off:.3g}, between them {d_pair:.3g}")
    assert max(d_on, d_off, d_pair) <= LOGIT_TOL
    # ids: equal to the oracle's stream up to its first step whose top-1/top-2 margin is within the 2e-2 logits
    # tolerance (summation order decides such a step, and the streams may part there)
    for i, (a, b, c) in enumerate(zip(ids_on.tolist(), ids_off.tolist(), want_ids.tolist())):
        top2 = np.sort(want_logits[i].astype(np.float32))[-2:]
        if top2[1] - top2[0] <= LOGIT_TOL:
            print(f"step {i}: oracle margin {top2[1] - top2[0]:.4f}; streams compared up to it")
            break
        assert a == b == c, f"step {i}: persistent {a}, separate {b}, oracle {c}"


def test_arg_max_ties(ctx, vk, monkeypatch):
    """The persistent step's arg max (each workgroup publishes its best, the last to finish reduces them) under the
    reference's tie rule (src/shaders/vkllm_arg_max.comp:40-97): output weights zero except rows +u at 5, 37, 70,
    12345, 31999 and -u at 3, 35, 99, 20000, 31998, so five rows tie for the maximum; the rule picks 70 or 20000."""
    from helpers import argmax_tie_rule

    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160)
    prompt = vk.prompt_tokens(11, 20, shape["vocab"])
    plus, minus = [5, 37, 70, 12345, 31999], [3, 35, 99, 20000, 31998]
    w = np.zeros((shape["vocab"], shape["dim"]), np.float16)
    w[plus] = 0.01
    w[minus] = -0.01
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=7)
    try:
        ctx.upload(model.m.weights.output_weight, w)
        ids, logits = model.token_loop(prompt, 6, want_logits=True)
        assert _persistent(model)
    finally:
        model.close()
    for step in range(1, 6):
        row = logits[step].astype(np.float32)
        tied = np.nonzero(row == row.max())[0].tolist()
        assert tied in (plus, minus), tied
        assert int(ids[step]) == argmax_tie_rule(row) and int(ids[step]) in (70, 20000)
