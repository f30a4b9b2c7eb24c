"""Single-token attention at the end of the QKV product's launch (VKLLM_QKV_ATTN=1; off by default). For caches of at
most 512 positions the decode step then runs no separate attention kernel: the workgroup that completes a head's q, k
and v rows (counted per head across the launch) computes that head's attention
(src/models/vkllm_llama2_layers.c:223-257 with src/shaders/vkllm_softmax.comp:42-96), including the reference's
transposed P.V at kv == head_dim. Longer caches go back to the separate kernels. VKLLM_QKV_ATTN=0 (the default) keeps
the separate kernel everywhere.

Each case runs the same calls on the oracle: prompts and teacher-forced decode steps across kv == head_dim and across
kv 512 -> 513, then a few steps with per-launch timing on, whose kernel counts show which path ran. Bar as for every
decode step: logits within 2e-2 of the oracle, ids equal except at a one-ulp tie of the oracle's logits.
"""
import numpy as np
import pytest

from helpers import fp16_ulp

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
SHAPES = {
    "hd32": dict(n_layer=2, dim=256, n_head=8, ffn=512, vocab=1000, ctx=544),
    "hd128": dict(n_layer=2, dim=512, n_head=4, ffn=1024, vocab=1000, ctx=544),
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


@pytest.mark.parametrize("tail", ["1", "0"])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_decode_attention_in_qkv_launch(ctx, vk, oracle, monkeypatch, name, tail):
    shape = SHAPES[name]
    hd = shape["dim"] // shape["n_head"]
    monkeypatch.setenv("VKLLM_QKV_ATTN", tail)  # read when the model's first step sets up its state
    monkeypatch.setenv("VKLLM_PERSIST", "0")  # the separate decode kernels
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=91)
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=91)
    what = f"{name} tail={tail}"
    try:
        print(f"[{what}] start", flush=True)
        tok, _ = _step(ref, model, oracle.prompt_tokens(92, 28, cfg.vocab), 0, what + " prompt")
        tok = _decode(ref, model, tok, 28, 7, what)          # kv 29..35: kv == 32 == head_dim of hd32
        tok, _ = _step(ref, model, oracle.prompt_tokens(93, 90, cfg.vocab), 35, what + " prompt")
        tok = _decode(ref, model, tok, 125, 7, what)         # kv 126..132: kv == 128 == head_dim of hd128
        tok, _ = _step(ref, model, oracle.prompt_tokens(94, 375, cfg.vocab), 132, what + " prompt")
        tok = _decode(ref, model, tok, 507, 10, what)        # kv 508..517: the last short-cache positions and past
        # per-launch timing: which attention kernels the steps launched
        ctx.set_timing(True)
        try:
            ctx.reset_kernel_stats()
            _decode(ref, model, tok, 517, 2, what + " timed, kv > 512")
            long_stats = ctx.kernel_stats()
            ctx.reset_kernel_stats()
            _decode(ref, model, 5, hd - 1, 2, what + " timed, kv == head_dim")  # back to earlier positions
            _decode(ref, model, 9, 300, 2, what + " timed, kv 301")
            short_stats = ctx.kernel_stats()
        finally:
            ctx.set_timing(False)
        n = lambda st, k: st.get(k, (0, 0))[0]
        print(f"[{what}] attention launches kv > 512: {n(long_stats, 'fused_attn_small')}, kv <= 512: "
              f"{n(short_stats, 'fused_attn_small')}", flush=True)
        L = shape["n_layer"]
        assert n(long_stats, "fused_attn_small") == 2 * L
        assert n(short_stats, "fused_qkv_rope") == 4 * L
        assert n(short_stats, "fused_attn_small") == (0 if tail == "1" else 4 * L)
    finally:
        ref.close()
        model.close()
