"""Every VKLLM_* execution switch of the fused token step, each against the oracle (not against another path of this
library): with the switch set when the model's step state is made, a prompt in three chunks (two of the streamed
short-prompt products, one of 130 tokens on the tile GEMMs, at nonzero offsets), then 100 teacher-forced decode steps
that run past a short-cache bound of 64 positions, so that the long-cache attention (in one launch or two, over
several chunks of the 600-position cache) is reached where a switch moves the switch-over there.

Switches (read in vkllm.c_amd/csrc/fused.cpp): RoPE and the K/V append in a separate pass (VKLLM_ROPE_EPI=0), the
RMSNorm as its own pass (VKLLM_NORM_EPI=0), prompt steps on the tile GEMMs only (VKLLM_PREFILL_TILED=0), the arg max
as its own kernel (VKLLM_ARGMAX_EPI=0), 4 or 2 decode-attention blocks per head (VKLLM_ATTN_GROUPS), no launch-ahead
(VKLLM_LAUNCH_AHEAD=0), attention and the output projection in one launch (VKLLM_ATTN_O=1), the attention in the
QKV product's launch (VKLLM_QKV_ATTN=1), the persistent single-token step (VKLLM_PERSIST=1), and the long-cache
attention from position 64 in one launch or in two (VKLLM_ATTN_SMALL_MAX=64, VKLLM_ATTN_LONG=0).
Reference path: src/models/vkllm_llama2_layers.c:98-354, tests/vkllm_test_infer_gguf.c:181-272. Bar: logits within
2e-2 of the oracle on every prompt row and decode step (two layers); ids equal except at one-ulp ties.
"""
import pytest

from helpers import forced_decode, prompt_rows

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
SHAPE = dict(n_layer=2, dim=256, n_head=4, ffn=512, vocab=1000, ctx=600)
CHUNKS = [60, 90, 130]
N_DECODE = 100

SWITCHES = {
    "rope-pass": {"VKLLM_ROPE_EPI": "0"},
    "norm-pass": {"VKLLM_NORM_EPI": "0"},
    "tiled-prefill": {"VKLLM_PREFILL_TILED": "0"},
    "argmax-kernel": {"VKLLM_ARGMAX_EPI": "0"},
    "attn-groups-4": {"VKLLM_ATTN_GROUPS": "4"},
    "attn-groups-2": {"VKLLM_ATTN_GROUPS": "2"},
    "no-launch-ahead": {"VKLLM_LAUNCH_AHEAD": "0"},
    "attn-o": {"VKLLM_ATTN_O": "1"},
    "qkv-attn": {"VKLLM_QKV_ATTN": "1"},
    "persist": {"VKLLM_PERSIST": "1"},
    "long-from-64": {"VKLLM_ATTN_SMALL_MAX": "64"},
    "long-from-64-two-kernels": {"VKLLM_ATTN_SMALL_MAX": "64", "VKLLM_ATTN_LONG": "0"},
}


@pytest.mark.parametrize("name", sorted(SWITCHES))
def test_switch_against_oracle(ctx, vk, oracle, monkeypatch, name):
    for k, v in SWITCHES[name].items():
        monkeypatch.setenv(k, v)
    ref = oracle.Model(cfg=oracle.make_cfg(**SHAPE), seed=95)
    model = vk.Model(ctx, config=vk.llama_config(SHAPE["n_layer"], SHAPE["dim"], SHAPE["n_head"], SHAPE["ffn"],
                                                 SHAPE["vocab"], SHAPE["ctx"]), seed=95)
    try:
        prompt = oracle.prompt_tokens(96, sum(CHUNKS), SHAPE["vocab"])
        offset, ties = 0, 0
        for n in CHUNKS:
            want_ids, t = prompt_rows(ref, model, prompt[offset:offset + n], offset, name, LOGIT_TOL)
            ties += t
            offset += n
        assert ties <= 3
        _, t, _ = forced_decode(ref, model, want_ids[-1], offset, N_DECODE, name, LOGIT_TOL)
        assert t <= 1
    finally:
        ref.close()
        model.close()
