"""REF16: the oracle's restatement of the reference's fp16-arithmetic shader variants (src/shaders/BUILD:81,101,120,
140; selected by src/core/vkllm_op_matmul.c:92-101, vkllm_op_rope.c:22 and vkllm_op_softmax.c:24 when the device has
fp16 arithmetic), against values derived by hand from fp16 rounding, and the drift it measures between such a device
and the fp32-arithmetic variants the library follows.

Pins: the double -> fp16 rounding against numpy's own float64 -> float16 conversion; the GEMV's per-lane fp16
accumulation by its stagnation point (adding 4 to 8192 is a tie that rounds back to 8192); its fp16 scale and SiLU by
a hand-rounded chain; the GEMM's fp16 pair dot by a pair whose exact sum lies 3/4 ulp above 1; the softmax's fp16 sum
by 4096 equal scores (an fp16 sum of ones stops at 2048); RoPE's fp16 angle by position 2049 (rounds to 2048) and by
the rotation at angle 1 with fp16 cos and sin. The orders the Vulkan driver decides (subgroupAdd, dot()) are one
fixed choice each (oracle/oracle.h), so the model-level numbers are a measured drift, not parity.
"""
import numpy as np
import pytest


@pytest.fixture
def ref16(oracle):
    yield oracle
    oracle.set_numerics(False)


def f16(bits):
    return float(np.uint16(bits).view(np.float16))


def h(x):
    return np.float16(x).view(np.uint16)


def test_f64_to_f16_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    mags = np.exp2(rng.uniform(-27, 17, 20000))
    vals = np.concatenate([mags, -mags, [0.0, -0.0, 65504.0, 65519.99, 65520.0, 2.0**-24, 2.0**-25,
                                         2.0**-25 * (1 + 2.0**-40), 3 * 2.0**-26, 1 + 2.0**-11, 1 + 3 * 2.0**-11,
                                         np.inf, -np.inf]])
    # exact fp16 ties and neighbours of ties (double rounding through fp32 would get some of these wrong)
    ties = (np.arange(1, 2048, dtype=np.float64) + 0.5) * 2.0**-10
    vals = np.concatenate([vals, ties, ties * (1 + 2.0**-30), ties * (1 - 2.0**-30)])
    got = np.array([oracle.f64_to_f16_bits(v) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want), vals[got != want][:5]


def test_gemv16_accumulates_in_fp16(oracle):
    ones = h(np.ones(32768))
    # lane sums of 4096 dot4s of value 4: exact to 8192, where + 4 is a tie that rounds to the even 8192
    assert f16(oracle.gemv16(ones, ones, subgroup=2)) == 16384.0
    # eight lanes of 1024 dot4s: 4096 each, exact; their fp16 sum 32768
    assert f16(oracle.gemv16(ones, ones, subgroup=8)) == 32768.0
    # the fp32 variant: 32768 exactly, fp16 32768
    small = h(np.arange(64) % 3 - 1.0)
    ref = float(np.dot(h(np.arange(64) % 3 - 1.0).view(np.float16).astype(np.float64),
                       small.view(np.float16).astype(np.float64)))
    assert f16(oracle.gemv16(small, small, subgroup=8)) == ref  # small integers: every partial sum exact


def test_gemv16_scale_and_silu_in_fp16(oracle):
    x = h([1.0, 1.0, 1.0, 1.0])
    # 4 * fp16(0.5) = 2; exp(-2) -> fp16 0.1353759765625 (1109 * 2^-13); 1 + that -> 1.1357421875 (1163 / 1024);
    # 2 / 1.1357421875 = 1.76096... -> 1.7607421875 (1803 / 1024). The fp32 variant rounds silu(2) = 1.76159 once:
    # 1.76171875 (1804 / 1024).
    assert f16(oracle.gemv16(x, x, scale=0.5, act=1, subgroup=8)) == 1.7607421875


def test_gemm16_pair_dot(oracle):
    a = h([1.0, 1.0, 1.0, 1.0])
    b = h([1.0, 3 * 2.0**-12, 1.0, 3 * 2.0**-12])
    # each pair: 1 + 3 * 2^-12 is 3/4 of an ulp above 1 -> 1 + 2^-10; two pairs in fp32: 2.001953125 (exact sum
    # 2.00146484375)
    assert oracle.gemm16_dot(a, b) == 2.001953125
    # odd K pads the last pair with 0
    assert oracle.gemm16_dot(h([2.0, 3.0, 5.0]), h([1.0, 1.0, 1.0])) == 10.0


def test_softmax16(oracle):
    z = h(np.zeros(4096))
    # one lane: the fp16 sum of 4096 ones stops at 2048 (2048 + 1 is a tie to the even 2048)
    assert f16(oracle.softmax16_row(z, subgroup=1)[0]) == 2.0**-11
    # eight lanes of 512 ones: exact sums, 4096 in all
    assert f16(oracle.softmax16_row(z, subgroup=8)[0]) == 2.0**-12
    # masking: entries past the limit are 0 and out of the sum; the max still covers the whole row
    out = oracle.softmax16_row(h([0.0, 0.0, 0.0, 7.0, 7.0]), limit=2, subgroup=4)
    # max 7: exp(-7) -> fp16 0.0009117126 (3824 * 2^-22); sum of three -> 0.002735137939453125 (2868 * 2^-20);
    # quotient 0.3333 -> fp16(1/3) = 0.333251953125
    assert [f16(v) for v in out] == [0.333251953125] * 3 + [0.0, 0.0]


def test_rope16(oracle):
    v0, v1 = h(0.5), h(-0.25)
    assert oracle.rope16_pair(v0, v1, 0, 5, 128) == (v0, v1)  # angle 0
    # fp16(2049) = 2048
    assert oracle.rope16_pair(v0, v1, 2049, 7, 128) == oracle.rope16_pair(v0, v1, 2048, 7, 128)
    # w = 0: angle = position; cos 1 -> 0.54052734375 (1107 / 2048), sin 1 -> 0.84130859375 (1723 / 2048)
    o0, o1 = oracle.rope16_pair(h(1.0), h(0.0), 1, 0, 128)
    assert (f16(o0), f16(o1)) == (0.54052734375, 0.84130859375)


def test_mode_switch_restores_fp32(ref16):
    cfg = ref16.make_cfg(n_layer=2, dim=64, n_head=2, ffn=96, vocab=500, ctx=64)
    prompt = ref16.prompt_tokens(3, 9, cfg.vocab)
    m = ref16.Model(cfg=cfg, seed=4)
    try:
        a_ids, a_logits = m.token_loop(prompt, 6, want_logits=True)
        ref16.set_numerics(True, 8)
        m2 = ref16.Model(cfg=cfg, seed=4)
        b_ids, b_logits = m2.token_loop(prompt, 6, want_logits=True)
        m2.close()
        ref16.set_numerics(False)
        m3 = ref16.Model(cfg=cfg, seed=4)
        c_ids, c_logits = m3.token_loop(prompt, 6, want_logits=True)
        m3.close()
    finally:
        m.close()
    assert not np.array_equal(a_logits, b_logits)  # the fp16 variants change the numbers
    assert np.array_equal(a_logits, c_logits) and a_ids.tolist() == c_ids.tolist()


def _drift(oracle, cfg, seed, prompt_len, steps, subgroup):
    prompt = oracle.prompt_tokens(1, prompt_len, cfg.vocab)
    m = oracle.Model(cfg=cfg, seed=seed)
    ids32, lg32 = m.token_loop(prompt, steps, want_logits=True)
    m.close()
    oracle.set_numerics(True, subgroup)
    m = oracle.Model(cfg=cfg, seed=seed)
    ids16, lg16 = m.token_loop(prompt, steps, want_logits=True)
    m.close()
    oracle.set_numerics(False)
    # teacher-forced comparison is what the logits give while the streams agree; after the first different id the
    # two loops decode different texts
    first = next((i for i in range(steps) if ids32[i] != ids16[i]), steps)
    d = np.abs(lg32[:first].astype(np.float32) - lg16[:first].astype(np.float32)).max(axis=1) if first else [0.0]
    return first, float(np.max(d)), float(np.mean(d))


@pytest.mark.parametrize("subgroup", [8, 32])
def test_ref16_drift_tiny_workload(ref16, subgroup):
    """The tiny workload (dim 288, 6 layers, 6 heads of 48, vocab 32000), 16-token prompt, 64 greedy steps: how long
    the fp16-arithmetic variants keep the fp32 variants' token stream, and their logit distance until then."""
    cfg = ref16.make_cfg(n_layer=6, dim=288, n_head=6, ffn=768, vocab=32000, ctx=256)
    first, dmax, dmean = _drift(ref16, cfg, 7, 16, 64, subgroup)
    print(f"[REF16 subgroup {subgroup}] identical ids for {first} of 64 steps; max|dlogit| {dmax:.3g}, "
          f"mean {dmean:.3g} per step until then")
    assert first >= 1 and dmax > 0.0
