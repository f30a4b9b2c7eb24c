"""The short-prompt product of the fused step (vkllm_hip_gemm_streamed): weights read from the fragment-tiled copy
and streamed into the matrix cores, the activations fragment-ordered, against a float32 product of the same fp16
operands (the bar of tests/test_gemm_gpu.py: the fp16 rounding of an fp32 sum, |C - ref| <= 1e-3 + 2e-3 |ref|, twice
that for the residual and SwiGLU epilogues, which round twice).

The fused step runs the QKV (split K, then the RoPE reduce), output (split K, then the residual + RMSNorm reduce),
gate/up (SwiGLU) and vocabulary products of prompts of at most 128 tokens on this kernel (src/core/vkllm_op_matmul.c
replaced for those nodes). The cases reach the LLaMA-2-7B and 13B shapes at 128 tokens, 1 to 4 token blocks with a
partial last block, K ranges ending in a partial LDS chunk (K not a multiple of 128), split K with a one-step last
range, row counts that are not a multiple of 32 (zero rows in the tiled copy) and workgroups whose last waves have
no row block.
"""
import ctypes

import numpy as np
import pytest

from test_gemm_gpu import PLAIN, RESID, SWIGLU, reference

pytestmark = pytest.mark.gpu

# (M, N, K, epi, splits): N is the product's rows (2F for the SwiGLU epilogue)
CASES = [
    (128, 12288, 4096, RESID, 0),   # 7B [Wq; Wk; Wv] at 128 tokens: 96 workgroups, K split in 2
    (128, 12288, 4096, RESID, 1),   # the same unsplit
    (128, 4096, 4096, RESID, 0),    # 7B Wo: 32 workgroups, K split in 8
    (128, 22016, 4096, SWIGLU, 0),  # 7B [Wu; Wg]: three compute waves, 230 workgroups
    (128, 27648, 5120, SWIGLU, 0),  # 13B [Wu; Wg]: four compute waves (288 workgroups of three would not fit)
    (128, 32000, 4096, PLAIN, 0),   # vocabulary product
    (128, 15360, 5120, RESID, 0),   # 13B [Wq; Wk; Wv]
    (1, 4096, 4096, PLAIN, 0),      # one token
    (31, 1000, 288, PLAIN, 0),      # N % 32 != 0; K = 18 steps: two chunks and a 2-step chunk
    (33, 3072, 272, RESID, 3),      # two token blocks; 17 steps in ranges of 8, 8 and 1
    (64, 1536, 4096, SWIGLU, 0),    # two token blocks, 48 row blocks
    (65, 2048, 2048, RESID, 8),     # three token blocks, 8 ranges of 16 steps
    (96, 1024, 1040, PLAIN, 0),     # 65 steps: 8 chunks and a 1-step chunk
    (100, 32000, 512, PLAIN, 0),    # ragged M, K of 32 steps: the weight ring's tail only
    (127, 288, 4096, PLAIN, 0),     # 9 row blocks: the last workgroup has one live compute wave
    (128, 96, 128, SWIGLU, 0),      # F = 48: three row blocks, one chunk
    (128, 64, 16, PLAIN, 0),        # one K step
]


def run_streamed(ctx, vk, a, b, c0, epi, splits):
    M, K = a.shape
    N = b.shape[0]
    ldc = c0.shape[1]
    ta = ctx.tensor_from(a, name="A")
    tb = ctx.tensor_from(b, name="B")
    tc = ctx.tensor_from(c0, name="C")
    try:
        dev = [t.contents.data.dev for t in (ta, tb, tc)]
        rc = vk.lib().vkllm_hip_gemm_streamed(ctx.vp, epi, dev[0], dev[1], dev[2], M, N, K, ldc, splits)
        vk.check("vkllm_hip_gemm_streamed", rc)
        return ctx.download(tc).reshape(M, ldc)
    finally:
        for t in (ta, tb, tc):
            ctx.free(t)


def _operands(M, N, K, epi, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    b = (rng.standard_normal((N, K), dtype=np.float32) * (1.0 / np.sqrt(K))).astype(np.float16)
    width = N // 2 if epi == SWIGLU else N
    c0 = rng.standard_normal((M, width), dtype=np.float32).astype(np.float16) if epi == RESID else \
        np.zeros((M, width), np.float16)
    return a, b, c0


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}-e{c[3]}-s{c[4]}")
def test_streamed_gemm(ctx, vk, case):
    M, N, K, epi, splits = case
    print(f"[stream gemm] M={M} N={N} K={K} epi={epi} splits={splits}", flush=True)
    a, b, c0 = _operands(M, N, K, epi, M * 7 + N * 3 + K + epi)
    got = run_streamed(ctx, vk, a, b, c0, epi, splits).astype(np.float32)
    ref = reference(a, b, c0, epi, N // 2 if epi == SWIGLU else 0)
    tol = (1e-3 + 2e-3 * np.abs(ref)) * (2.0 if epi in (RESID, SWIGLU) else 1.0)
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} outside tolerance; worst at "
                           f"{np.unravel_index(np.argmax(err - tol), err.shape)}: got "
                           f"{got.flat[np.argmax(err - tol)]} ref {ref.flat[np.argmax(err - tol)]}")


def test_streamed_gemm_is_deterministic(ctx, vk):
    """Fixed split ranges added in order by the reduce: repeated calls give identical bits."""
    a, b, c0 = _operands(128, 4096, 4096, RESID, 11)
    first = run_streamed(ctx, vk, a, b, c0, RESID, 0)
    second = run_streamed(ctx, vk, a, b, c0, RESID, 0)
    assert np.array_equal(first.view(np.uint16), second.view(np.uint16))


def test_streamed_gemm_rejects_bad_arguments(ctx, vk):
    L = vk.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the argument checks fail first
    assert L.vkllm_hip_gemm_streamed(ctx.vp, PLAIN, p, p, p, 129, 64, 64, 64, 0) == vk.ERR_ARGS  # M > 128
    assert L.vkllm_hip_gemm_streamed(ctx.vp, PLAIN, p, p, p, 4, 64, 24, 64, 0) == vk.ERR_ARGS  # K % 16 != 0
    assert L.vkllm_hip_gemm_streamed(ctx.vp, 1, p, p, p, 4, 64, 64, 64, 0) == vk.ERR_ARGS  # no SiLU epilogue
    assert L.vkllm_hip_gemm_streamed(ctx.vp, RESID, p, p, p, 4, 48, 64, 48, 0) == vk.ERR_ARGS  # N % 32 != 0
    assert L.vkllm_hip_gemm_streamed(ctx.vp, RESID, p, p, p, 4, 64, 64, 64, 9) == vk.ERR_ARGS  # splits > 8
    assert L.vkllm_hip_gemm_streamed(ctx.vp, SWIGLU, p, p, p, 4, 64, 64, 16, 0) == vk.ERR_ARGS  # ldc < F
    assert L.vkllm_hip_gemm_streamed(ctx.vp, PLAIN, p, p, p, 4, 64, 64, 60, 0) == vk.ERR_ARGS  # ldc < N


@pytest.mark.parametrize("prompt_len", [1, 8, 33, 100, 128])
def test_streamed_prefill_matches_oracle(ctx, vk, oracle, prompt_len):
    """Prompt steps of at most 128 tokens at the 7B widths (two layers) on the streamed products, against the oracle:
    identical greedy ids over the prompt step and 4 decode steps, logits within 2e-2."""
    from test_model_gpu import LOGIT_TOL, _gpu_vs_oracle

    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160)
    ids, want_ids, err = _gpu_vs_oracle(ctx, vk, oracle, shape, seed=5, prompt_len=prompt_len, n_steps=4,
                                        prompt_seed=prompt_len)
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


def test_streamed_prefill_against_tile_gemms(ctx, vk, monkeypatch):
    """The same 100-token prompt step with and without the tiled copies (VKLLM_PREFILL_TILED=0: the 128 x 128 tile
    GEMMs): identical greedy ids; logits within 2e-2 (the two sum in different orders)."""
    from test_model_gpu import LOGIT_TOL, _device_loop

    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160)
    prompt = vk.prompt_tokens(12, 100, shape["vocab"])
    monkeypatch.setenv("VKLLM_PREFILL_TILED", "1")
    ids_a, logits_a = _device_loop(ctx, vk, shape, 7, prompt, 4)
    monkeypatch.setenv("VKLLM_PREFILL_TILED", "0")
    ids_b, logits_b = _device_loop(ctx, vk, shape, 7, prompt, 4)
    assert ids_a.tolist() == ids_b.tolist()
    assert np.max(np.abs(logits_a.astype(np.float32) - logits_b.astype(np.float32))) <= LOGIT_TOL


def test_streamed_prefill_in_chunks(ctx, vk, oracle):
    """A 300-token prompt at the 7B widths (two layers) in chunks of 100, 128 and 72 rows, each a streamed prompt step
    at a nonzero offset (RoPE angles, K/V rows and causal limits past the first chunk), then 4 decode steps: every
    row's logits within 2e-2 of the oracle's, ids as tests/helpers.py::assert_prefill_ids allows, decode steps fed the
    oracle's ids with their logits within 2e-2."""
    from helpers import assert_prefill_ids
    from test_long_gpu import LOGIT_TOL, _forced_decode, _models

    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=320)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=31)
    try:
        prompt = oracle.prompt_tokens(32, 300, cfg.vocab)
        offset = 0
        for n in (100, 128, 72):
            part = prompt[offset:offset + n]
            print(f"[streamed chunks] rows {offset}..{offset + n - 1}", flush=True)
            want_ids, want_logits, _ = ref.step(part, offset, want_logits=True)
            ids = model.step(part, offset)
            logits = model.last_logits(n)
            err = float(np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))))
            print(f"[streamed chunks] max|dlogit| {err:.3g}")
            assert err <= LOGIT_TOL
            assert_prefill_ids(ids, want_ids, want_logits, f"{n}-row chunk at {offset}")
            offset += n
        # every decode step's logits within the tolerance; an id may differ only at a one-ulp tie (fp32 summation
        # order decides those), at most one of the four steps
        worst, ties = _forced_decode(ref, model, want_ids[-1], offset, 4)
        print(f"[streamed chunks] decode max|dlogit| {worst:.3g}, {ties} one-ulp ties")
        assert ties <= 1
    finally:
        ref.close()
        model.close()


@pytest.mark.parametrize("prompt_len", [40, 100])
def test_streamed_prefill_13b_widths(ctx, vk, oracle, prompt_len):
    """Prompt steps at the 13B widths (dim 5120, 40 heads of 128, FFN 13824; one layer, vocabulary 1000) on the
    streamed products: [Wq;Wk;Wv] in two token parts per row group (320 workgroups), [Wu;Wg] with four compute waves
    (216 workgroups), Wo split over K with the residual-norm reduce, and a vocabulary product whose last row block
    is partial. Every prompt row against the oracle, then 3 decode steps fed the oracle's ids."""
    from helpers import assert_prefill_ids
    from test_long_gpu import LOGIT_TOL, _forced_decode, _models

    shape = dict(n_layer=1, dim=5120, n_head=40, ffn=13824, vocab=1000, ctx=128)
    cfg, ref, model = _models(oracle, vk, ctx, shape, seed=41)
    try:
        prompt = oracle.prompt_tokens(42, prompt_len, cfg.vocab)
        want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
        ids = model.step(prompt, 0)
        err = float(np.max(np.abs(model.last_logits(prompt_len).astype(np.float32) -
                                  want_logits.astype(np.float32))))
        print(f"[13b streamed] {prompt_len} rows: max|dlogit| {err:.3g}")
        assert err <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, f"{prompt_len}-row prompt")
        worst, ties = _forced_decode(ref, model, want_ids[-1], prompt_len, 3)
        print(f"[13b streamed] decode max|dlogit| {worst:.3g}, {ties} one-ulp ties")
        assert ties <= 1
    finally:
        ref.close()
        model.close()
