"""The prompt-step GEMM (vkllm_hip_gemm) on each of its tile and split-K paths, against a float32 product of the
same fp16 operands.

The fused prompt step runs every matmul node of the reference graph (src/core/vkllm_op_matmul.c, shader
src/shaders/vkllm_matmul.comp) through this GEMM: C = A . B^T with fp16 operands and fp32 accumulation, rounded
once to fp16, with the SiLU or residual epilogue fused. The model tests reach it only at the tiny workload's
sizes; these cases reach the paths that 7B and 13B prompts take: 256 x 256 tiles, the split-K tail of a partial
last round of those tiles, one round of them with K split (residual products of long rows), 128 x 128 tiles with
and without split K, the 64-wide fallback tiles (K not a multiple of 64), ragged M and N, and the SwiGLU epilogue
that reads [Wu; Wg] as interleaved row blocks. The bar is the fp16 rounding of an fp32 sum:
|C - ref| <= 1e-3 + 2e-3 |ref|, twice that for the residual and SwiGLU epilogues, which round twice.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PLAIN, SILU_HI, RESID, SWIGLU = 0, 1, 2, 3
WORK_ELEMS = 16 << 20  # the fused step's split-K buffer (floats)

# (M, N, K, epi, split, with_work): sizes assume the 256 CUs of an MI355X where a path depends on the CU count
CASES = [
    (1024, 12288, 4096, PLAIN, 0, True),      # 7B QKV, 1024 tokens: one round of 256 x 256 tiles
    (1024, 22016, 4096, SILU_HI, 11008, True),  # 7B gate+up: full round + split-K tail, SiLU split before the tail
    (1024, 22016, 1024, SILU_HI, 20000, True),  # SiLU split inside the tail columns
    (2048, 27648, 512, SILU_HI, 13824, True),   # 13B gate+up shape, 2048 tokens: three full rounds + tail
    (1200, 15300, 1024, RESID, 0, True),      # ragged M and N through the tail split, residual epilogue
    (2048, 5120, 512, RESID, 0, True),        # 13B Wo shape: 256 tiles of 128 x 320 instead of 160 of 256 x 256
    (2000, 5000, 512, RESID, 0, True),        # the same rule, ragged M and N (partial 128 x 320 tiles)
    (2048, 5120, 512, PLAIN, 0, True),        # plain epilogue: 160 tiles of 256 x 256 beat 2.5 rounds of 128 x 128
    (1100, 9000, 256, PLAIN, 0, True),        # the same rule, ragged M and N
    (128, 12288, 4096, PLAIN, 0, True),       # 128-token prompt: 128 x 128 tiles, split K, two K steps in flight
    (128, 12288, 4096, PLAIN, 0, False),      # the same without a work buffer: no split
    # prompts of <= 128 tokens with tiles for most CUs: whole K per tile, four K steps of loads in flight
    (128, 22016, 4096, SILU_HI, 11008, True),  # 7B gate+up, 128 tokens
    (128, 22016, 1216, SILU_HI, 11008, True),  # 19 K steps: four groups of four and a tail of three
    (100, 32000, 512, PLAIN, 0, True),        # logits shape, ragged M
    (64, 24576, 1024, RESID, 0, True),        # residual epilogue
    (96, 24576, 128, PLAIN, 0, True),         # two K steps: tail only
    (96, 24576, 192, PLAIN, 0, True),         # three K steps: tail only
    (512, 4096, 4096, RESID, 0, True),        # 128 x 128 split K with the residual epilogue
    (2048, 4096, 1024, RESID, 0, True),       # 128 x 128 tiles, enough of them that K is not split
    # SwiGLU epilogue: B = [Wu; Wg] read as interleaved 32-row blocks, C = fp16(fp16(up) * fp16(silu(gate)))
    (1024, 22016, 4096, SWIGLU, 11008, True),  # 7B, 1024 tokens: 256 x 256 tiles and the split-K tail
    (2048, 27648, 512, SWIGLU, 13824, True),  # 13B FFN widths, 2048 tokens
    (128, 22016, 1216, SWIGLU, 11008, True),  # 128 tokens: whole K per 128 x 128 tile, four steps in flight
    (128, 12288, 1024, SWIGLU, 6144, True),   # 128 x 128 tiles with split K and the reduce
    (100, 3072, 512, SWIGLU, 1536, False),    # ragged M, no work buffer
    # the LLaMA-2-13B prompt products at 2048 tokens with their real K (dim 5120, FFN 13824)
    (2048, 15360, 5120, PLAIN, 0, True),      # [Wq; Wk; Wv]
    (2048, 5120, 5120, RESID, 0, True),       # Wo + residual: 256 tiles of 128 x 320
    (2048, 27648, 5120, SWIGLU, 13824, True),  # [Wu; Wg] with SwiGLU: three full rounds and the split-K tail
    (2048, 5120, 13824, RESID, 0, True),      # Wd + residual: 256 tiles of 128 x 320
    (2048, 32000, 5120, PLAIN, 0, True),      # logits
    # residual products with long rows whose 256 x 256 tiles leave CUs idle: K split over one round of them
    (1024, 4096, 11008, RESID, 0, True),      # 7B Wd, 1024 tokens: 64 tiles x 4 K ranges
    (1024, 5120, 5120, RESID, 0, True),       # 13B Wo, 1024 tokens: 80 tiles x 3
    (640, 4096, 11008, RESID, 0, True),       # ragged last row tile: 48 tiles x 5
    (1024, 4096, 4096, RESID, 0, True),       # 7B Wo (K 4096) stays on 128 x 128 tiles
    (77, 1000, 256, PLAIN, 0, True),          # ragged, one partial tile row
    (77, 1000, 1000, PLAIN, 0, True),         # K % 64 != 0: 128 x 64 tiles
    (300, 1000, 1000, SILU_HI, 500, True),    # K % 64 != 0, M > 128
]


def reference(a, b, c0, epi, split):
    acc = a.astype(np.float32) @ b.astype(np.float32).T
    if epi == SWIGLU:
        # B = [Wu; Wg]: fp16(fp16(up) * fp16(silu(gate))) as the reference's ffn_up_and_gate rounds it
        up, gate = acc[:, :split], acc[:, split:]
        sg = (gate / (1.0 + np.exp(-gate))).astype(np.float16).astype(np.float32)
        return (up.astype(np.float16).astype(np.float32) * sg).astype(np.float16).astype(np.float32)
    if epi == SILU_HI:
        hi = acc[:, split:]
        acc[:, split:] = hi / (1.0 + np.exp(-hi))
        return acc
    if epi == RESID:
        return c0.astype(np.float32) + acc.astype(np.float16).astype(np.float32)
    return acc


def run_gemm(ctx, vk, a, b, c0, epi, split, with_work):
    M, K = a.shape
    N = b.shape[0]
    ldc = c0.shape[1]
    ta = ctx.tensor_from(a, name="A")
    tb = ctx.tensor_from(b, name="B")
    tc = ctx.tensor_from(c0, name="C")
    tw = ctx.tensor([1, 1, 1, WORK_ELEMS], vk.F32, name="work") if with_work else None
    try:
        if tw is not None:
            ctx.upload(tw, np.zeros(WORK_ELEMS, np.float32))  # allocates the device memory
        dev = [t.contents.data.dev for t in (ta, tb, tc)]
        work = tw.contents.data.dev if tw is not None else None
        rc = vk.lib().vkllm_hip_gemm(ctx.vp, epi, dev[0], dev[1], dev[2], M, N, K, ldc, split, work,
                                     WORK_ELEMS if tw is not None else 0)
        vk.check("vkllm_hip_gemm", rc)
        return ctx.download(tc).reshape(M, ldc)
    finally:
        for t in (ta, tb, tc, tw):
            if t is not None:
                ctx.free(t)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}-e{c[3]}-s{c[4]}-w{int(c[5])}")
def test_gemm_paths(ctx, vk, case):
    M, N, K, epi, split, with_work = case
    print(f"[gemm] M={M} N={N} K={K} epi={epi} split={split} work={with_work}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 3 + K + epi)
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    b = (rng.standard_normal((N, K), dtype=np.float32) * (1.0 / np.sqrt(K))).astype(np.float16)
    width = split if epi == SWIGLU else N
    c0 = rng.standard_normal((M, width), dtype=np.float32).astype(np.float16) if epi == RESID else \
        np.zeros((M, width), np.float16)
    got = run_gemm(ctx, vk, a, b, c0, epi, split, with_work).astype(np.float32)
    ref = reference(a, b, c0, epi, split)
    # the residual and SwiGLU epilogues round twice
    tol = (1e-3 + 2e-3 * np.abs(ref)) * (2.0 if epi in (RESID, SWIGLU) else 1.0)
    err = np.abs(got - ref)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} outside tolerance; worst at "
                           f"{np.unravel_index(np.argmax(err - tol), err.shape)}: got "
                           f"{got.flat[np.argmax(err - tol)]} ref {ref.flat[np.argmax(err - tol)]}")


def test_gemm_split_k_is_deterministic(ctx, vk):
    """The split-K reduce adds the partial tiles in a fixed order: repeated calls give identical bits."""
    M, N, K = 1024, 22016, 1024
    rng = np.random.default_rng(5)
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    b = (rng.standard_normal((N, K), dtype=np.float32) * (1.0 / np.sqrt(K))).astype(np.float16)
    c0 = np.zeros((M, N), np.float16)
    first = run_gemm(ctx, vk, a, b, c0, SILU_HI, 11008, True)
    second = run_gemm(ctx, vk, a, b, c0, SILU_HI, 11008, True)
    assert np.array_equal(first.view(np.uint16), second.view(np.uint16))


def test_gemm_rejects_bad_arguments(ctx, vk):
    L = vk.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the argument checks fail first
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, p, p, p, 4, 4, 12, 4, 0, None, 0) == vk.ERR_ARGS  # K % 8 != 0
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, p, p, p, 4, 8, 16, 4, 0, None, 0) == vk.ERR_ARGS  # ldc < N
    assert L.vkllm_hip_gemm(ctx.vp, 4, p, p, p, 4, 4, 16, 4, 0, None, 0) == vk.ERR_ARGS  # unknown epilogue
    assert L.vkllm_hip_gemm(ctx.vp, SWIGLU, p, p, p, 4, 128, 64, 64, 32, None, 0) == vk.ERR_ARGS  # N != 2 split
    assert L.vkllm_hip_gemm(ctx.vp, SWIGLU, p, p, p, 4, 128, 96, 64, 64, None, 0) == vk.ERR_ARGS  # K % 64 != 0
    assert L.vkllm_hip_gemm(ctx.vp, SWIGLU, p, p, p, 4, 96, 64, 48, 48, None, 0) == vk.ERR_ARGS  # N % 64 != 0
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, p, p, p, 4, 4, 16, 4, 0, None, 64) == vk.ERR_ARGS  # work size, no work
    q = ctypes.c_void_p(18)  # 2-byte aligned only
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, q, p, p, 4, 4, 16, 4, 0, None, 0) == vk.ERR_ARGS  # A not 16-byte aligned
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, p, q, p, 4, 4, 16, 4, 0, None, 0) == vk.ERR_ARGS  # B not 16-byte aligned
    assert L.vkllm_hip_gemm(ctx.vp, PLAIN, p, p, p, 4, 4, 16, 4, 0, q, 64) == vk.ERR_ARGS  # work not aligned
    assert L.vkllm_hip_gemm(ctx.vp, SWIGLU, p, p, q, 4, 128, 64, 64, 64, None, 0) == vk.ERR_ARGS  # C not aligned
