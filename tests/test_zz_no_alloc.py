"""vkllm_hip_gemm_noalloc (split-K partials in the library's fixed scratch array) against vkllm_hip_gemm with a
caller work buffer of the same size: the same tile and split choices, so identical bits. Two calls in a row share
the scratch, the second on a smaller product; the first leaves its partials behind, which the second must not read.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

PLAIN, SILU_HI, RESID, SWIGLU = 0, 1, 2, 3
MAX_WORK = 8 << 20  # floats in the library's scratch array


def _operands(rng, M, N, K, epi, split):
    a = rng.standard_normal((M, K), dtype=np.float32).astype(np.float16)
    b = (rng.standard_normal((N, K), dtype=np.float32) * (1.0 / np.sqrt(K))).astype(np.float16)
    width = split if epi == SWIGLU else N
    c0 = rng.standard_normal((M, width), dtype=np.float32).astype(np.float16) if epi == RESID else \
        np.zeros((M, width), np.float16)
    return a, b, c0


def _run(ctx, vk, a, b, c0, epi, split, work_elems, noalloc):
    M, K = a.shape
    N = b.shape[0]
    ldc = c0.shape[1]
    ta, tb, tc = ctx.tensor_from(a, name="A"), ctx.tensor_from(b, name="B"), ctx.tensor_from(c0, name="C")
    tw = None
    try:
        dev = [t.contents.data.dev for t in (ta, tb, tc)]
        L = vk.lib()
        if noalloc:
            vk.check("vkllm_hip_gemm_noalloc", L.vkllm_hip_gemm_noalloc(ctx.vp, epi, dev[0], dev[1], dev[2], M, N, K,
                                                                        ldc, split, work_elems))
            ctx.sync()
        else:
            tw = ctx.tensor([1, 1, 1, max(work_elems, 1)], vk.F32, name="work")
            ctx.upload(tw, np.zeros(max(work_elems, 1), np.float32))
            vk.check("vkllm_hip_gemm", L.vkllm_hip_gemm(ctx.vp, epi, dev[0], dev[1], dev[2], M, N, K, ldc, split,
                                                        tw.contents.data.dev, work_elems))
        return ctx.download(tc).reshape(M, ldc)
    finally:
        for t in (ta, tb, tc, tw):
            if t is not None:
                ctx.free(t)


# (M, N, K, epi, split, work_elems): each pair is run back to back, the second product smaller than the first
PAIRS = [
    ((128, 12288, 4096, PLAIN, 0, MAX_WORK), (64, 4096, 1024, RESID, 0, 1 << 20)),
    ((128, 22016, 1024, SWIGLU, 11008, MAX_WORK), (100, 3072, 512, SILU_HI, 1536, 2 << 20)),
    ((512, 4096, 4096, RESID, 0, MAX_WORK), (77, 1000, 1000, PLAIN, 0, MAX_WORK)),
]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0][0]}x{p[0][1]}x{p[0][2]}-then-{p[1][0]}x{p[1][1]}x{p[1][2]}")
def test_noalloc_gemm_matches_gemm_with_work_buffer(ctx, vk, pair):
    rng = np.random.default_rng(sum(pair[0][:3]) + pair[1][0])
    ops = [_operands(rng, M, N, K, epi, split) for (M, N, K, epi, split, _) in pair]
    got = []
    for (M, N, K, epi, split, work), (a, b, c0) in zip(pair, ops):
        print(f"[noalloc] M={M} N={N} K={K} epi={epi} split={split} work={work}", flush=True)
        got.append(_run(ctx, vk, a, b, c0, epi, split, work, noalloc=True))
    for (M, N, K, epi, split, work), (a, b, c0), g in zip(pair, ops, got):
        want = _run(ctx, vk, a, b, c0, epi, split, work, noalloc=False)
        assert np.array_equal(g.view(np.uint16), want.view(np.uint16)), f"{M}x{N}x{K} epi {epi} differs"


def test_noalloc_gemm_rejects_work_beyond_its_scratch(ctx, vk):
    L = vk.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the argument checks fail first
    assert L.vkllm_hip_gemm_noalloc(ctx.vp, PLAIN, p, p, p, 4, 4, 16, 4, 0, MAX_WORK + 1) == vk.ERR_ARGS
    assert L.vkllm_hip_gemm_noalloc(ctx.vp, PLAIN, p, p, p, 4, 4, 12, 4, 0, 0) == vk.ERR_ARGS  # K % 8 != 0
