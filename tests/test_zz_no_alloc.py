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


def _hip_runtime():
    """The HIP runtime libvkllm itself is linked against (found among the process's mapped files), so the stream
    handle the context hands out belongs to it."""
    with open("/proc/self/maps") as f:
        paths = {line.split()[-1] for line in f if "libamdhip64.so" in line}
    assert paths, "libamdhip64 is not mapped"
    H = ctypes.CDLL(sorted(paths)[0])
    vp = ctypes.c_void_p
    for name, args in (("hipStreamBeginCapture", [vp, ctypes.c_int]), ("hipStreamEndCapture", [vp, ctypes.POINTER(vp)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipStreamSynchronize", [vp]),
                       ("hipGraphExecDestroy", [vp]), ("hipGraphDestroy", [vp])):
        fn = getattr(H, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    return H


def test_noalloc_gemm_under_stream_capture(ctx, vk):
    """One split-K call captured into a hipGraph (global capture mode, where an allocating call would fail the
    capture), replayed three times with eager calls of other shapes between the replays (each overwrites the shared
    scratch): every replay's output is bit-identical to the eager call's."""
    M, N, K = 64, 1024, 8192  # 8 tiles of 128 x 128 on 256 CUs: K is split, the partials go through the scratch
    rng = np.random.default_rng(5)
    a, b, c0 = _operands(rng, M, N, K, PLAIN, 0)
    want = _run(ctx, vk, a, b, c0, PLAIN, 0, MAX_WORK, noalloc=True)
    H = _hip_runtime()
    L = vk.lib()
    stream = ctypes.c_void_p()
    vk.check("vkllm_hip_context_stream", L.vkllm_hip_context_stream(ctx.vp, ctypes.byref(stream)))
    ta, tb = ctx.tensor_from(a, name="A"), ctx.tensor_from(b, name="B")
    tc = ctx.tensor_from(np.zeros((M, N), np.float16), name="C")
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        dev = [t.contents.data.dev for t in (ta, tb, tc)]
        print(f"[noalloc capture] M={M} N={N} K={K}", flush=True)
        assert H.hipStreamBeginCapture(stream, 0) == 0  # hipStreamCaptureModeGlobal
        rc = L.vkllm_hip_gemm_noalloc(ctx.vp, PLAIN, dev[0], dev[1], dev[2], M, N, K, N, 0, MAX_WORK)
        end = H.hipStreamEndCapture(stream, ctypes.byref(graph))
        assert rc == vk.ERR_OK and end == 0, (rc, end)
        assert H.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        other = _operands(rng, 100, 3072, 512, SILU_HI, 1536)
        for rep in range(3):
            ctx.upload(tc, np.zeros((M, N), np.float16))
            assert H.hipGraphLaunch(exe, stream) == 0
            assert H.hipStreamSynchronize(stream) == 0
            got = ctx.download(tc).reshape(M, N)
            assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), f"replay {rep} differs"
            _run(ctx, vk, *other, SILU_HI, 1536, 2 << 20, noalloc=True)  # eager work on the same scratch
    finally:
        if exe.value:
            H.hipGraphExecDestroy(exe)
        if graph.value:
            H.hipGraphDestroy(graph)
        for t in (ta, tb, tc):
            ctx.free(t)
