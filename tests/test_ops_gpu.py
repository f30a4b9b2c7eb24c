"""VKLLM_OP_* operators on the GPU through the C API, against the oracle on the same inputs.

Case tables follow the reference's op tests (tests/vkllm_test_op_*.c); the bar is bit-exact for copy, update_rows,
embedding, bin and arg_max, and at most one fp16 ulp (fp32 summation order) for the arithmetic ops.
"""
import ctypes

import numpy as np
import pytest

from helpers import argmax_tie_rule, assert_fp16_close, dot_atol, mse, rand

pytestmark = pytest.mark.gpu


def oview(oracle, arr, t=None, strides=None):
    """oracle tensor over a numpy buffer, with the library tensor's element strides when given"""
    if t is not None:
        tc = t.contents
        es = arr.itemsize
        return oracle.tensor(arr, shapes=list(tc.shapes), strides=[s // es for s in tc.strides])
    return oracle.tensor(arr, strides=strides)


def np_of(dt):
    return {1: np.float32, 2: np.float16, 4: np.uint32}[dt]


# ---------------------------------------------------------------------------------------------------------------
# MATMUL: every case of tests/vkllm_test_op_matmul.c:179-286 in its order (B_a, C_a, B_b, C_b, M, K, N, dtype,
# transposed_b, act), then the token step's decode shapes
MATMUL_CASES = [
    (1, 1, 1, 1, 1, 1024, 2048, "f32", True, False),
    (1, 1, 1, 1, 1, 1024, 2048, "f16", True, False),
    (1, 1, 1, 1, 512, 1024, 2048, "f16", True, False),
    (1, 1, 1, 1, 333, 1259, 365, "f16", True, False),
    (1, 1, 1, 1, 512, 1024, 2048, "f32", True, False),
    (1, 1, 1, 1, 333, 1259, 365, "f32", True, False),
    (1, 1, 1, 1, 512, 1024, 2048, "f16", False, False),
    (1, 1, 1, 1, 333, 1259, 365, "f16", False, False),
    (1, 1, 1, 1, 512, 1024, 2048, "f32", False, False),
    (1, 1, 1, 1, 333, 1259, 365, "f32", False, False),
    (4, 1, 4, 1, 256, 512, 1024, "f16", True, False),
    (8, 1, 8, 1, 128, 256, 512, "f32", True, False),
    (16, 1, 16, 1, 64, 128, 256, "f16", True, False),
    (4, 1, 4, 1, 256, 512, 1024, "f16", False, False),
    (8, 1, 8, 1, 128, 256, 512, "f32", False, False),
    (16, 1, 16, 1, 64, 128, 256, "f16", False, False),
    (2, 4, 2, 4, 128, 256, 512, "f16", True, False),
    (4, 2, 4, 2, 256, 512, 1024, "f32", True, False),
    (2, 4, 2, 4, 128, 256, 512, "f16", False, False),
    (4, 2, 4, 2, 256, 512, 1024, "f32", False, False),
    (1, 1, 4, 1, 128, 256, 512, "f16", True, False),
    (1, 1, 8, 1, 64, 128, 256, "f32", True, False),
    (1, 1, 4, 1, 128, 256, 512, "f16", False, False),
    (1, 1, 8, 1, 64, 128, 256, "f32", False, False),
    (4, 1, 1, 1, 128, 256, 512, "f16", True, False),
    (8, 1, 1, 1, 64, 128, 256, "f32", True, False),
    (4, 1, 1, 1, 128, 256, 512, "f16", False, False),
    (8, 1, 1, 1, 64, 128, 256, "f32", False, False),
    (1, 1, 1, 4, 128, 256, 512, "f16", True, False),
    (1, 1, 1, 8, 64, 128, 256, "f32", True, False),
    (1, 1, 1, 4, 128, 256, 512, "f16", False, False),
    (1, 1, 1, 8, 64, 128, 256, "f32", False, False),
    (1, 4, 1, 1, 128, 256, 512, "f16", True, False),
    (1, 8, 1, 1, 64, 128, 256, "f32", True, False),
    (1, 4, 1, 1, 128, 256, 512, "f16", False, False),
    (1, 8, 1, 1, 64, 128, 256, "f32", False, False),
    (1, 1, 4, 4, 64, 128, 256, "f16", True, False),
    (1, 1, 2, 8, 64, 128, 256, "f32", True, False),
    (1, 1, 4, 4, 64, 128, 256, "f16", False, False),
    (1, 1, 2, 8, 64, 128, 256, "f32", False, False),
    (4, 4, 1, 1, 64, 128, 256, "f16", True, False),
    (2, 8, 1, 1, 64, 128, 256, "f32", True, False),
    (4, 4, 1, 1, 64, 128, 256, "f16", False, False),
    (2, 8, 1, 1, 64, 128, 256, "f32", False, False),
    (1, 4, 4, 1, 64, 128, 256, "f16", True, False),
    (1, 8, 8, 1, 64, 128, 256, "f32", True, False),
    (1, 4, 4, 1, 64, 128, 256, "f16", False, False),
    (1, 8, 8, 1, 64, 128, 256, "f32", False, False),
    (1, 1, 1, 1, 512, 1024, 2048, "f16", True, True),
    (1, 1, 1, 1, 333, 1259, 365, "f32", True, True),
    (1, 1, 1, 1, 256, 512, 1024, "f16", False, True),
    (1, 1, 1, 1, 128, 256, 512, "f32", False, True),
    (4, 1, 4, 1, 256, 512, 1024, "f16", True, True),
    (8, 1, 8, 1, 128, 256, 512, "f32", True, True),
    (4, 1, 4, 1, 256, 512, 1024, "f16", False, True),
    (8, 1, 8, 1, 128, 256, 512, "f32", False, True),
    (2, 4, 2, 4, 128, 256, 512, "f16", True, True),
    (4, 2, 4, 2, 256, 512, 1024, "f32", True, True),
    (1, 1, 4, 1, 128, 256, 512, "f16", True, True),
    (4, 1, 1, 1, 128, 256, 512, "f32", True, True),
    (1, 1, 1, 4, 128, 256, 512, "f16", True, True),
    (1, 4, 1, 1, 64, 128, 256, "f32", True, True),
    (1, 1, 4, 4, 64, 128, 256, "f16", True, True),
    (4, 4, 1, 1, 64, 128, 256, "f32", True, True),
    (1, 4, 4, 1, 64, 128, 256, "f16", True, True),
    # the token step's decode shapes
    (1, 1, 1, 1, 1, 4096, 11008, "f16", True, False),
    (1, 1, 1, 1, 1, 288, 768, "f16", True, True),
]


@pytest.mark.parametrize("case", MATMUL_CASES, ids=lambda c: "x".join(str(v) for v in c))
def test_matmul(ctx, vk, oracle, case):
    Ba, Ca, Bb, Cb, M, K, N, dts, tb, act = case
    dt = vk.F16 if dts == "f16" else vk.F32
    npdt = np_of(dt)
    Bc, Cc = max(Ba, Bb), max(Ca, Cb)
    a = rand((Ba, Ca, M, K), npdt, seed=1)
    b = rand((Bb, Cb, N, K) if tb else (Bb, Cb, K, N), npdt, seed=2)
    ta = ctx.tensor_from(a, "a")
    tbt = ctx.tensor_from(b, "b")
    p = vk.MatmulParams(1.0, int(act))
    out = ctx.tensor([Bc, Cc, M, N], dt, "out", vk.OP_MATMUL, [ta, tbt], p, mapped=True)
    assert ctx.run_op("matmul", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros((Bc, Cc, M, N), dtype=npdt)
    assert oracle.matmul(oview(oracle, a), oview(oracle, b), oview(oracle, want), 1.0, int(act)) == 0
    if dt == vk.F16:
        atol = dot_atol(a, b, transposed=tb) * (1.0 + 0.25 * act)
        assert_fp16_close(got, want, max_ulp=1.0, what="matmul", atol=atol)
        assert mse(got, want) <= 1e-2  # the reference's own bar, tests/vkllm_test_op_matmul.c:382
    else:
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5 * np.sqrt(K))
    for t in (ta, tbt, out):
        ctx.free(t)


def test_matmul_transposed_rule_on_attention_shapes(ctx, vk, oracle):
    """attn . V with kv == head_dim is read as attn . V^T (src/core/vkllm_op_matmul.c:14-24)."""
    hd = 48
    attn = rand((1, 6, 1, hd), np.float16, 0, 1, seed=3)
    v = rand((1, 6, hd, hd), np.float16, seed=4)
    ta = ctx.tensor_from(attn)
    tv = ctx.tensor_from(v)
    out = ctx.tensor([1, 6, 1, hd], vk.F16, "o", vk.OP_MATMUL, [ta, tv], vk.MatmulParams(1.0, 0))
    assert ctx.run_op("matmul", out) == vk.ERR_OK
    got = ctx.download(out)
    want_t = np.einsum("bcmk,bcnk->bcmn", attn.astype(np.float64), v.astype(np.float64))
    want_n = np.einsum("bcmk,bckn->bcmn", attn.astype(np.float64), v.astype(np.float64))
    assert np.max(np.abs(got - want_t)) < 2e-2
    assert np.max(np.abs(got - want_n)) > 0.1
    for t in (ta, tv, out):
        ctx.free(t)


def test_matmul_errors(ctx, vk):
    a = ctx.tensor([1, 1, 4, 8], vk.F16)
    b = ctx.tensor([1, 1, 8, 8], vk.F32)
    out = ctx.tensor([1, 1, 4, 8], vk.F16, op=vk.OP_MATMUL, srcs=[a, b], params=vk.MatmulParams(1.0, 0))
    assert ctx.run_op("matmul", out) == vk.ERR_PIPELINE_NOT_FOUND
    b2 = ctx.tensor([1, 1, 8, 8], vk.F16)
    out2 = ctx.tensor([1, 1, 4, 8], vk.F32, op=vk.OP_MATMUL, srcs=[a, b2], params=vk.MatmulParams(1.0, 0))
    assert ctx.run_op("matmul", out2) == vk.ERR_PIPELINE_NOT_FOUND
    for t in (a, b, out, b2, out2):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# RMSNORM: tests/vkllm_test_op_rmsnorm.c; the isolated [512, 4096] case of the workload list
@pytest.mark.parametrize("shape", [(1, 1, 1, 288), (1, 1, 16, 4096), (1, 1, 512, 4096), (2, 3, 7, 1000)])
def test_rmsnorm(ctx, vk, oracle, shape):
    x = rand(shape, np.float16, -2, 2, seed=5)
    w = rand((1, 1, 1, shape[3]), np.float32, 0.5, 1.5, seed=6)
    tx, tw = ctx.tensor_from(x), ctx.tensor_from(w)
    out = ctx.tensor(list(shape), vk.F16, "n", vk.OP_RMSNORM, [tx, tw], vk.RmsnormParams(2.0, 1e-5))
    assert ctx.run_op("rmsnorm", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shape, np.float16)
    assert oracle.rmsnorm(oview(oracle, x), oview(oracle, w), oview(oracle, want), 1e-5) == 0
    assert_fp16_close(got, want, max_ulp=1.0, frac_exact=0.99, what="rmsnorm")
    for t in (tx, tw, out):
        ctx.free(t)


def test_rmsnorm_needs_f32_weight(ctx, vk):
    x = ctx.tensor([1, 1, 2, 64], vk.F16)
    w = ctx.tensor([1, 1, 1, 64], vk.F16)
    out = ctx.tensor([1, 1, 2, 64], vk.F16, op=vk.OP_RMSNORM, srcs=[x, w], params=vk.RmsnormParams(2.0, 1e-5))
    assert ctx.run_op("rmsnorm", out) == vk.ERR_PIPELINE_NOT_FOUND
    for t in (x, w, out):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# ROPE: tests/vkllm_test_op_rope.c; model layout: a [1,S,H,hd] view permuted to [1,H,S,hd]
@pytest.mark.parametrize("neox", [False, True])
# (4, 40, 128, 7): more 16-byte vectors per position (640) than a workgroup requests before its angle table (512)
@pytest.mark.parametrize("S,H,hd,offset", [(512, 32, 128, 0), (16, 6, 48, 0), (1, 32, 128, 383), (3, 4, 64, 4093),
                                           (4, 40, 128, 7)])
def test_rope(ctx, vk, oracle, neox, S, H, hd, offset):
    x = rand((1, 1, S, H * hd), np.float16, -2, 2, seed=7)
    base = ctx.tensor_from(x)
    L = vk.lib()
    ref = vk.TensorP()
    vk.check("copy_ref", L.vkllm_tensor_copy_ref(ctx.vp, base, ctypes.byref(ref)))
    vk.check("reshape", L.vkllm_tensor_reshape(ctx.vp, ref, (ctypes.c_uint32 * 4)(1, S, H, hd)))
    vk.check("permute", L.vkllm_tensor_permute(ctx.vp, ref, (ctypes.c_uint32 * 4)(0, 2, 1, 3)))
    shapes = list(ref.contents.shapes)
    out = ctx.tensor(shapes, vk.F16, "r", vk.OP_ROPE, [ref], vk.RopeParams(offset, 10000.0, neox))
    assert ctx.run_op("rope", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shapes, np.float16)
    xin = oracle.tensor(x, shapes=shapes, strides=vk.tensor_element_strides(ref))
    assert oracle.rope(xin, oview(oracle, want), offset, 10000.0, neox) == 0
    # cos/sin of the same fp32 angle differ by an fp32 ulp between libraries; near-cancelling pairs show it
    assert_fp16_close(got, want, max_ulp=1.0, frac_exact=0.99, what="rope", atol=4e-7 * float(np.abs(x).max()))
    for t in (out, ref, base):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# SOFTMAX: tests/vkllm_test_op_softmax.c
@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("shape,mask,offsets", [((1, 4, 16, 64), 1, 10), ((1, 32, 1, 385), 1, 384),
                                                ((2, 3, 5, 1000), 0, 0), ((1, 6, 16, 16), 1, 0)])
def test_softmax(ctx, vk, oracle, dt, shape, mask, offsets):
    d = vk.F16 if dt == "f16" else vk.F32
    x = rand(shape, np_of(d), -4, 4, seed=8)
    tx = ctx.tensor_from(x)
    out = ctx.tensor(list(shape), d, "s", vk.OP_SOFTMAX, [tx], vk.SoftmaxParams(mask, offsets))
    assert ctx.run_op("softmax", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shape, np_of(d))
    assert oracle.softmax(oview(oracle, x), oview(oracle, want), mask, offsets) == 0
    if d == vk.F16:
        assert_fp16_close(got, want, max_ulp=1.0, frac_exact=0.98, what="softmax")
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)
    for t in (tx, out):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# UPDATE_ROWS and COPY: bit-exact moves (tests/vkllm_test_op_update_rows.c:124-135, tests/vkllm_test_op_copy.c)
@pytest.mark.parametrize("S,offset", [(1, 0), (1, 255), (16, 0), (7, 100)])
def test_update_rows(ctx, vk, oracle, S, offset):
    H, ctxlen, hd = 6, 256, 48
    cache0 = rand((1, H, ctxlen, hd), np.float16, seed=9)
    src = rand((1, H, S, hd), np.float16, seed=10)
    tc = ctx.tensor([1, H, ctxlen, hd], vk.F16, "cache", vk.OP_UPDATE_ROWS, [], vk.UpdateRowsParams(offset))
    ctx.upload(tc, cache0)
    ts = ctx.tensor_from(src)
    tc.contents.srcs[0] = ts
    assert ctx.run_op("update_rows", tc) == vk.ERR_OK
    got = ctx.download(tc)
    want = cache0.copy()
    assert oracle.update_rows(oview(oracle, src), oview(oracle, want), offset) == 0
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    tc.contents.srcs[0] = vk.TensorP()
    for t in (ts, tc):
        ctx.free(t)


def test_update_rows_out_of_range(ctx, vk):
    tc = ctx.tensor([1, 2, 8, 16], vk.F16, "cache", vk.OP_UPDATE_ROWS, [], vk.UpdateRowsParams(6))
    ts = ctx.tensor([1, 2, 3, 16], vk.F16)
    tc.contents.srcs[0] = ts
    assert ctx.run_op("update_rows", tc) == vk.ERR_ARGS
    tc.contents.srcs[0] = vk.TensorP()
    ctx.free(ts)
    ctx.free(tc)


def test_copy_concat_heads(ctx, vk, oracle):
    """[1,H,S,hd] -> permute -> COPY -> [1,S,H,hd] contiguous (src/models/vkllm_llama2_layers.c:259-281)"""
    H, S, hd = 32, 5, 128
    x = rand((1, H, S, hd), np.float16, seed=11)
    base = ctx.tensor_from(x)
    L = vk.lib()
    ref = vk.TensorP()
    vk.check("copy_ref", L.vkllm_tensor_copy_ref(ctx.vp, base, ctypes.byref(ref)))
    vk.check("permute", L.vkllm_tensor_permute(ctx.vp, ref, (ctypes.c_uint32 * 4)(0, 2, 1, 3)))
    out = ctx.tensor(list(ref.contents.shapes), vk.F16, "c", vk.OP_COPY, [ref])
    assert ctx.run_op("copy", out) == vk.ERR_OK
    got = ctx.download(out)
    assert np.array_equal(got.view(np.uint16), np.transpose(x, (0, 2, 1, 3)).view(np.uint16))
    for t in (out, ref, base):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# BIN: tests/vkllm_test_op_bin.c; one IEEE fp32 operation then the output rounding, so bit-exact
@pytest.mark.parametrize("op", [0, 1, 2, 3])
@pytest.mark.parametrize("dts", [("f16", "f16"), ("f16", "f32"), ("f32", "f32"), ("f32", "f16")])
def test_bin(ctx, vk, oracle, op, dts):
    din = vk.F16 if dts[0] == "f16" else vk.F32
    dout = vk.F16 if dts[1] == "f16" else vk.F32
    shape = (2, 3, 17, 129)
    a = rand(shape, np_of(din), -3, 3, seed=12)
    b = rand(shape, np_of(din), 0.5, 3, seed=13)
    ta, tb = ctx.tensor_from(a), ctx.tensor_from(b)
    out = ctx.tensor(list(shape), dout, "o", vk.OP_BIN, [ta, tb], ctypes.c_int32(op))
    assert ctx.run_op("bin", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shape, np_of(dout))
    assert oracle.bin_op(oview(oracle, a), oview(oracle, b), oview(oracle, want), op) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    for t in (ta, tb, out):
        ctx.free(t)


def test_bin_f32_to_f16_rounding(ctx, vk, oracle):
    """fp32 -> fp16 conversion on the device is round-to-nearest-even, subnormals included."""
    r = np.random.default_rng(14)
    a = np.concatenate([r.standard_normal(4000).astype(np.float32) * 3,
                        r.standard_normal(1000).astype(np.float32) * 1e-5,
                        np.float32([65504, 65519.9, 65520, 6.0e-8, 2.98e-8, 2.99e-8, -0.0, 1.0 + 2 ** -11])])
    a = a.reshape(1, 1, 1, -1)
    z = np.full_like(a, -0.0)  # x + (-0) == x for every x, -0 included
    ta, tz = ctx.tensor_from(a), ctx.tensor_from(z)
    out = ctx.tensor(list(a.shape), vk.F16, "o", vk.OP_BIN, [ta, tz], ctypes.c_int32(0))
    assert ctx.run_op("bin", out) == vk.ERR_OK
    got = ctx.download(out)
    assert np.array_equal(got.view(np.uint16), a.astype(np.float16).view(np.uint16))
    for t in (ta, tz, out):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# EMBEDDING: tests/vkllm_test_op_embedding.c (there only token 0 is exercised); ids >= rows read the unk row
@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_embedding(ctx, vk, oracle, dt):
    d = vk.F16 if dt == "f16" else vk.F32
    V, D, S, unk = 1000, 288, 37, 3
    table = rand((1, 1, V, D), np_of(d), seed=15)
    ids = np.random.default_rng(16).integers(0, V, size=(1, 1, 1, S)).astype(np.uint32)
    ids[0, 0, 0, 5] = V + 7
    ids[0, 0, 0, 9] = 0xFFFFFFFF
    ti, tt = ctx.tensor_from(ids), ctx.tensor_from(table)
    out = ctx.tensor([1, 1, S, D], d, "e", vk.OP_EMBEDDING, [ti, tt], ctypes.c_uint32(unk))
    assert ctx.run_op("embedding", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros((1, 1, S, D), np_of(d))
    assert oracle.embedding(oview(oracle, ids), oview(oracle, table), oview(oracle, want), unk) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    assert np.array_equal(got[0, 0, 5], table[0, 0, unk])
    for t in (ti, tt, out):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# ARG_MAX: tests/vkllm_test_op_arg_max.c:73-83 (exact); plus engineered ties for the lane tie rule
def _argmax_rows(seed):
    r = np.random.default_rng(seed)
    rows = []
    for W in (32000, 31, 32, 33, 1000, 4096):
        x = r.standard_normal(W).astype(np.float16)
        rows.append(x)
    for W in (32000, 1000, 100):
        x = r.standard_normal(W).astype(np.float16)
        m = np.float16(10.0)
        for k in r.choice(W, size=min(6, W), replace=False):
            x[k] = m
        rows.append(x)
    x = np.full(512, np.float16(1.0))
    rows.append(x)  # all tied
    return rows


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_arg_max(ctx, vk, oracle, dt):
    d = vk.F16 if dt == "f16" else vk.F32
    for i, row in enumerate(_argmax_rows(17)):
        x = row.astype(np_of(d)).reshape(1, 1, 1, -1)
        x = np.concatenate([x, x[..., ::-1].copy()], axis=2)  # two rows
        tx = ctx.tensor_from(x)
        out = ctx.tensor([1, 1, 2, 1], vk.U32, "a", vk.OP_ARG_MAX, [tx], mapped=True)
        assert ctx.run_op("arg_max", out) == vk.ERR_OK
        got = ctx.download(out).reshape(-1)
        want = np.zeros((1, 1, 2, 1), np.uint32)
        assert oracle.arg_max(oview(oracle, x), oview(oracle, want)) == 0
        assert got.tolist() == want.reshape(-1).tolist(), f"row set {i}"
        assert got.tolist() == [argmax_tie_rule(x[0, 0, 0]), argmax_tie_rule(x[0, 0, 1])]
        ctx.free(tx)
        ctx.free(out)


# ---------------------------------------------------------------------------------------------------------------
# FFN_UP_AND_GATE (tests/vkllm_test_op_ffn_up_and_gate.c never compares; here against the oracle)
@pytest.mark.parametrize("M,K,N", [(1, 288, 768), (16, 288, 768), (33, 256, 130)])
def test_ffn_up_and_gate(ctx, vk, oracle, M, K, N):
    x = rand((1, 1, M, K), np.float16, seed=18)
    wu = rand((1, 1, N, K), np.float16, -0.1, 0.1, seed=19)
    wg = rand((1, 1, N, K), np.float16, -0.1, 0.1, seed=20)
    tx, tu, tg = ctx.tensor_from(x), ctx.tensor_from(wu), ctx.tensor_from(wg)
    out = ctx.tensor([1, 1, M, N], vk.F16, "f", vk.OP_FFN_UP_AND_GATE, [tx, tu, tg])
    assert ctx.run_op("ffn_up_and_gate", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros((1, 1, M, N), np.float16)
    assert oracle.ffn_up_and_gate(oview(oracle, x), oview(oracle, wu), oview(oracle, wg), oview(oracle, want)) == 0
    u_atol = dot_atol(x, wu)
    g_atol = dot_atol(x, wg)
    assert_fp16_close(got, want, max_ulp=1.0, what="ffn", atol=2 * (u_atol + g_atol))
    for t in (tx, tu, tg, out):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
def test_tensor_new_rejects_zero_shape(ctx, vk):
    L = vk.lib()
    out = vk.TensorP()
    rc = L.vkllm_tensor_new(ctx.vp, b"z", (ctypes.c_uint32 * 4)(1, 0, 2, 2), vk.F16, vk.OP_NONE, None, 0, None, 0,
                            False, ctypes.byref(out))
    assert rc == vk.ERR_ARGS


def test_context_bad_device(vk):
    L = vk.lib()
    p = ctypes.POINTER(vk.Context)()
    assert L.vkllm_context_new(1000, ctypes.byref(p)) == vk.ERR_DEV_NOT_FOUND


def test_upload_too_large(ctx, vk):
    t = ctx.tensor([1, 1, 1, 8], vk.F16)
    buf = np.zeros(1024, np.uint8)
    assert vk.lib().vkllm_commands_upload(ctx.vp, ctx.cmds, t, buf.ctypes.data, 1024) == vk.ERR_ARGS
    ctx.free(t)
