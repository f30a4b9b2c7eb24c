"""The reference's op-test case tables, replayed in their order through the C API against the oracle.

Each table is the reference test's own list of (shapes, dtype, parameters), with the test's own construction of
its operands (views, permutes, output shapes); the inputs are seeded here instead of the tests' unseeded rand().
The bars: bit-exact for update_rows, copy, embedding, bin and arg_max; for the arithmetic ops at most one fp16 ulp
of the oracle (fp16 outputs) or a few fp32 ulps (fp32 outputs), which is far inside the reference tests' own MSE
bars (1e-2 / 1e-3 / 1e-4).
"""
import ctypes

import numpy as np
import pytest

from helpers import argmax_tie_rule, assert_fp16_close, dot_atol, rand

pytestmark = pytest.mark.gpu

F16, F32 = "f16", "f32"


def _dt(vk, d):
    return vk.F16 if d == F16 else vk.F32


def _np(d):
    return np.float16 if d == F16 else np.float32


def _view(oracle, vk, arr, t):
    """oracle tensor over numpy buffer `arr` with the library tensor t's shapes and element strides"""
    return oracle.tensor(arr, shapes=list(t.contents.shapes), strides=vk.tensor_element_strides(t))


def _case_id(case):
    return "-".join(str(x) if not isinstance(x, (tuple, list)) else "x".join(map(str, x)) for x in case)


def _close(got, want, d, what, atol16=0.0, atol32=1e-6):
    if d == F16:
        assert_fp16_close(got, want, max_ulp=1.0, frac_exact=0.98, what=what, atol=atol16)
    else:
        np.testing.assert_allclose(got, want, rtol=4e-6, atol=atol32, err_msg=what)


# ---------------------------------------------------------------------------------------------------------------
# ROPE: tests/vkllm_test_op_rope.c:102-108 (neox_style false). Case 0 views its [1,1,11,3200] input as
# [1,11,32,100] and permutes it to [1,32,11,100] (:126-132); the output takes the input's (permuted) shapes.
ROPE_CASES = [((1, 1, 11, 3200), 0, F16), ((1, 1, 10, 128), 0, F32), ((2, 1, 5, 64), 0, F32),
              ((1, 2, 8, 256), 5, F32), ((3, 4, 6, 32), 10, F32), ((8, 32, 32, 128), 0, F16),
              ((2, 1, 5, 64), 0, F16), ((1, 2, 8, 256), 5, F16), ((3, 4, 6, 32), 10, F16)]


@pytest.mark.parametrize("i,case", list(enumerate(ROPE_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_rope_table(ctx, vk, oracle, i, case):
    shapes, offset, d = case
    L = vk.lib()
    x = rand(shapes, _np(d), -1.0, 1.0, seed=100 + i)
    tin = ctx.tensor_from(x, "input", mapped=True)
    if i == 0:
        vk.check("reshape", L.vkllm_tensor_reshape(ctx.vp, tin, (ctypes.c_uint32 * 4)(1, 11, 32, 100)))
        vk.check("permute", L.vkllm_tensor_permute(ctx.vp, tin, (ctypes.c_uint32 * 4)(0, 2, 1, 3)))
    oshapes = list(tin.contents.shapes)
    out = ctx.tensor(oshapes, _dt(vk, d), "output", vk.OP_ROPE, [tin], vk.RopeParams(offset, 10000.0, False),
                     mapped=True)
    assert ctx.run_op("rope", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(oshapes, _np(d))
    assert oracle.rope(_view(oracle, vk, x, tin), oracle.tensor(want), offset, 10000.0, False) == 0
    # the rotation angle is the same fp32 number on both sides; cos/sin of it differ by at most an fp32 ulp
    _close(got, want, d, f"rope case {i}", atol16=4e-7, atol32=1e-6)
    for t in (out, tin):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# UPDATE_ROWS: tests/vkllm_test_op_update_rows.c:130-135, (in_shapes, out_shapes, offset_rows, dtype)
UPDATE_ROWS_CASES = [((1, 1, 5, 32), (1, 1, 10, 32), 0, F32), ((1, 1, 5, 32), (1, 1, 10, 32), 5, F32),
                     ((2, 3, 4, 64), (2, 3, 10, 64), 2, F32), ((1, 2, 8, 128), (1, 2, 16, 128), 4, F32),
                     ((1, 1, 5, 32), (1, 1, 10, 32), 0, F16), ((1, 1, 5, 32), (1, 1, 10, 32), 5, F16),
                     ((2, 3, 4, 64), (2, 3, 10, 64), 2, F16), ((1, 2, 8, 128), (1, 2, 16, 128), 4, F16)]


@pytest.mark.parametrize("i,case", list(enumerate(UPDATE_ROWS_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_update_rows_table(ctx, vk, oracle, i, case):
    ishapes, oshapes, off, d = case
    src = rand(ishapes, _np(d), -1.0, 1.0, seed=200 + i)
    cache0 = rand(oshapes, _np(d), -1.0, 1.0, seed=300 + i)  # rows outside the update must survive
    tin = ctx.tensor_from(src, "input", mapped=True)
    out = ctx.tensor(list(oshapes), _dt(vk, d), "output", vk.OP_UPDATE_ROWS, [tin], vk.UpdateRowsParams(off),
                     mapped=True)
    ctx.upload(out, cache0)
    assert ctx.run_op("update_rows", out) == vk.ERR_OK
    got = ctx.download(out)
    want = cache0.copy()
    assert oracle.update_rows(oracle.tensor(src), oracle.tensor(want), off) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    closed = cache0.copy()
    closed[:, :, off:off + ishapes[2], :] = src
    assert np.array_equal(want.view(np.uint8), closed.view(np.uint8))
    for t in (out, tin):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# COPY: tests/vkllm_test_op_copy.c:74-82; the input is permuted (0, 2, 1, 3) and copied into a contiguous output
COPY_CASES = [((1, 1, 128, 256), F16), ((2, 4, 64, 128), F16), ((1, 1, 128, 256), F32), ((2, 4, 64, 128), F32),
              ((4, 8, 32, 64), F32), ((8, 16, 128, 256), F16), ((8, 16, 128, 256), F32), ((1, 1, 1, 1), F16),
              ((1, 1, 1, 1), F32)]


@pytest.mark.parametrize("i,case", list(enumerate(COPY_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_copy_table(ctx, vk, oracle, i, case):
    shapes, d = case
    L = vk.lib()
    x = rand(shapes, _np(d), 0.0, 1.0, seed=400 + i)
    tin = ctx.tensor_from(x, "input")
    vk.check("permute", L.vkllm_tensor_permute(ctx.vp, tin, (ctypes.c_uint32 * 4)(0, 2, 1, 3)))
    oshapes = list(tin.contents.shapes)
    out = ctx.tensor(oshapes, _dt(vk, d), "output", vk.OP_COPY, [tin], mapped=True)
    assert ctx.run_op("copy", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(oshapes, _np(d))
    assert oracle.copy(_view(oracle, vk, x, tin), oracle.tensor(want)) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    assert np.array_equal(want, np.transpose(x, (0, 2, 1, 3)))
    for t in (out, tin):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# ARG_MAX: tests/vkllm_test_op_arg_max.c:77-83, values uniform in [-1000, 1000) (:115)
ARG_MAX_CASES = [((1, 1, 10, 128), F32), ((2, 4, 8, 64), F32), ((2, 4, 8, 64), F16), ((3, 5, 7, 256), F32),
                 ((1, 12, 16, 512), F16), ((8, 16, 32, 1024), F32), ((1, 1, 1, 10), F32), ((4, 8, 16, 32), F16)]


def _arg_max_run(ctx, vk, oracle, x, d):
    tin = ctx.tensor_from(x, "input", mapped=True)
    oshapes = list(x.shape[:3]) + [1]
    out = ctx.tensor(oshapes, vk.U32, "output", vk.OP_ARG_MAX, [tin], mapped=True)
    assert ctx.run_op("arg_max", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(oshapes, np.uint32)
    assert oracle.arg_max(oracle.tensor(x), oracle.tensor(want)) == 0
    for t in (out, tin):
        ctx.free(t)
    return got, want


@pytest.mark.parametrize("i,case", list(enumerate(ARG_MAX_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_arg_max_table(ctx, vk, oracle, i, case):
    shapes, d = case
    x = rand(shapes, _np(d), -1000.0, 1000.0, seed=500 + i)
    got, want = _arg_max_run(ctx, vk, oracle, x, d)
    assert np.array_equal(got, want)
    rows = x.reshape(-1, shapes[3])
    assert got.reshape(-1).tolist() == [argmax_tie_rule(r) for r in rows]


@pytest.mark.parametrize("d", [F16, F32])
def test_arg_max_short_rows_keep_the_reference_sentinel(ctx, vk, oracle, d):
    """Rows shorter than the reference's 32 lanes: lanes past the row start from (-FLT_MAX, lane) and are never
    overwritten (src/shaders/vkllm_arg_max.comp:55-60), so a row of -inf answers the first such lane in the
    reduction order (16 for a 10-wide row), and a row holding -FLT_MAX ties with them."""
    W = 10
    rows = np.array([np.full(W, -np.inf), np.r_[np.full(W - 1, -np.inf), 5.0],
                     np.full(W, -np.finfo(np.float32).max), rand(W, np.float32, -3, 3, seed=7),
                     np.r_[-np.inf, np.full(W - 1, np.finfo(np.float32).min)]], dtype=np.float32)
    x = rows.astype(_np(d)).reshape(1, 1, len(rows), W)
    got, want = _arg_max_run(ctx, vk, oracle, x, d)
    assert np.array_equal(got, want)
    assert want.reshape(-1)[0] == 16 and want.reshape(-1)[1] == W - 1
    assert want.reshape(-1)[3] == argmax_tie_rule(x[0, 0, 3])


# ---------------------------------------------------------------------------------------------------------------
# SOFTMAX: tests/vkllm_test_op_softmax.c:127-145, (shapes, dtype, seq_mask, offsets)
SOFTMAX_CASES = [((1, 1, 10, 128), F32, 0, 0), ((2, 1, 5, 256), F32, 0, 0), ((1, 2, 8, 512), F32, 0, 0),
                 ((3, 4, 6, 64), F32, 0, 0), ((1, 1, 10, 128), F32, 1, 0), ((2, 1, 5, 256), F32, 1, 0),
                 ((1, 1, 10, 128), F16, 0, 0), ((2, 1, 5, 256), F16, 0, 0), ((1, 2, 8, 512), F16, 0, 0),
                 ((1, 1, 10, 128), F16, 1, 0)]


@pytest.mark.parametrize("i,case", list(enumerate(SOFTMAX_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_softmax_table(ctx, vk, oracle, i, case):
    shapes, d, mask, offsets = case
    x = rand(shapes, _np(d), -5.0, 5.0, seed=600 + i)
    tin = ctx.tensor_from(x, "input")
    out = ctx.tensor(list(shapes), _dt(vk, d), "output", vk.OP_SOFTMAX, [tin], vk.SoftmaxParams(mask, offsets),
                     mapped=True)
    assert ctx.run_op("softmax", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shapes, _np(d))
    assert oracle.softmax(oracle.tensor(x), oracle.tensor(want), mask, offsets) == 0
    _close(got, want, d, f"softmax case {i}", atol32=1e-7)
    # the reference test's own row-sum check (:254): each row sums to 1 within 5e-2
    assert np.all(np.abs(got.astype(np.float64).sum(axis=-1) - 1.0) <= 5e-2)
    if mask:
        h = np.arange(shapes[2])[:, None]
        w = np.arange(shapes[3])[None, :]
        assert np.all(got[..., (w > h + offsets)] == 0)
    for t in (out, tin):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# RMSNORM: tests/vkllm_test_op_rmsnorm.c:112-118 (fp16 in and out, fp32 weight)
RMSNORM_CASES = [(1, 1, 10, 128), (2, 1, 5, 256), (1, 2, 8, 512), (3, 4, 6, 64)]


@pytest.mark.parametrize("i,shapes", list(enumerate(RMSNORM_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_rmsnorm_table(ctx, vk, oracle, i, shapes):
    x = rand(shapes, np.float16, -1.0, 1.0, seed=700 + i)
    w = rand((1, 1, 1, shapes[3]), np.float32, 0.0, 1.0, seed=800 + i)
    tx, tw = ctx.tensor_from(x, "input"), ctx.tensor_from(w, "weight")
    out = ctx.tensor(list(shapes), vk.F16, "output", vk.OP_RMSNORM, [tx, tw], vk.RmsnormParams(2.0, 1e-5),
                     mapped=True)
    assert ctx.run_op("rmsnorm", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shapes, np.float16)
    assert oracle.rmsnorm(oracle.tensor(x), oracle.tensor(w), oracle.tensor(want), 1e-5) == 0
    assert_fp16_close(got, want, max_ulp=1.0, frac_exact=0.99, what=f"rmsnorm case {i}")
    for t in (out, tx, tw):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# EMBEDDING: tests/vkllm_test_op_embedding.c:17-30 and :114-118: indices [1,1,32,W] u32, table [1,1,128,64], output
# [1,32,W,64], unk token 0. The reference's indices are all 0 ((rand() % 10) / 10); here they cover the table and
# run past it (ids >= 128 read the unk row).
EMBEDDING_CASES = [((1, 1, 32, 32), (1, 1, 128, 64), F32), ((1, 1, 32, 99), (1, 1, 128, 64), F32),
                   ((1, 1, 32, 32), (1, 1, 128, 64), F16), ((1, 1, 32, 99), (1, 1, 128, 64), F16)]


@pytest.mark.parametrize("i,case", list(enumerate(EMBEDDING_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_embedding_table(ctx, vk, oracle, i, case):
    s0, s1, d = case
    ids = np.random.default_rng(900 + i).integers(0, s1[2] + 32, size=s0).astype(np.uint32)
    table = rand(s1, _np(d), 0.0, 1.0, seed=950 + i)
    ti, tt = ctx.tensor_from(ids, "indices"), ctx.tensor_from(table, "params")
    oshapes = [s0[1], s0[2], s0[3], s1[3]]
    out = ctx.tensor(oshapes, _dt(vk, d), "out0", vk.OP_EMBEDDING, [ti, tt], ctypes.c_uint32(0), mapped=True)
    assert ctx.run_op("embedding", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(oshapes, _np(d))
    assert oracle.embedding(oracle.tensor(ids), oracle.tensor(table), oracle.tensor(want), 0) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    rows = np.where(ids >= s1[2], 0, ids).reshape(s0[1], s0[2], s0[3])
    assert np.array_equal(want, table[0, 0][rows])
    for t in (out, ti, tt):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# BIN: tests/vkllm_test_op_bin.c:139-173, (shapes, dtype a, dtype b, op); the output takes a's dtype
BIN_CASES = [((1, 1, 128, 256), F16, F16, 0), ((2, 4, 64, 128), F16, F16, 0), ((1, 1, 128, 256), F32, F32, 0),
             ((2, 4, 64, 128), F32, F32, 0), ((4, 8, 32, 64), F32, F32, 0),
             ((1, 1, 128, 256), F16, F16, 1), ((2, 4, 64, 128), F16, F16, 1), ((1, 1, 128, 256), F32, F32, 1),
             ((2, 4, 64, 128), F32, F32, 1), ((4, 8, 32, 64), F32, F32, 1),
             ((1, 1, 128, 256), F16, F16, 2), ((2, 4, 64, 128), F16, F16, 2), ((1, 1, 128, 256), F32, F32, 2),
             ((2, 4, 64, 128), F32, F32, 2), ((4, 8, 32, 64), F32, F32, 2),
             ((1, 1, 128, 256), F16, F16, 3), ((2, 4, 64, 128), F16, F16, 3), ((1, 1, 128, 256), F32, F32, 3),
             ((2, 4, 64, 128), F32, F32, 3), ((4, 8, 32, 64), F32, F32, 3),
             ((8, 16, 128, 256), F16, F16, 0), ((8, 16, 128, 256), F16, F16, 1), ((8, 16, 128, 256), F16, F16, 2),
             ((8, 16, 128, 256), F16, F16, 3)]


@pytest.mark.parametrize("i,case", list(enumerate(BIN_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_bin_table(ctx, vk, oracle, i, case):
    shapes, da, db, op = case
    a = rand(shapes, _np(da), -1.0, 1.0, seed=1000 + i)
    b = rand(shapes, _np(db), 0.1, 1.0, seed=1100 + i)  # away from 0 for the division
    ta, tb = ctx.tensor_from(a, "a"), ctx.tensor_from(b, "b")
    out = ctx.tensor(list(shapes), _dt(vk, da), "c", vk.OP_BIN, [ta, tb], ctypes.c_int32(op), mapped=True)
    assert ctx.run_op("bin", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros(shapes, _np(da))
    assert oracle.bin_op(oracle.tensor(a), oracle.tensor(b), oracle.tensor(want), op) == 0
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    f = [np.add, np.subtract, np.multiply, np.divide][op]
    closed = f(a.astype(np.float32), b.astype(np.float32)).astype(_np(da))  # one fp32 operation, then the rounding
    assert np.array_equal(want.view(np.uint8), closed.view(np.uint8))
    for t in (out, ta, tb):
        ctx.free(t)


# ---------------------------------------------------------------------------------------------------------------
# FFN_UP_AND_GATE: tests/vkllm_test_op_ffn_up_and_gate.c (x [1,1,128,64], W_up and W_gate [1,1,256,64]) in each
# of the reference's variants, src/shaders/BUILD:170-186: f16 in / f16 out, f16 in / f32 out, f32 in / f32 out;
# then the token step's widths
FFN_CASES = [(128, 64, 256, F16, F16), (128, 64, 256, F16, F32), (128, 64, 256, F32, F32),
             (7, 288, 768, F32, F32), (1, 4096, 1000, F16, F32)]


@pytest.mark.parametrize("i,case", list(enumerate(FFN_CASES)), ids=lambda c: _case_id(c) if isinstance(c, tuple) else str(c))
def test_ffn_up_and_gate_table(ctx, vk, oracle, i, case):
    M, K, N, din, dout = case
    x = rand((1, 1, M, K), _np(din), -1.0, 1.0, seed=1200 + i)
    wu = rand((1, 1, N, K), _np(din), -0.2, 0.2, seed=1300 + i)
    wg = rand((1, 1, N, K), _np(din), -0.2, 0.2, seed=1400 + i)
    tx, tu, tg = ctx.tensor_from(x, "input_x"), ctx.tensor_from(wu, "input_w_up"), ctx.tensor_from(wg, "input_w_gate")
    out = ctx.tensor([1, 1, M, N], _dt(vk, dout), "output", vk.OP_FFN_UP_AND_GATE, [tx, tu, tg], mapped=True)
    assert ctx.run_op("ffn_up_and_gate", out) == vk.ERR_OK
    got = ctx.download(out)
    want = np.zeros((1, 1, M, N), _np(dout))
    assert oracle.ffn_up_and_gate(oracle.tensor(x), oracle.tensor(wu), oracle.tensor(wg), oracle.tensor(want)) == 0
    atol = 2 * (dot_atol(x, wu) + dot_atol(x, wg))
    if dout == F16:
        assert_fp16_close(got, want, max_ulp=1.0, what=f"ffn case {i}", atol=atol)
    else:
        np.testing.assert_allclose(got, want, rtol=4e-6, atol=float(atol.max()) + 1e-7, err_msg=f"ffn case {i}")
    # float64 closed form: up * silu(gate)
    x64, u64, g64 = (v.astype(np.float64)[0, 0] for v in (x, wu, wg))
    u, g = x64 @ u64.T, x64 @ g64.T
    assert np.max(np.abs(want.astype(np.float64)[0, 0] - u * g / (1 + np.exp(-g)))) < 2e-2
    for t in (out, tx, tu, tg):
        ctx.free(t)
