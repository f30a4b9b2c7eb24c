"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

The reference ships no golden vectors, no known-answer tests and no fixtures for this path, and it cannot be built
here (Vulkan, glslc, Bazel and its fetched dependencies are absent). Each oracle function is therefore checked
against something it does not share code with: independent numpy restatements, closed forms and invariants,
brute force over engineered ties, published known-answer values, and a pure-Python GGUF parser.
"""
import os
import struct

import numpy as np
import pytest

from helpers import argmax_tie_rule, assert_fp16_close, bitrev5, rand

M64 = (1 << 64) - 1


# ---------------------------------------------------------------------------------------------------------------
# fp16 conversions: numpy's float16 cast is IEEE round-to-nearest-even
def test_f16_to_f32_exhaustive(oracle):
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([L.oracle_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even(oracle):
    L = oracle.lib()
    r = np.random.default_rng(0)
    xs = [r.standard_normal(20000).astype(np.float32) * 4, r.standard_normal(5000).astype(np.float32) * 1e-5,
          (r.standard_normal(2000) * 3e4).astype(np.float32)]
    # exact halfway points between neighbouring fp16 values, normal and subnormal, both parities
    h = np.arange(1, 65000, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(1, 65000, 97, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    mid = ((h + nxt) / 2).astype(np.float32)
    edge = np.float32([65504, 65519.99, 65520, 70000, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001, 2 ** -26, -0.0, np.inf,
                       -np.inf, 1 + 2 ** -11, 1 + 3 * 2 ** -11])
    x = np.concatenate(xs + [mid[np.isfinite(mid)], edge])
    got = np.array([L.oracle_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------------------------------------------
# synthetic inputs
def test_splitmix64_known_answers(oracle):
    """published SplitMix64 outputs for seed 1234567"""
    L = oracle.lib()
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    assert [L.oracle_splitmix64(1234567, n) for n in range(5)] == want


def _py_normal(stream, i):
    def sm(n):
        z = (stream + (n + 1) * 0x9E3779B97F4A7C15) & M64
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    s = sum((sm(3 * i + r) >> (16 * k)) & 0xFFFF for r in range(3) for k in range(4))
    return (s + 6 - 6 * 65536) / 65536.0


def test_normal_generator(oracle):
    L = oracle.lib()
    stream = L.oracle_tensor_stream(0, 5)
    for i in (0, 1, 2, 1000, 123456):
        assert L.oracle_normal(stream, i) == np.float32(_py_normal(stream, i))
    z = np.array([L.oracle_normal(stream, i) for i in range(200000)], dtype=np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert z.min() >= -6 and z.max() <= 6
    w = oracle.weights_f16(0, 5, 1000, 0.02).view(np.float16).astype(np.float32)
    zz = np.array([_py_normal(stream, i) for i in range(1000)], dtype=np.float32)
    assert np.array_equal(w.astype(np.float16), (zz * np.float32(0.02)).astype(np.float16))


def test_prompt_tokens(oracle):
    p = oracle.prompt_tokens(1, 64, 32000)
    assert p.min() >= 0 and p.max() < 32000 and len(set(p.tolist())) > 55


# ---------------------------------------------------------------------------------------------------------------
# operators
def ot(oracle, arr):
    return oracle.tensor(arr)


@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("shapes", [((1, 1), (1, 1)), ((4, 1), (4, 1)), ((1, 1), (4, 1)), ((1, 4), (4, 1)),
                                    ((2, 4), (2, 4)), ((1, 1), (2, 3))])
@pytest.mark.parametrize("M,K,N", [(1, 64, 48), (7, 33, 5), (16, 128, 64)])
def test_matmul_vs_numpy(oracle, tb, shapes, M, K, N):
    (Ba, Ca), (Bb, Cb) = shapes
    a = rand((Ba, Ca, M, K), np.float16, seed=1)
    b = rand((Bb, Cb, N, K) if tb else (Bb, Cb, K, N), np.float16, seed=2)
    if not tb and K == N:
        return
    out = np.zeros((max(Ba, Bb), max(Ca, Cb), M, N), np.float16)
    assert oracle.matmul(ot(oracle, a), ot(oracle, b), ot(oracle, out), 0.5, 0) == 0
    bb = b if not tb else np.swapaxes(b, 2, 3)
    want = (np.matmul(a.astype(np.float64), bb.astype(np.float64)).astype(np.float32) * np.float32(0.5))
    assert np.array_equal(out.view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_matmul_silu(oracle):
    a = rand((1, 1, 9, 40), np.float32, seed=3)
    b = rand((1, 1, 11, 40), np.float32, seed=4)
    out = np.zeros((1, 1, 9, 11), np.float32)
    assert oracle.matmul(ot(oracle, a), ot(oracle, b), ot(oracle, out), 1.0, 1) == 0
    v = a[0, 0].astype(np.float64) @ b[0, 0].T.astype(np.float64)
    np.testing.assert_allclose(out[0, 0], v / (1 + np.exp(-v)), rtol=1e-6, atol=1e-7)


def test_is_transposed_b_rule(oracle):
    """scores are always [N,K]-stored; attn.V only when kv == head_dim (src/core/vkllm_op_matmul.c:14-24)"""
    hd = 48
    z = np.zeros(1, np.float16)

    def t(shape):
        return oracle.tensor(z, shapes=list(shape), strides=[0, 0, 0, 0])

    for kv in (1, 16, 47, 48, 49, 256):
        assert oracle.is_transposed_b(t((1, 6, 1, hd)), t((1, 6, kv, hd)), t((1, 6, 1, kv)))
        assert oracle.is_transposed_b(t((1, 6, 1, kv)), t((1, 6, kv, hd)), t((1, 6, 1, hd))) == (kv == hd)


def test_rmsnorm_closed_form(oracle):
    x = rand((2, 3, 5, 288), np.float16, -3, 3, seed=5)
    w = rand((1, 1, 1, 288), np.float32, 0.5, 2, seed=6)
    out = np.zeros_like(x)
    assert oracle.rmsnorm(ot(oracle, x), ot(oracle, w), ot(oracle, out), 1e-5) == 0
    xd = x.astype(np.float64)
    alpha = (1.0 / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-5)).astype(np.float32)
    want = ((x.astype(np.float32) * w) * alpha).astype(np.float16)
    assert_fp16_close(out, want, max_ulp=1.0, frac_exact=0.999)
    ones = np.ones_like(w)
    assert oracle.rmsnorm(ot(oracle, x), ot(oracle, ones), ot(oracle, out), 0.0) == 0
    rms = np.sqrt((out.astype(np.float64) ** 2).mean(-1))
    assert np.max(np.abs(rms - 1)) < 2e-3


@pytest.mark.parametrize("offset", [0, 7, 4095])
def test_rope_vs_complex_rotation(oracle, offset):
    H, S, D = 3, 5, 64
    x = rand((1, H, S, D), np.float16, -2, 2, seed=7)
    out = np.zeros_like(x)
    assert oracle.rope(ot(oracle, x), ot(oracle, out), offset, 10000.0, False) == 0
    xd = x.astype(np.float64)
    z = xd[..., 0::2] + 1j * xd[..., 1::2]
    w = np.arange(D // 2)
    # the reference computes the angle in fp32: float(pos) / float(base^(2w/D))
    pos = (offset + np.arange(S)[:, None]).astype(np.float32)
    freq = (10000.0 ** (2 * w / D)).astype(np.float32)
    theta = (pos / freq).astype(np.float64)
    r = z * np.exp(1j * theta)
    want = np.empty_like(xd)
    want[..., 0::2] = r.real
    want[..., 1::2] = r.imag
    want = want.astype(np.float16)
    assert_fp16_close(out, want, max_ulp=1.0, frac_exact=0.99, atol=4e-7 * float(np.abs(x).max()))
    if offset == 0:
        assert np.array_equal(out[:, :, 0].view(np.uint16), x[:, :, 0].view(np.uint16))  # position 0: identity
    n_in = (xd[..., 0::2] ** 2 + xd[..., 1::2] ** 2)
    n_out = (out.astype(np.float64)[..., 0::2] ** 2 + out.astype(np.float64)[..., 1::2] ** 2)
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-3)) < 4e-3  # rotations keep pair norms


def test_rope_neox_is_permuted_normal(oracle):
    """NeoX rotates (w, w + D/2); on the de-interleaved input it must equal the normal style exactly"""
    D = 32
    x = rand((1, 2, 3, D), np.float16, seed=8)
    inter = np.empty_like(x)
    inter[..., 0::2] = x[..., : D // 2]
    inter[..., 1::2] = x[..., D // 2:]
    a = np.zeros_like(x)
    b = np.zeros_like(x)
    assert oracle.rope(ot(oracle, x), ot(oracle, a), 3, 10000.0, True) == 0
    assert oracle.rope(ot(oracle, inter), ot(oracle, b), 3, 10000.0, False) == 0
    assert np.array_equal(a[..., : D // 2].view(np.uint16), b[..., 0::2].view(np.uint16))
    assert np.array_equal(a[..., D // 2:].view(np.uint16), b[..., 1::2].view(np.uint16))


def test_softmax_properties(oracle):
    x = rand((1, 4, 6, 40), np.float32, -5, 5, seed=9)
    out = np.zeros_like(x)
    assert oracle.softmax(ot(oracle, x), ot(oracle, out), 1, 10) == 0
    for h in range(6):
        lim = h + 10
        assert np.all(out[:, :, h, lim + 1:] == 0)
        xd = x[:, :, h, : lim + 1].astype(np.float64)
        e = np.exp(xd - x[:, :, h, :].max(-1, keepdims=True))
        np.testing.assert_allclose(out[:, :, h, : lim + 1], e / e.sum(-1, keepdims=True), rtol=2e-6, atol=1e-9)
        np.testing.assert_allclose(out[:, :, h].sum(-1), 1.0, rtol=1e-5)
    # the max runs over the whole row, masked entries included; results are unchanged up to rounding
    x2 = x.copy()
    x2[..., -1] = 80.0
    out2 = np.zeros_like(x)
    assert oracle.softmax(ot(oracle, x2), ot(oracle, out2), 1, 10) == 0
    np.testing.assert_allclose(out2[:, :, :5], out[:, :, :5], rtol=1e-5, atol=1e-30)


def test_copy_update_rows_embedding_bin(oracle):
    x = rand((2, 3, 4, 5), np.float16, seed=10)
    xt = np.transpose(x, (0, 2, 1, 3))
    out = np.zeros((2, 4, 3, 5), np.float16)
    assert oracle.copy(oracle.tensor(x, shapes=[2, 4, 3, 5], strides=[60, 5, 20, 1]), ot(oracle, out)) == 0
    assert np.array_equal(out, xt)
    cache = rand((1, 3, 10, 5), np.float16, seed=11)
    src = rand((1, 3, 2, 5), np.float16, seed=12)
    want = cache.copy()
    want[:, :, 6:8] = src
    assert oracle.update_rows(ot(oracle, src), ot(oracle, cache), 6) == 0
    assert np.array_equal(cache, want)
    assert oracle.update_rows(ot(oracle, src), ot(oracle, cache), 9) == -1
    table = rand((1, 1, 50, 8), np.float32, seed=13)
    ids = np.array([[[[3, 49, 50, 7, 1000]]]], np.uint32)
    emb = np.zeros((1, 1, 5, 8), np.float32)
    assert oracle.embedding(ot(oracle, ids), ot(oracle, table), ot(oracle, emb), 2) == 0
    assert np.array_equal(emb[0, 0], table[0, 0][[3, 49, 2, 7, 2]])
    a = rand((1, 2, 3, 4), np.float16, seed=14)
    b = rand((1, 2, 3, 4), np.float16, 0.5, 1, seed=15)
    for op, f in enumerate([np.add, np.subtract, np.multiply, np.divide]):
        o = np.zeros((1, 2, 3, 4), np.float32)
        assert oracle.bin_op(ot(oracle, a), ot(oracle, b), ot(oracle, o), op) == 0
        assert np.array_equal(o, f(a.astype(np.float32), b.astype(np.float32)))


def test_arg_max_tie_rule(oracle):
    """the oracle's literal 32-lane scan against the bit-reversed-lane characterisation of the tie rule"""
    r = np.random.default_rng(16)
    for trial in range(300):
        W = int(r.choice([1, 5, 31, 32, 33, 64, 100, 1000, 32000]))
        x = r.integers(-3, 3, size=W).astype(np.float32)  # many ties
        x = x.reshape(1, 1, 1, W)
        out = np.zeros((1, 1, 1, 1), np.uint32)
        assert oracle.arg_max(ot(oracle, x), ot(oracle, out)) == 0
        assert int(out[0, 0, 0, 0]) == argmax_tie_rule(x[0, 0, 0])
    # without ties it is the plain arg max
    x = r.standard_normal(32000).astype(np.float32).reshape(1, 1, 1, -1)
    out = np.zeros((1, 1, 1, 1), np.uint32)
    oracle.arg_max(ot(oracle, x), ot(oracle, out))
    assert int(out[0, 0, 0, 0]) == int(np.argmax(x))
    # ties at indices 1 and 16: lane 16 (bit-reversed 1) beats lane 1 (bit-reversed 16)
    x = np.zeros((1, 1, 1, 64), np.float32)
    x[..., 1] = x[..., 16] = 5
    oracle.arg_max(ot(oracle, x), ot(oracle, out))
    assert out[0, 0, 0, 0] == 16 and bitrev5(16) < bitrev5(1)


def test_ffn_up_and_gate(oracle):
    x = rand((1, 2, 3, 40), np.float32, seed=17)
    wu = rand((1, 1, 7, 40), np.float32, seed=18)
    wg = rand((1, 1, 7, 40), np.float32, seed=19)
    out = np.zeros((1, 2, 3, 7), np.float32)
    assert oracle.ffn_up_and_gate(ot(oracle, x), ot(oracle, wu), ot(oracle, wg), ot(oracle, out)) == 0
    u = x.astype(np.float64) @ wu[0, 0].T.astype(np.float64)
    g = x.astype(np.float64) @ wg[0, 0].T.astype(np.float64)
    np.testing.assert_allclose(out, u * g / (1 + np.exp(-g)), rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------------------------------------------------------
# GGUF: the oracle's writer checked with a pure-Python parser of the public GGUF v3 layout
def parse_gguf(path):
    with open(path, "rb") as f:
        buf = f.read()
    p = 0

    def take(fmt):
        nonlocal p
        v = struct.unpack_from(fmt, buf, p)
        p += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def string():
        n = take("<Q")
        nonlocal p
        s = buf[p: p + n].decode()
        p += n
        return s

    scalar = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        return take(scalar[t])

    assert buf[:4] == b"GGUF"
    p = 4
    version, nt, nkv = take("<I"), take("<Q"), take("<Q")
    kv = {}
    for _ in range(nkv):
        k = string()
        t = take("<I")
        kv[k] = (t, value(t))
    tensors = []
    for _ in range(nt):
        name = string()
        nd = take("<I")
        dims = [take("<Q") for _ in range(nd)]
        ty, off = take("<I"), take("<Q")
        tensors.append((name, dims, ty, off))
    align = kv.get("general.alignment", (4, 32))[1]
    data = (p + align - 1) // align * align
    return version, kv, tensors, buf, data


def test_gguf_writer_layout(oracle, tmp_path):
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=4, ffn=96, vocab=500, ctx=32)
    path = str(tmp_path / "m.gguf")
    oracle.write_gguf(path, cfg, 3)
    version, kv, tensors, buf, data = parse_gguf(path)
    assert version == 3
    assert kv["llama.block_count"] == (4, 2) and kv["llama.embedding_length"] == (4, 64)
    assert kv["llama.attention.head_count"] == (4, 4) and kv["llama.context_length"] == (4, 32)
    assert kv["llama.attention.layer_norm_rms_epsilon"][0] == 6
    assert abs(kv["llama.attention.layer_norm_rms_epsilon"][1] - 1e-5) < 1e-12
    assert kv["tokenizer.ggml.tokens"][0] == 9 and len(kv["tokenizer.ggml.tokens"][1]) == 500
    assert kv["tokenizer.ggml.tokens"][1][:3] == ["<unk>", "<s>", "</s>"]
    names = [t[0] for t in tensors]
    assert names[0] == "token_embd.weight" and names[-1] == "output.weight" and len(names) == 9 * 2 + 3
    byname = {t[0]: t for t in tensors}
    assert byname["blk.1.ffn_down.weight"][1] == [96, 64] and byname["blk.1.ffn_down.weight"][2] == 1
    assert byname["blk.0.attn_norm.weight"][1] == [64] and byname["blk.0.attn_norm.weight"][2] == 0
    for i, (name, dims, ty, off) in enumerate(tensors):
        assert off % 32 == 0
        n = int(np.prod(dims))
        if ty == 0:
            v = np.frombuffer(buf, np.float32, n, data + off)
            assert np.all(v == 1.0)
        else:
            v = np.frombuffer(buf, np.uint16, n, data + off)
            idx = [0, n // 2, n - 1]
            assert v[idx].tolist() == [oracle.lib().oracle_weight_f16(3, i, j, 0.02) for j in idx]
    m = oracle.Model(path)
    r = oracle.Model(cfg=cfg, seed=3)
    for tid in range(len(tensors)):
        if byname[names[tid]][2] == 1:
            assert np.array_equal(m.weight(tid), r.weight(tid))


# ---------------------------------------------------------------------------------------------------------------
# model: an independent float64 numpy LLaMA-2 with the reference's conventions (GPT-J pair RoPE, causal softmax,
# up * silu(gate), the kv == head_dim transposition) against the oracle's fp16-rounded graph
def np_llama(weights, cfg, toks):
    D, H, L = cfg.dim, cfg.n_head, cfg.n_layer
    hd = D // H
    W = lambda i, shape: weights(i).view(np.float16).astype(np.float64).reshape(shape)
    emb = W(0, (cfg.vocab, D))
    x = emb[np.where(np.asarray(toks) < cfg.vocab, toks, cfg.pad_id)]
    S = len(toks)

    def norm(v):
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + cfg.eps)

    pos = np.arange(S)[:, None]
    theta = pos / (cfg.theta ** (2 * np.arange(hd // 2) / hd))

    def rope(m):  # [S, H, hd]
        z = m[..., 0::2] + 1j * m[..., 1::2]
        r = z * np.exp(1j * theta)[:, None, :]
        out = np.empty_like(m)
        out[..., 0::2], out[..., 1::2] = r.real, r.imag
        return out

    for l in range(L):
        b = 1 + 9 * l
        xn = norm(x)
        q = rope((xn @ W(b + 1, (D, D)).T).reshape(S, H, hd))
        k = rope((xn @ W(b + 2, (D, D)).T).reshape(S, H, hd))
        v = (xn @ W(b + 3, (D, D)).T).reshape(S, H, hd)
        att = np.zeros((S, H, hd))
        for h in range(H):
            sc = q[:, h] @ k[:, h].T / np.sqrt(hd)
            sc = np.where(np.tril(np.ones((S, S))) > 0, sc, -np.inf)
            p = np.exp(sc - sc.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            att[:, h] = p @ (v[:, h].T if S == hd else v[:, h])
        x = x + att.reshape(S, D) @ W(b + 4, (D, D)).T
        xn = norm(x)
        g = xn @ W(b + 6, (cfg.ffn, D)).T
        u = xn @ W(b + 7, (cfg.ffn, D)).T
        x = x + (u * g / (1 + np.exp(-g))) @ W(b + 8, (D, cfg.ffn)).T
    return norm(x) @ W(2 + 9 * L, (cfg.vocab, D)).T


@pytest.mark.parametrize("S", [1, 5, 16])
def test_oracle_model_vs_float64(oracle, S):
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=4, ffn=96, vocab=300, ctx=64)
    m = oracle.Model(cfg=cfg, seed=4)
    toks = oracle.prompt_tokens(5, S, cfg.vocab)
    ids, logits, _ = m.step(toks, 0, want_logits=True)
    want = np_llama(m.weight, cfg, toks)
    assert np.max(np.abs(logits.astype(np.float64) - want)) < 2e-2
    assert np.corrcoef(logits.astype(np.float64).ravel(), want.ravel())[0, 1] > 0.999


def test_oracle_model_transposition_at_kv_equal_head_dim(oracle):
    """S == head_dim triggers attn . V^T in the oracle exactly as in the float64 restatement"""
    cfg = oracle.make_cfg(n_layer=1, dim=64, n_head=4, ffn=96, vocab=300, ctx=64)  # head_dim 16
    m = oracle.Model(cfg=cfg, seed=6)
    toks = oracle.prompt_tokens(7, 16, cfg.vocab)
    _, logits, _ = m.step(toks, 0, want_logits=True)
    want = np_llama(m.weight, cfg, toks)
    assert np.max(np.abs(logits.astype(np.float64) - want)) < 2e-2


def test_oracle_kv_cache_consistency(oracle):
    """decode steps over the cache reproduce the logits of one longer prefill (rounding-level differences only)"""
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=4, ffn=96, vocab=300, ctx=64)
    toks = oracle.prompt_tokens(8, 12, cfg.vocab)
    a = oracle.Model(cfg=cfg, seed=9)
    _, full, _ = a.step(toks, 0, want_logits=True)
    b = oracle.Model(cfg=cfg, seed=9)
    b.step(toks[:6], 0)
    rows = []
    for i in range(6, 12):
        _, lg, _ = b.step(toks[i:i + 1], i, want_logits=True)
        rows.append(lg[0])
    assert np.max(np.abs(np.stack(rows).astype(np.float32) - full[6:].astype(np.float32))) < 1e-2


def test_oracle_token_loop_tiny_deterministic(oracle, tiny_gguf):
    m = oracle.Model(tiny_gguf)
    p = oracle.prompt_tokens(1, 16, 32000)
    a, _ = m.token_loop(p, 8)
    m2 = oracle.Model(tiny_gguf)
    b, _ = m2.token_loop(p, 8)
    assert a.tolist() == b.tolist()


# ---------------------------------------------------------------------------------------------------------------
# the token loop (tests/vkllm_test_infer_gguf.c:181-272): step 0 runs the whole prompt at offset 0, every later step
# the previous step's output id at offset += S (:255-269); the id fed back is the LAST row's (extract_output_tok,
# :100-120)
def chained_steps(m, prompt, n_steps):
    """The driver's protocol written out with explicit oracle_model_step calls."""
    toks, offset, ids, logits = np.asarray(prompt, np.uint32), 0, [], []
    for _ in range(n_steps):
        out, lg, _ = m.step(toks, offset, want_logits=True)
        ids.append(int(out[len(toks) - 1]))
        logits.append(lg[len(toks) - 1])
        offset += len(toks)
        toks = np.array([ids[-1]], np.uint32)
    return np.array(ids, np.uint32), np.stack(logits)


@pytest.mark.parametrize("prompt_len", [1, 7])
def test_oracle_token_loop_equals_chained_steps(oracle, prompt_len):
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=4, ffn=96, vocab=300, ctx=64)
    prompt = oracle.prompt_tokens(21, prompt_len, cfg.vocab)
    a = oracle.Model(cfg=cfg, seed=12)
    ids, logits = a.token_loop(prompt, 12, want_logits=True)
    b = oracle.Model(cfg=cfg, seed=12)
    want_ids, want_logits = chained_steps(b, prompt, 12)
    assert ids.tolist() == want_ids.tolist()
    assert np.array_equal(logits.view(np.uint16), want_logits.view(np.uint16))


def test_oracle_token_loop_vs_float64_recompute(oracle):
    """Teacher-forced against a float64 LLaMA-2 that recomputes the whole sequence (prompt + ids so far) at every
    step, with no KV cache: the loop's logits for step t must be the float64 model's last-row logits for that
    sequence (within 2e-2), and each id its arg max (or, at a float64 top-2 gap under 2e-2, one of the two). A loop
    that fed back another row's id, advanced the offset wrongly or re-used a stale cache row fails this.
    Two heads of 32 keep kv below head_dim: at kv == head_dim the reference's shape rule transposes attn . V for
    that one step (src/core/vkllm_op_matmul.c:14-24), which a whole-sequence recompute cannot reproduce."""
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=2, ffn=96, vocab=300, ctx=64)
    m = oracle.Model(cfg=cfg, seed=13)
    prompt = oracle.prompt_tokens(22, 9, cfg.vocab)
    n = 10
    ids, logits = m.token_loop(prompt, n, want_logits=True)
    seq = list(map(int, prompt))
    for t in range(n):
        want = np_llama(m.weight, cfg, np.array(seq, np.int64))[-1]
        err = np.max(np.abs(logits[t].astype(np.float64) - want))
        assert err < 2e-2, f"step {t}: logits differ from the float64 recompute by {err}"
        top = np.sort(want)[::-1]
        if top[0] - top[1] >= 2e-2:
            assert int(ids[t]) == int(np.argmax(want)), f"step {t}: id {ids[t]} != {np.argmax(want)}"
        else:
            assert int(ids[t]) in np.argsort(want)[::-1][:2].tolist()
        seq.append(int(ids[t]))


def test_oracle_token_loop_planted_offset_error_is_caught(oracle):
    """The float64 recompute detects a loop that advances the offset by one position too many: the same chain with
    offset += S + 1 gives logits far from the float64 model's (the check above is not blind to the offset)."""
    cfg = oracle.make_cfg(n_layer=2, dim=64, n_head=2, ffn=96, vocab=300, ctx=64)
    m = oracle.Model(cfg=cfg, seed=13)
    prompt = oracle.prompt_tokens(22, 9, cfg.vocab)
    toks, offset, seq, worst = prompt, 0, list(map(int, prompt)), 0.0
    for _ in range(6):
        out, lg, _ = m.step(toks, offset, want_logits=True)
        if offset:
            want = np_llama(m.weight, cfg, np.array(seq, np.int64))[-1]
            worst = max(worst, float(np.max(np.abs(lg[-1].astype(np.float64) - want))))
        offset += len(toks) + 1  # the planted mistake
        seq.append(int(out[-1]))
        toks = np.array([seq[-1]], np.uint32)
    assert worst > 2e-2  # the recompute check's tolerance


# ---------------------------------------------------------------------------------------------------------------
# the fp32 mode's two summation orders (oracle_set_accumulation): double sums, or sequential fp32 sums
def _zero_layer_model(path, out_rows, dim=64, n_head=2, ffn=64):
    """A one-layer GGUF whose projection weights are all zero, so the residual stream stays the embedding row; the
    embedding rows are all 1.0 (RMSNorm of such a row is exactly 1.0 in fp16), so logit n is the plain sum of output
    row n, added in index order by the sequential mode."""
    import gguf_util as G

    V = len(out_rows)
    z = lambda r, c: np.zeros((r, c), np.float16)
    ones32 = np.ones(dim, np.float32)
    kvs = [("general.architecture", G.STRING, "llama"), ("llama.block_count", G.U32, 1),
           ("llama.context_length", G.U32, 8), ("llama.embedding_length", G.U32, dim),
           ("llama.feed_forward_length", G.U32, ffn), ("llama.attention.head_count", G.U32, n_head),
           ("llama.attention.head_count_kv", G.U32, n_head), ("llama.attention.layer_norm_rms_epsilon", G.F32, 1e-5),
           ("llama.rope.freq_base", G.F32, 10000.0), ("llama.vocab_size", G.U32, V)]
    out = np.zeros((V, dim), np.float16)
    for n, row in enumerate(out_rows):
        out[n, :len(row)] = row
    tensors = [("token_embd.weight", [dim, V], G.GGML_F16, np.ones((V, dim), np.float16)),
               ("blk.0.attn_norm.weight", [dim], G.GGML_F32, ones32)]
    tensors += [(f"blk.0.{n}.weight", [dim, dim], G.GGML_F16, z(dim, dim)) for n in ("attn_q", "attn_k", "attn_v",
                                                                                        "attn_output")]
    tensors += [("blk.0.ffn_norm.weight", [dim], G.GGML_F32, ones32),
                ("blk.0.ffn_gate.weight", [dim, ffn], G.GGML_F16, z(ffn, dim)),
                ("blk.0.ffn_up.weight", [dim, ffn], G.GGML_F16, z(ffn, dim)),
                ("blk.0.ffn_down.weight", [ffn, dim], G.GGML_F16, z(dim, ffn)),
                ("output_norm.weight", [dim], G.GGML_F32, ones32), ("output.weight", [dim, V], G.GGML_F16, out)]
    G.write(str(path), kvs, tensors)


def test_sequential_fp32_accumulation_known_answers(oracle, tmp_path):
    """32768 + 2^-10 rounds back to 32768 in fp32 (2^-10 is under half of 32768's fp32 spacing 2^-8), so a
    sequential fp32 sum of [32768, 2^-10, -32768] is 0 while the double sum is 2^-10; in the order
    [32768, -32768, 2^-10] both give 2^-10; a sum that never leaves fp32's exact range agrees in both."""
    t = 2.0 ** -10
    rows = [[32768, t, -32768], [32768, -32768, t], [1.0] * 64, [0.5, 0.25, 0.125]]
    path = tmp_path / "zero_layer.gguf"
    _zero_layer_model(path, rows)
    got = {}
    for mode in (False, True):
        oracle.set_accumulation(mode)
        try:
            m = oracle.Model(str(path))
            _, logits, _ = m.step(np.array([0], np.uint32), 0, want_logits=True)
            m.close()
        finally:
            oracle.set_accumulation(False)
        got[mode] = logits[0].astype(np.float64)
    assert got[False].tolist() == [t, t, 64.0, 0.875]
    assert got[True].tolist() == [0.0, t, 64.0, 0.875]


def test_sequential_fp32_order_is_the_same_graph(oracle):
    """The two orders differ only by fp32 rounding: over two layers at a small width their logits agree within the
    2e-2 bar but not bit for bit (the switch reaches the model step)."""
    cfg = oracle.make_cfg(n_layer=2, dim=256, n_head=4, ffn=512, vocab=500, ctx=64)
    toks = oracle.prompt_tokens(3, 24, cfg.vocab)
    out = {}
    for mode in (False, True):
        oracle.set_accumulation(mode)
        try:
            m = oracle.Model(cfg=cfg, seed=11)
            _, out[mode], _ = m.step(toks, 0, want_logits=True)
            m.close()
        finally:
            oracle.set_accumulation(False)
    d = np.abs(out[True].astype(np.float64) - out[False].astype(np.float64))
    assert 0 < d.max() < 2e-2
