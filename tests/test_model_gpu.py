"""The LLaMA-2 token loop on the GPU through the C API (tests/vkllm_test_infer_gguf.c:173-272), against the oracle.

Workload: the tiny LLaMA-2 (dim 288, 6 layers, 6 heads of 48, FFN 768, vocab 32000, ctx 256) from the seeded
random-init GGUF, a 16-token prompt from seed 1, 64 greedy steps. Bar: identical greedy ids, logits within 2e-2.
"""
import numpy as np
import pytest

from helpers import assert_prefill_ids

pytestmark = pytest.mark.gpu

N_STEPS = 64
LOGIT_TOL = 2e-2


@pytest.fixture(scope="module")
def reference_run(oracle, tiny_gguf):
    m = oracle.Model(tiny_gguf)
    prompt = oracle.prompt_tokens(1, 16, m.cfg.vocab)
    ids, logits = m.token_loop(prompt, N_STEPS, want_logits=True)
    m.close()
    return prompt, ids, logits


def _run(ctx, vk, path, prompt, mode, replay=True):
    ctx.set_exec_mode(mode)
    ctx.set_graph_replay(replay)
    model = vk.Model(ctx, path=path)
    try:
        if mode == vk.EXEC_FUSED:
            return model.token_loop(prompt, N_STEPS, want_logits=True)
        ids, _ = model.token_loop(prompt, N_STEPS)
        return ids, None
    finally:
        model.close()
        ctx.set_exec_mode(vk.EXEC_FUSED)
        ctx.set_graph_replay(True)


def test_token_loop_fused_matches_oracle(ctx, vk, tiny_gguf, reference_run):
    prompt, want_ids, want_logits = reference_run
    ids, logits = _run(ctx, vk, tiny_gguf, prompt, vk.EXEC_FUSED)
    err = np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32)), axis=1)
    print(f"fused: max|dlogit| per step max {err.max():.3g} mean {err.mean():.3g}")
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


def test_token_loop_nodes_matches_oracle(ctx, vk, tiny_gguf, reference_run):
    """node-by-node execution of the same graphs through the VKLLM_OP_* kernels"""
    prompt, want_ids, _ = reference_run
    ids, _ = _run(ctx, vk, tiny_gguf, prompt, vk.EXEC_NODES)
    assert ids.tolist() == want_ids.tolist()


def test_graph_replay_matches_direct_launches(ctx, vk, tiny_gguf, reference_run):
    prompt, _, _ = reference_run
    a, la = _run(ctx, vk, tiny_gguf, prompt, vk.EXEC_FUSED, replay=True)
    b, lb = _run(ctx, vk, tiny_gguf, prompt, vk.EXEC_FUSED, replay=False)
    assert a.tolist() == b.tolist()
    assert np.array_equal(la.view(np.uint16), lb.view(np.uint16))


def test_prefill_at_kv_equal_head_dim(ctx, vk, oracle, tiny_gguf):
    """A 48-token prompt makes kv == head_dim for the whole prefill: attn . V^T (src/core/vkllm_op_matmul.c:14-24)."""
    m = oracle.Model(tiny_gguf)
    prompt = oracle.prompt_tokens(2, 48, m.cfg.vocab)
    want_ids, want_logits, _ = m.step(prompt, 0, want_logits=True)
    m.close()
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        ids = model.step(prompt, 0)
        logits = model.last_logits(48)
    finally:
        model.close()
    assert np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32))) <= LOGIT_TOL
    assert_prefill_ids(ids, want_ids, want_logits, "48-row prefill")


def test_init_random_equals_gguf(ctx, vk, oracle, tiny_gguf):
    """device-side random init (no file) gives the same weights as the GGUF written by the oracle"""
    cfg = vk.llama_config(6, 288, 6, 768, vocab=32000, ctx=256)
    a = vk.Model(ctx, path=tiny_gguf)
    b = vk.Model(ctx, config=cfg, seed=0)
    try:
        for getter in (lambda m: m.weights.tok_embed_weights, lambda m: m.weights.output_weight,
                       lambda m: m.weights.blocks.contents.data[0].contents.WQ,
                       lambda m: m.weights.blocks.contents.data[5].contents.WD,
                       lambda m: m.weights.blocks.contents.data[3].contents.WG,
                       lambda m: m.weights.blocks.contents.data[3].contents.ffn_norm_weight):
            ta, tb = getter(a.m), getter(b.m)
            n = int(np.prod(list(ta.contents.shapes))) * (4 if ta.contents.dtype == vk.F32 else 2)
            da, db = ctx.download_raw(ta, n), ctx.download_raw(tb, n)
            assert np.array_equal(da, db)
        prompt = oracle.prompt_tokens(1, 16, 32000)
        assert a.step(prompt, 0).tolist() == b.step(prompt, 0).tolist()
    finally:
        a.close()
        b.close()


def test_graph_structure_matches_reference(ctx, vk, tiny_gguf):
    """build_graph creates the reference's nodes: 23*L + 5 of them, names and ops in order
    (src/models/vkllm_models_llama2.c:488-602, src/models/vkllm_llama2_layers.c:98-340)."""
    import ctypes

    L = vk.lib()
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        inp = ctx.tensor([1, 1, 1, 3], vk.U32, "input_toks", mapped=True)
        g = ctypes.POINTER(vk.Graph)()
        vk.check("graph_new", L.vkllm_graph_new(ctx.vp, ctypes.byref(g)))
        vk.check("build", L.vkllm_models_llama2_build_graph(ctx.vp, ctypes.byref(model.m), inp, g, 5))
        nodes = g.contents.nodes.contents
        names = [nodes.data[i].contents.name.decode() for i in range(nodes.used_n)]
        ops = [nodes.data[i].contents.op for i in range(nodes.used_n)]
        assert len(names) == 23 * 6 + 5
        assert names[:4] == ["input_toks", "embedded", "block.0.attn.norm", "block.0.attn.Q"]
        blk = names[2:25]
        assert blk == ["block.0.attn.norm", "block.0.attn.Q", "block.0.attn.K", "block.0.attn.V",
                       "block.0.attn.Q_ref", "block.0.attn.K_ref", "block.0.attn.V_ref", "block.0.attn.RQ",
                       "block.0.attn.RK", "block.0.attn.scores", "block.0.attn.attn_weights", "block.0.attn",
                       "block.0.attn_ref", "block.0.attn.concated_heads", "block.0.attn.concated_heads_ref",
                       "block.0.attn.final_output", "block.0.attn.final_output_add", "block.0.ffn.norm",
                       "block.0.ffn.up", "block.0.ffn.gate", "block.0.ffn.mul", "block.0.ffn.down",
                       "block.0.ffn.add"]
        assert names[-3:] == ["output_norm", "logits", "output"]
        assert ops[-1] == vk.OP_ARG_MAX and ops[-2] == vk.OP_MATMUL
        out = g.contents.output_node.contents
        assert list(out.shapes) == [1, 1, 3, 1] and out.dtype == vk.U32 and out.data.mapped
        scores = nodes.data[11].contents
        assert list(scores.shapes) == [1, 6, 3, 8]  # key_num = offset + S
        vk.check("graph_free", L.vkllm_graph_free(ctx.vp, g))
    finally:
        model.close()


def test_tokenizer(ctx, vk, tiny_gguf):
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        ids = model.tokenize("Q: What is the largest animal? A:")
        texts = [model.meta.tokens.contents.data[i].text.decode() for i in ids[1:]]
        assert ids[0] == model.meta.bos_token_id
        assert "".join(texts).replace("▁", " ") == " Q: What is the largest animal? A:"
        assert model.tokenize("") == []
    finally:
        model.close()


def _gpu_vs_oracle(ctx, vk, oracle, shape, seed, prompt_len, n_steps, prompt_seed):
    """Greedy loop of a device-initialised model against the oracle's loop on the same seeded weights."""
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=seed)
    prompt = oracle.prompt_tokens(prompt_seed, prompt_len, cfg.vocab)
    want_ids, want_logits = ref.token_loop(prompt, n_steps, want_logits=True)
    ref.close()
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=seed)
    try:
        ids, logits = model.token_loop(prompt, n_steps, want_logits=True)
    finally:
        model.close()
    err = np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32)), axis=1)
    print(f"max|dlogit| per step max {err.max():.3g} mean {err.mean():.3g}")
    return ids, want_ids, err


def test_7b_widths_two_layers(ctx, vk, oracle):
    """The LLaMA-2-7B widths (dim 4096, 32 heads of 128, FFN 11008, vocab 32000) on two layers: the decode GEMVs,
    attention and logits at their real shapes. 8-token prefill, then 6 greedy steps."""
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=64)
    ids, want_ids, err = _gpu_vs_oracle(ctx, vk, oracle, shape, seed=3, prompt_len=8, n_steps=6, prompt_seed=4)
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


@pytest.mark.parametrize("dim,heads,ffn", [(4096, 32, 11008), (5120, 40, 13824)], ids=["7b", "13b"])
def test_300_token_prompt_at_real_widths(ctx, vk, oracle, dim, heads, ffn):
    """A 300-token prompt at the 7B and 13B widths (one layer, vocabulary 1000 to keep the oracle quick): the down
    product (K 11008 / 13824) splits K 8 / 6 ways over one round of 256 x 256 tiles, and the reduce adds the residual
    and the next RMSNorm. Every prompt row against the oracle (logits within 2e-2, ids identical but at one-ulp
    ties), then 3 decode steps fed the oracle's ids (free-running streams part at the first one-ulp tie: with seed 13
    the 13B widths have one at the first decode step, top-2 logits 0.0039 apart)."""
    from test_long_gpu import _forced_decode

    shape = dict(n_layer=1, dim=dim, n_head=heads, ffn=ffn, vocab=1000, ctx=320)
    cfg = oracle.make_cfg(**shape)
    ref = oracle.Model(cfg=cfg, seed=13)
    model = vk.Model(ctx, config=vk.llama_config(1, dim, heads, ffn, 1000, 320), seed=13)
    try:
        prompt = oracle.prompt_tokens(14, 300, cfg.vocab)
        want_ids, want_logits, _ = ref.step(prompt, 0, want_logits=True)
        ids = model.step(prompt, 0)
        err = float(np.max(np.abs(model.last_logits(300).astype(np.float32) - want_logits.astype(np.float32))))
        print(f"[300-token prompt] max|dlogit| {err:.3g}")
        assert err <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, "300-token prompt")
        worst, ties = _forced_decode(ref, model, want_ids[-1], 300, 3)
        print(f"[decode] max|dlogit| {worst:.3g}, {ties} one-ulp ties")
        assert ties <= 1
    finally:
        ref.close()
        model.close()


@pytest.mark.parametrize("small_max,long_one", [("1536", "1"), ("512", "1"), ("512", "0")])
def test_long_context_decode(ctx, vk, oracle, monkeypatch, small_max, long_one):
    """Decode at kv 1001..1008 (head_dim 128, a 1000-token prompt, 8 steps). With the one-kernel attention admitted
    up to 1536 positions the blocks hold 4 passes of V rows; capped at 512 the step takes the long-cache path:
    8 chunks of 256 positions per head, merged by the last chunk's block, in one launch or in two."""
    monkeypatch.setenv("VKLLM_ATTN_SMALL_MAX", small_max)
    monkeypatch.setenv("VKLLM_ATTN_LONG", long_one)
    monkeypatch.setenv("VKLLM_PERSIST", "0")  # the separate attention kernels (the persistent step has its own tests)
    shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=2048)
    ids, want_ids, err = _gpu_vs_oracle(ctx, vk, oracle, shape, seed=5, prompt_len=1000, n_steps=8, prompt_seed=6)
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


def _device_loop(ctx, vk, shape, seed, prompt, n_steps):
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=seed)
    try:
        return model.token_loop(prompt, n_steps, want_logits=True)
    finally:
        model.close()


def test_attention_and_projection_in_one_launch(ctx, vk, monkeypatch):
    """The one-kernel attention followed by Wo + residual inside the same launch (projection workgroups wait for
    the attention workgroups) against the two separate launches, at the 7B widths: identical ids and logits."""
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160)
    prompt = vk.prompt_tokens(8, 20, shape["vocab"])
    monkeypatch.setenv("VKLLM_PERSIST", "0")
    monkeypatch.setenv("VKLLM_ATTN_O", "1")
    ids_a, logits_a = _device_loop(ctx, vk, shape, 7, prompt, 24)
    monkeypatch.setenv("VKLLM_ATTN_O", "0")
    ids_b, logits_b = _device_loop(ctx, vk, shape, 7, prompt, 24)
    assert ids_a.tolist() == ids_b.tolist()
    assert np.array_equal(logits_a.view(np.uint16), logits_b.view(np.uint16))


def test_arg_max_in_the_vocabulary_product(ctx, vk, monkeypatch):
    """A single-token step's arg max in the vocabulary product's epilogue (each workgroup publishes its best, the last
    to finish reduces them) against the separate ARG_MAX kernel and the reference's tie rule
    (src/shaders/vkllm_arg_max.comp:40-97), with exact ties spread over the vocabulary: the output weights are zero
    except rows +u at 5, 37, 70, 12345, 31999 and -u at 3, 35, 99, 20000, 31998 (u = 0.01 in every column), so one of
    the two sets holds the row's maximum five times; the rule then picks 70 or 20000, neither the smallest tied
    index. Identical ids and logits on both paths."""
    from helpers import argmax_tie_rule

    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160)
    prompt = vk.prompt_tokens(11, 20, shape["vocab"])
    plus, minus = [5, 37, 70, 12345, 31999], [3, 35, 99, 20000, 31998]
    w = np.zeros((shape["vocab"], shape["dim"]), np.float16)
    w[plus] = 0.01
    w[minus] = -0.01

    monkeypatch.setenv("VKLLM_PERSIST", "0")

    def run(epi):
        monkeypatch.setenv("VKLLM_ARGMAX_EPI", epi)
        vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                               shape["ctx"])
        model = vk.Model(ctx, config=vcfg, seed=7)
        try:
            ctx.upload(model.m.weights.output_weight, w)
            return model.token_loop(prompt, 6, want_logits=True)
        finally:
            model.close()

    ids_a, logits_a = run("1")
    ids_b, logits_b = run("0")
    assert ids_a.tolist() == ids_b.tolist()
    assert np.array_equal(logits_a.view(np.uint16), logits_b.view(np.uint16))
    for step in range(1, 6):  # the decode steps (step 0 is the prompt's last row)
        row = logits_a[step].astype(np.float32)
        tied = np.nonzero(row == row.max())[0].tolist()
        assert tied in (plus, minus), tied
        assert int(ids_a[step]) == argmax_tie_rule(row) and int(ids_a[step]) in (70, 20000)


@pytest.mark.parametrize("prompt_len", [100, 300, 1030])
def test_qkv_rope_epilogue_matches_separate_kernel(ctx, vk, monkeypatch, prompt_len):
    """RoPE and the K/V append in the prompt step's QKV product epilogue against the stored product and the separate
    RoPE kernel (src/shaders/vkllm_rope.comp, src/shaders/vkllm_update_rows.comp), at the 7B widths: the split-K reduce
    (100 tokens), 128 x 128 tiles (300) and 256 x 256 tiles with a ragged last row block (1030), then decode steps
    reading the appended cache; identical ids and logits."""
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=1100)
    prompt = vk.prompt_tokens(9, prompt_len, shape["vocab"])
    # both arms on the tile GEMMs (the streamed short-prompt products need the epilogue and sum in another order)
    monkeypatch.setenv("VKLLM_PREFILL_TILED", "0")
    monkeypatch.setenv("VKLLM_ROPE_EPI", "1")
    ids_a, logits_a = _device_loop(ctx, vk, shape, 7, prompt, 4)
    monkeypatch.setenv("VKLLM_ROPE_EPI", "0")
    ids_b, logits_b = _device_loop(ctx, vk, shape, 7, prompt, 4)
    assert ids_a.tolist() == ids_b.tolist()
    assert np.array_equal(logits_a.view(np.uint16), logits_b.view(np.uint16))


@pytest.mark.parametrize("prompt_len,dim", [(20, 4096), (100, 4096), (100, 5120)])
def test_norm_in_split_k_reduce_matches_separate_pass(ctx, vk, monkeypatch, prompt_len, dim):
    """The residual add and the next RMSNorm in one pass over the split-K partials of Wo and Wd (prompts of at most
    128 tokens split K) against the reduce followed by the separate RMSNorm, at the 7B widths (one 16-byte vector
    per thread) and the 13B widths (two for some threads): identical ids and logits."""
    heads, ffn = {4096: (32, 11008), 5120: (40, 13824)}[dim]
    shape = dict(n_layer=2, dim=dim, n_head=heads, ffn=ffn, vocab=32000, ctx=160)
    prompt = vk.prompt_tokens(10, prompt_len, shape["vocab"])
    # both arms on the tile GEMMs (the streamed short-prompt products need the fused norm and sum in another order)
    monkeypatch.setenv("VKLLM_PREFILL_TILED", "0")
    monkeypatch.setenv("VKLLM_NORM_EPI", "1")
    ids_a, logits_a = _device_loop(ctx, vk, shape, 7, prompt, 4)
    monkeypatch.setenv("VKLLM_NORM_EPI", "0")
    ids_b, logits_b = _device_loop(ctx, vk, shape, 7, prompt, 4)
    assert ids_a.tolist() == ids_b.tolist()
    assert np.array_equal(logits_a.view(np.uint16), logits_b.view(np.uint16))


def test_long_cache_attention_in_one_launch(ctx, vk, monkeypatch):
    """The long-cache attention in one launch (chunk blocks wait for each other's statistics) against the scores and
    P.V kernels, at the 7B widths with a 640-position cache (3 chunks of 224): from the first long-cache step through
    kv == head_dim (the transposed product) to two chunks merged; identical ids and logits."""
    shape = dict(n_layer=2, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=640)
    prompt = vk.prompt_tokens(9, 60, shape["vocab"])
    monkeypatch.setenv("VKLLM_ATTN_SMALL_MAX", "64")
    monkeypatch.setenv("VKLLM_ATTN_LONG", "1")
    ids_a, logits_a = _device_loop(ctx, vk, shape, 7, prompt, 200)
    monkeypatch.setenv("VKLLM_ATTN_LONG", "0")
    ids_b, logits_b = _device_loop(ctx, vk, shape, 7, prompt, 200)
    assert ids_a.tolist() == ids_b.tolist()
    assert np.array_equal(logits_a.view(np.uint16), logits_b.view(np.uint16))


def test_13b_widths_one_layer(ctx, vk, oracle):
    """The LLaMA-2-13B widths (dim 5120, 40 heads of 128, FFN 13824, vocab 32000) on one layer: 6-token prefill,
    then 5 greedy steps."""
    shape = dict(n_layer=1, dim=5120, n_head=40, ffn=13824, vocab=32000, ctx=32)
    ids, want_ids, err = _gpu_vs_oracle(ctx, vk, oracle, shape, seed=9, prompt_len=6, n_steps=5, prompt_seed=10)
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


def _steps_vs_oracle(ctx, vk, oracle, shape, seed, chunks, prompt_seed):
    """Prefill chunks (token counts) back to back at growing offsets on a device-initialised model and on the
    oracle; per chunk: ids and the logits of every row."""
    cfg = oracle.make_cfg(**shape)
    toks = oracle.prompt_tokens(prompt_seed, sum(chunks), cfg.vocab)
    ref = oracle.Model(cfg=cfg, seed=seed)
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=seed)
    out = []
    try:
        offset = 0
        for n in chunks:
            part = toks[offset:offset + n]
            want_ids, want_logits, _ = ref.step(part, offset, want_logits=True)
            ids = model.step(part, offset)
            logits = model.last_logits(n)
            out.append((ids, want_ids, logits, want_logits))
            offset += n
    finally:
        ref.close()
        model.close()
    return out


def test_prefill_transposed_rule_head_dim_128(ctx, vk, oracle):
    """A 128-token prompt at head_dim 128 makes kv == hd (the reference's attn . V^T), on the MFMA prefill path;
    then two single-token steps."""
    shape = dict(n_layer=2, dim=256, n_head=2, ffn=512, vocab=1000, ctx=256)
    for ids, want_ids, logits, want_logits in _steps_vs_oracle(ctx, vk, oracle, shape, 11, [128], 12):
        err = np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32)))
        print(f"max|dlogit| {err:.3g}")
        assert err <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, "128-row prefill")
    ids, want_ids, err = _gpu_vs_oracle(ctx, vk, oracle, shape, seed=11, prompt_len=128, n_steps=3, prompt_seed=12)
    assert err.max() <= LOGIT_TOL
    assert ids.tolist() == want_ids.tolist()


@pytest.mark.parametrize("head_dim", [64, 128])
def test_chunked_prefill(ctx, vk, oracle, head_dim):
    """Prompt chunks at offsets 0, 40 and 130 (rows of a chunk attend to all earlier positions, the row max taken
    over the whole chunk's kv), partial 64-row blocks and key blocks, on the MFMA prefill path."""
    shape = dict(n_layer=2, dim=4 * head_dim, n_head=4, ffn=640, vocab=1000, ctx=512)
    for ids, want_ids, logits, want_logits in _steps_vs_oracle(ctx, vk, oracle, shape, 13, [40, 90, 77], 14):
        err = np.max(np.abs(logits.astype(np.float32) - want_logits.astype(np.float32)))
        print(f"max|dlogit| {err:.3g}")
        assert err <= LOGIT_TOL
        assert_prefill_ids(ids, want_ids, want_logits, f"{len(ids)}-row chunk")
