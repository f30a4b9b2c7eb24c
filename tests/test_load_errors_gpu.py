"""vkllm_models_llama2_load on files it must refuse. The reference returns VKLLM_ERR_ARGS when gguf_open fails
(src/models/vkllm_models_llama2.c:265-270); here also when a weight the graph reads is absent (the reference would
leave it NULL and fault in build_graph). After a failed load the model is empty: freeing it again is harmless, and
the same model struct then loads a good file.
"""
import ctypes
import os

import pytest

import gguf_util as G

pytestmark = pytest.mark.gpu

VOCAB = (["<unk>", "<s>", "</s>"] + [f"t{i}" for i in range(61)], [0.0] * 64)


def _model_file(path, n_layer=2):
    G.llama_model(str(path), *VOCAB, dim=64, n_head=2, ffn=96, ctx=32, n_layer=n_layer)
    return path


def _edit_tensor_names(src, dst, rename):
    """Copy of a GGUF file with tensor names replaced in place (same length, so every offset stays valid)."""
    blob = bytearray(src.read_bytes())
    for old, new in rename.items():
        assert len(old) == len(new)
        at = blob.index(old.encode())
        blob[at:at + len(old)] = new.encode()
    dst.write_bytes(bytes(blob))
    return dst


def _load(ctx, vk, path):
    m = vk.ModelStruct()
    L = vk.lib()
    print(f"[load] {os.path.basename(str(path))}", flush=True)
    rc = L.vkllm_models_llama2_load(ctx.vp, ctypes.byref(m), str(path).encode())
    return rc, m


def test_good_file_loads(ctx, vk, tmp_path):
    rc, m = _load(ctx, vk, _model_file(tmp_path / "good.gguf"))
    assert rc == vk.ERR_OK
    assert m.meta.block_count == 2 and m.weights.blocks.contents.used_n == 2
    assert vk.lib().vkllm_models_llama2_free(ctx.vp, ctypes.byref(m)) == vk.ERR_OK


@pytest.mark.parametrize("case", ["missing_path", "truncated_header", "truncated_data", "bad_magic",
                                  "missing_tensor", "duplicate_tensor", "missing_block"])
def test_refused_files(ctx, vk, tmp_path, case):
    good = _model_file(tmp_path / "good.gguf")
    path = tmp_path / f"{case}.gguf"
    if case == "missing_path":
        path = tmp_path / "does_not_exist.gguf"
    elif case == "truncated_header":
        path.write_bytes(good.read_bytes()[:300])
    elif case == "truncated_data":
        path.write_bytes(good.read_bytes()[:-100])
    elif case == "bad_magic":
        path.write_bytes(b"GGML" + good.read_bytes()[4:])
    elif case == "missing_tensor":
        # blk.1.ffn_down.weight renamed to a name the loader does not know
        _edit_tensor_names(good, path, {"blk.1.ffn_down.weight": "blk.1.ffn_dwn_.weight"})
    elif case == "duplicate_tensor":
        # blk.0.attn_k.weight renamed to blk.0.attn_q.weight: Q twice, K absent
        _edit_tensor_names(good, path, {"blk.0.attn_k.weight": "blk.0.attn_q.weight"})
    else:
        # block_count says 3, the file holds 2 blocks
        blob = bytearray(good.read_bytes())
        key = G._str("llama.block_count") + (4).to_bytes(4, "little")
        at = blob.index(key) + len(key)
        assert int.from_bytes(blob[at:at + 4], "little") == 2
        blob[at:at + 4] = (3).to_bytes(4, "little")
        path.write_bytes(bytes(blob))
    rc, m = _load(ctx, vk, path)
    assert rc == vk.ERR_ARGS, f"{case}: load returned {rc}"
    L = vk.lib()
    assert not m.priv and not m.weights.blocks and not m.weights.tok_embed_weights
    assert L.vkllm_models_llama2_free(ctx.vp, ctypes.byref(m)) == vk.ERR_OK
    # the same struct then takes a good file
    assert L.vkllm_models_llama2_load(ctx.vp, ctypes.byref(m), str(good).encode()) == vk.ERR_OK
    assert L.vkllm_models_llama2_free(ctx.vp, ctypes.byref(m)) == vk.ERR_OK
