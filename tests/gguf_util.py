"""A minimal GGUF v3 writer for tests (public GGUF layout: header, key/values, tensor infos, data aligned to 32
bytes), used to build models with a chosen vocabulary. It shares no code with the library's reader or the oracle's
writer."""
import struct

import numpy as np

U32, I32, F32, BOOL, STRING, ARRAY = 4, 5, 6, 7, 8, 9
GGML_F32, GGML_F16 = 0, 1
ALIGN = 32


def _str(b):
    b = b.encode() if isinstance(b, str) else bytes(b)
    return struct.pack("<Q", len(b)) + b


def _value(ty, v):
    if ty == U32:
        return struct.pack("<I", v)
    if ty == I32:
        return struct.pack("<i", v)
    if ty == F32:
        return struct.pack("<f", v)
    if ty == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if ty == STRING:
        return _str(v)
    raise ValueError(ty)


def write(path, kvs, tensors):
    """kvs: [(key, type, value)] with value a list and type (ARRAY, element type) for arrays;
    tensors: [(name, ne (innermost first), GGML type, numpy array)]"""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs) + 1))
    out += _str("general.alignment") + struct.pack("<I", U32) + struct.pack("<I", ALIGN)
    for key, ty, v in kvs:
        out += _str(key)
        if isinstance(ty, tuple):
            et = ty[1]
            out += struct.pack("<IIQ", ARRAY, et, len(v)) + b"".join(_value(et, x) for x in v)
        else:
            out += struct.pack("<I", ty) + _value(ty, v)
    offset, blobs = 0, []
    for name, ne, ty, arr in tensors:
        data = np.ascontiguousarray(arr).tobytes()
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", ty, offset)
        blobs.append(data)
        offset += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    out += b"\0" * ((-len(out)) % ALIGN)
    for data in blobs:
        out += data + b"\0" * ((-len(data)) % ALIGN)
    with open(path, "wb") as f:
        f.write(out)


def llama_model(path, texts, scores, dim=64, n_head=2, ffn=96, ctx=32, n_layer=1, bos=1, eos=2, add_bos=True,
                add_eos=False, seed=0):
    """A small random LLaMA-2 GGUF (fp16 weights, fp32 norms) with the vocabulary `texts`/`scores`."""
    V = len(texts)
    rng = np.random.default_rng(seed)

    def w(rows, cols):
        return (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16)

    kvs = [("general.architecture", STRING, "llama"), ("llama.block_count", U32, n_layer),
           ("llama.context_length", U32, ctx), ("llama.embedding_length", U32, dim),
           ("llama.feed_forward_length", U32, ffn), ("llama.attention.head_count", U32, n_head),
           ("llama.attention.head_count_kv", U32, n_head), ("llama.attention.layer_norm_rms_epsilon", F32, 1e-5),
           ("llama.rope.freq_base", F32, 10000.0), ("llama.vocab_size", U32, V),
           ("tokenizer.ggml.model", STRING, "llama"), ("tokenizer.ggml.tokens", (ARRAY, STRING), list(texts)),
           ("tokenizer.ggml.scores", (ARRAY, F32), [float(s) for s in scores]),
           ("tokenizer.ggml.token_type", (ARRAY, I32), [1] * V), ("tokenizer.ggml.bos_token_id", U32, bos),
           ("tokenizer.ggml.eos_token_id", U32, eos), ("tokenizer.ggml.add_bos_token", BOOL, add_bos),
           ("tokenizer.ggml.add_eos_token", BOOL, add_eos)]
    ones = np.ones(dim, np.float32)
    tensors = [("token_embd.weight", [dim, V], GGML_F16, w(V, dim))]
    for l in range(n_layer):
        b = f"blk.{l}."
        tensors += [(b + "attn_norm.weight", [dim], GGML_F32, ones), (b + "attn_q.weight", [dim, dim], GGML_F16, w(dim, dim)),
                    (b + "attn_k.weight", [dim, dim], GGML_F16, w(dim, dim)),
                    (b + "attn_v.weight", [dim, dim], GGML_F16, w(dim, dim)),
                    (b + "attn_output.weight", [dim, dim], GGML_F16, w(dim, dim)),
                    (b + "ffn_norm.weight", [dim], GGML_F32, ones), (b + "ffn_gate.weight", [dim, ffn], GGML_F16, w(ffn, dim)),
                    (b + "ffn_up.weight", [dim, ffn], GGML_F16, w(ffn, dim)),
                    (b + "ffn_down.weight", [ffn, dim], GGML_F16, w(dim, ffn))]
    tensors += [("output_norm.weight", [dim], GGML_F32, ones), ("output.weight", [dim, V], GGML_F16, w(V, dim))]
    write(path, kvs, tensors)
