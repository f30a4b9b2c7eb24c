"""ctypes access to the CPU oracle (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as
the side that the library's results are compared with. The shipped library never loads it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

F32, F16, I8, U32 = 1, 2, 3, 4
NP_DTYPE = {F32: np.float32, F16: np.float16, U32: np.uint32, I8: np.int8}


class OracleTensor(ctypes.Structure):
    _fields_ = [("shapes", ctypes.c_uint32 * 4), ("strides", ctypes.c_uint32 * 4), ("dtype", ctypes.c_int32),
                ("data", ctypes.c_void_p)]


class LlamaCfg(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_uint32), ("dim", ctypes.c_uint32), ("n_head", ctypes.c_uint32),
                ("n_head_kv", ctypes.c_uint32), ("ffn", ctypes.c_uint32), ("vocab", ctypes.c_uint32),
                ("ctx", ctypes.c_uint32), ("eps", ctypes.c_float), ("theta", ctypes.c_float),
                ("bos_id", ctypes.c_uint32), ("eos_id", ctypes.c_uint32), ("pad_id", ctypes.c_uint32),
                ("weight_std", ctypes.c_float)]


def make_cfg(n_layer, dim, n_head, ffn, vocab=32000, ctx=256, eps=1e-5, theta=10000.0, n_head_kv=None,
             bos_id=1, eos_id=2, pad_id=0, weight_std=0.02):
    return LlamaCfg(n_layer, dim, n_head, n_head if n_head_kv is None else n_head_kv, ffn, vocab, ctx, eps, theta,
                    bos_id, eos_id, pad_id, weight_std)


# the LLaMA-2 shapes the workloads name
TINY = dict(n_layer=6, dim=288, n_head=6, ffn=768, vocab=32000, ctx=256)
LLAMA7B = dict(n_layer=32, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=4096)
LLAMA13B = dict(n_layer=40, dim=5120, n_head=40, ffn=13824, vocab=32000, ctx=4096)

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C oracle")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(OracleTensor)
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_splitmix64.restype = ctypes.c_uint64
        L.oracle_splitmix64.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_normal.restype = ctypes.c_float
        L.oracle_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_weight_f16.restype = ctypes.c_uint16
        L.oracle_weight_f16.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float]
        L.oracle_tensor_stream.restype = ctypes.c_uint64
        L.oracle_tensor_stream.argtypes = [ctypes.c_uint64, ctypes.c_uint32]
        L.oracle_prompt_token.restype = ctypes.c_uint32
        L.oracle_prompt_token.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_is_transposed_b.argtypes = [P, P, P]
        L.oracle_matmul.argtypes = [P, P, P, ctypes.c_float, ctypes.c_int32]
        L.oracle_embedding.argtypes = [P, P, P, ctypes.c_uint32]
        L.oracle_rmsnorm.argtypes = [P, P, P, ctypes.c_float]
        L.oracle_rope.argtypes = [P, P, ctypes.c_uint32, ctypes.c_float, ctypes.c_int]
        L.oracle_rope_freqs.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.POINTER(ctypes.c_float)]
        L.oracle_softmax.argtypes = [P, P, ctypes.c_int32, ctypes.c_uint32]
        L.oracle_update_rows.argtypes = [P, P, ctypes.c_uint32]
        L.oracle_copy.argtypes = [P, P]
        L.oracle_bin.argtypes = [P, P, P, ctypes.c_int32]
        L.oracle_arg_max.argtypes = [P, P]
        L.oracle_ffn_up_and_gate.argtypes = [P, P, P, P]
        L.oracle_gguf_write_random.argtypes = [ctypes.c_char_p, ctypes.POINTER(LlamaCfg), ctypes.c_uint64]
        L.oracle_model_load.restype = ctypes.c_void_p
        L.oracle_model_load.argtypes = [ctypes.c_char_p]
        L.oracle_model_random.restype = ctypes.c_void_p
        L.oracle_model_random.argtypes = [ctypes.POINTER(LlamaCfg), ctypes.c_uint64]
        L.oracle_model_free.argtypes = [ctypes.c_void_p]
        L.oracle_model_cfg.argtypes = [ctypes.c_void_p, ctypes.POINTER(LlamaCfg)]
        L.oracle_model_weight.restype = ctypes.c_void_p
        L.oracle_model_weight.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_size_t)]
        L.oracle_model_step.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32,
                                        ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32), ctypes.c_void_p,
                                        ctypes.c_void_p]
        L.oracle_token_loop.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32,
                                        ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32), ctypes.c_void_p]
        L.oracle_set_numerics.argtypes = [ctypes.c_int, ctypes.c_uint32]
        L.oracle_set_accumulation.argtypes = [ctypes.c_int]
        L.oracle_f64_to_f16.restype = ctypes.c_uint16
        L.oracle_f64_to_f16.argtypes = [ctypes.c_double]
        L.oracle_gemv16.restype = ctypes.c_uint16
        L.oracle_gemv16.argtypes = [P16, P16, ctypes.c_uint32, ctypes.c_float, ctypes.c_int, ctypes.c_uint32]
        L.oracle_gemm16_dot.restype = ctypes.c_float
        L.oracle_gemm16_dot.argtypes = [P16, P16, ctypes.c_uint32]
        L.oracle_softmax16_row.argtypes = [P16, P16, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_rope16_pair.argtypes = [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, ctypes.c_float, P16, P16]
        _lib = L
    return _lib


P16 = ctypes.POINTER(ctypes.c_uint16)


def _p16(a):
    return a.ctypes.data_as(P16)


def set_numerics(ref16, subgroup=8):
    """REF16 (the reference's fp16-arithmetic shader variants, subgroups of `subgroup` lanes) or the fp32 mode"""
    lib().oracle_set_numerics(1 if ref16 else 0, subgroup if ref16 else 0)


def set_accumulation(fp32_sequential):
    """The fp32 mode's summation order: double sums (False, the default) or sequential fp32 sums (True)"""
    lib().oracle_set_accumulation(1 if fp32_sequential else 0)


def f64_to_f16_bits(x):
    return lib().oracle_f64_to_f16(float(x))


def gemv16(x, w, scale=1.0, act=0, subgroup=8):
    x = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint16)
    return lib().oracle_gemv16(_p16(x), _p16(w), len(x), scale, act, subgroup)


def gemm16_dot(a, b):
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    return lib().oracle_gemm16_dot(_p16(a), _p16(b), len(a))


def softmax16_row(x, limit=None, subgroup=8):
    x = np.ascontiguousarray(x, np.uint16)
    out = np.zeros_like(x)
    lib().oracle_softmax16_row(_p16(x), _p16(out), len(x), len(x) if limit is None else limit, subgroup)
    return out


def rope16_pair(v0, v1, pos, w, hd, base=10000.0):
    o0, o1 = ctypes.c_uint16(), ctypes.c_uint16()
    lib().oracle_rope16_pair(v0, v1, pos, w, hd, base, ctypes.byref(o0), ctypes.byref(o1))
    return o0.value, o1.value


def tensor(arr, shapes=None, strides=None, dtype=None):
    """Describe numpy array `arr` (its base buffer) as an oracle tensor; strides default to arr's, in elements."""
    if dtype is None:
        dtype = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint32): U32,
                 np.dtype(np.int8): I8}[arr.dtype]
    if shapes is None:
        shapes = list(arr.shape)
        assert len(shapes) == 4
    if strides is None:
        strides = [s // arr.itemsize for s in arr.strides]
    t = OracleTensor()
    for i in range(4):
        t.shapes[i] = shapes[i]
        t.strides[i] = strides[i]
    t.dtype = dtype
    t.data = arr.ctypes.data
    t._keep = arr
    return t


def _ref(t):
    return ctypes.byref(t)


def matmul(a, b, out, scale=1.0, act=0):
    return lib().oracle_matmul(_ref(a), _ref(b), _ref(out), scale, act)


def is_transposed_b(a, b, out):
    return bool(lib().oracle_is_transposed_b(_ref(a), _ref(b), _ref(out)))


def embedding(idx, table, out, unk):
    return lib().oracle_embedding(_ref(idx), _ref(table), _ref(out), unk)


def rmsnorm(x, w, out, eps):
    return lib().oracle_rmsnorm(_ref(x), _ref(w), _ref(out), eps)


def rope(x, out, offset, base, neox=False):
    return lib().oracle_rope(_ref(x), _ref(out), offset, base, int(neox))


def rope_freqs(base, D):
    f = (ctypes.c_float * (D // 2))()
    lib().oracle_rope_freqs(base, D, f)
    return np.array(f[:], dtype=np.float32)


def softmax(x, out, seq_mask, offsets):
    return lib().oracle_softmax(_ref(x), _ref(out), seq_mask, offsets)


def update_rows(src, cache, offset):
    return lib().oracle_update_rows(_ref(src), _ref(cache), offset)


def copy(x, out):
    return lib().oracle_copy(_ref(x), _ref(out))


def bin_op(a, b, out, op):
    return lib().oracle_bin(_ref(a), _ref(b), _ref(out), op)


def arg_max(x, out):
    return lib().oracle_arg_max(_ref(x), _ref(out))


def ffn_up_and_gate(x, wu, wg, out):
    return lib().oracle_ffn_up_and_gate(_ref(x), _ref(wu), _ref(wg), _ref(out))


def f32_to_f16_bits(x):
    return lib().oracle_f32_to_f16(float(x))


def weights_f16(seed, tensor_id, count, std=0.02):
    L = lib()
    return np.array([L.oracle_weight_f16(seed, tensor_id, i, std) for i in range(count)], dtype=np.uint16)


def prompt_tokens(seed, n, vocab):
    return np.array([lib().oracle_prompt_token(seed, i, vocab) for i in range(n)], dtype=np.uint32)


def write_gguf(path, cfg, seed):
    rc = lib().oracle_gguf_write_random(path.encode(), ctypes.byref(cfg), seed)
    if rc != 0:
        raise RuntimeError(f"oracle_gguf_write_random({path}) failed")


class Model:
    """oracle LLaMA-2 model: loaded from a GGUF file or built from (cfg, seed)."""

    def __init__(self, path=None, cfg=None, seed=0):
        L = lib()
        if path is not None:
            self.h = L.oracle_model_load(path.encode())
        else:
            self.h = L.oracle_model_random(ctypes.byref(cfg), seed)
        if not self.h:
            raise RuntimeError("oracle model creation failed")
        c = LlamaCfg()
        L.oracle_model_cfg(self.h, ctypes.byref(c))
        self.cfg = c

    def close(self):
        if self.h:
            lib().oracle_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def weight(self, tensor_id):
        n = ctypes.c_size_t()
        p = lib().oracle_model_weight(self.h, tensor_id, ctypes.byref(n))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), shape=(n.value,)).copy()

    def step(self, toks, offset, want_logits=False, want_hidden=False):
        toks = np.ascontiguousarray(toks, dtype=np.uint32)
        S = len(toks)
        ids = np.zeros(S, dtype=np.uint32)
        logits = np.zeros((S, self.cfg.vocab), dtype=np.float16) if want_logits else None
        hidden = np.zeros((S, self.cfg.dim), dtype=np.float16) if want_hidden else None
        rc = lib().oracle_model_step(self.h, toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), S, offset,
                                     ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                     logits.ctypes.data if logits is not None else None,
                                     hidden.ctypes.data if hidden is not None else None)
        if rc != 0:
            raise RuntimeError("oracle_model_step failed")
        return ids, logits, hidden

    def token_loop(self, prompt, n_steps, want_logits=False):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        ids = np.zeros(n_steps, dtype=np.uint32)
        logits = np.zeros((n_steps, self.cfg.vocab), dtype=np.float16) if want_logits else None
        rc = lib().oracle_token_loop(self.h, prompt.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(prompt),
                                     n_steps, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                     logits.ctypes.data if logits is not None else None)
        if rc != 0:
            raise RuntimeError("oracle_token_loop failed")
        return ids, logits
