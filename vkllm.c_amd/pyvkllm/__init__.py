"""ctypes binding of libvkllm (the vkllm.c C API on HIP/gfx950).

The structs below mirror include/vkllm/*.h field for field; `abi_check()` compares them with the layout the
library reports. Helpers follow the reference's usage: ops are run with a commands object
(tests/vkllm_test_op_matmul.c:288-420), the token loop is the one of tests/vkllm_test_infer_gguf.c:173-272.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "build", "libvkllm.so")

# enums (include/vkllm/vkllm_errors.h, vkllm_dtypes.h, vkllm_ops.h)
ERR_OK, ERR_ALLOC, ERR_VULKAN, ERR_DEV_NOT_FOUND, ERR_PIPELINE_NOT_FOUND, ERR_ARGS = 1, 2, 3, 4, 5, 6
F32, F16, I8, U32 = 1, 2, 3, 4
(OP_NONE, OP_COPY, OP_BIN, OP_EMBEDDING, OP_RMSNORM, OP_MATMUL, OP_ROPE, OP_SOFTMAX, OP_FFN_UP_AND_GATE,
 OP_UPDATE_ROWS, OP_ARG_MAX, OP_REF) = range(12)
EXEC_FUSED, EXEC_NODES = 0, 1
NP_DTYPE = {F32: np.float32, F16: np.float16, U32: np.uint32, I8: np.int8}
DTYPE_OF = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint32): U32, np.dtype(np.int8): I8}


class VkllmError(RuntimeError):
    def __init__(self, fn, code):
        super().__init__(f"{fn} failed: {err_s(code)} ({code})")
        self.code = code


class TensorData(ctypes.Structure):
    _fields_ = [("dev", ctypes.c_void_p), ("host", ctypes.c_void_p), ("mapped", ctypes.c_bool),
                ("is_ref", ctypes.c_bool), ("borrowed", ctypes.c_bool), ("valid", ctypes.c_bool),
                ("host_current", ctypes.c_bool)]


class Tensor(ctypes.Structure):
    pass


Tensor._fields_ = [("name", ctypes.c_char * 128), ("dtype", ctypes.c_int), ("shapes", ctypes.c_uint32 * 4),
                   ("strides", ctypes.c_uint32 * 4), ("bytes", ctypes.c_uint32), ("device", ctypes.c_void_p),
                   ("data", TensorData), ("access_flags", ctypes.c_uint32), ("pipeline_stage", ctypes.c_uint32),
                   ("op", ctypes.c_int), ("pipeline", ctypes.c_void_p), ("srcs", ctypes.POINTER(Tensor) * 4)]
TensorP = ctypes.POINTER(Tensor)


class ArrayTensor(ctypes.Structure):
    _fields_ = [("alloc_n", ctypes.c_size_t), ("used_n", ctypes.c_size_t), ("data", ctypes.POINTER(TensorP))]


class Graph(ctypes.Structure):
    _fields_ = [("nodes", ctypes.POINTER(ArrayTensor)), ("input_nodes", ctypes.POINTER(ArrayTensor)),
                ("output_node", TensorP), ("commands", ctypes.c_void_p), ("plan", ctypes.c_void_p)]


class Stats(ctypes.Structure):
    _fields_ = [("tensor_alloc_counts", ctypes.c_int), ("tensor_free_counts", ctypes.c_int),
                ("op_time_costs", ctypes.c_uint64 * 12), ("node_time_cost", ctypes.c_void_p)]


class Context(ctypes.Structure):
    _fields_ = [("appname", ctypes.c_char_p), ("device", ctypes.c_void_p), ("pipelines", ctypes.c_void_p),
                ("stats", Stats)]


class Pipeline(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("kernel_id", ctypes.c_int), ("last_ns", ctypes.c_uint64),
                ("total_ns", ctypes.c_uint64), ("launches", ctypes.c_uint64), ("ev_begin", ctypes.c_void_p),
                ("ev_end", ctypes.c_void_p), ("pending", ctypes.c_int)]


class Token(ctypes.Structure):
    _fields_ = [("text", ctypes.c_char_p), ("score", ctypes.c_float), ("type", ctypes.c_int32)]


class ArrayToken(ctypes.Structure):
    _fields_ = [("alloc_n", ctypes.c_size_t), ("used_n", ctypes.c_size_t), ("data", ctypes.POINTER(Token))]


class ArrayTokenId(ctypes.Structure):
    _fields_ = [("alloc_n", ctypes.c_size_t), ("used_n", ctypes.c_size_t), ("data", ctypes.POINTER(ctypes.c_uint32))]


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, TensorP) for n in ("attn_norm_weight", "ffn_norm_weight", "WQ", "WK", "WV", "WO", "WU", "WG",
                                       "WD")]


class ArrayBlockWeights(ctypes.Structure):
    _fields_ = [("alloc_n", ctypes.c_size_t), ("used_n", ctypes.c_size_t),
                ("data", ctypes.POINTER(ctypes.POINTER(BlockWeights)))]


class Meta(ctypes.Structure):
    _fields_ = [("block_count", ctypes.c_uint32), ("context_length", ctypes.c_uint32),
                ("embedding_length", ctypes.c_uint32), ("rope_freq_base", ctypes.c_float),
                ("layer_norm_rms_epsilon", ctypes.c_float), ("key_length", ctypes.c_uint32),
                ("value_length", ctypes.c_uint32), ("vocab_size", ctypes.c_uint32), ("head_count", ctypes.c_uint32),
                ("head_count_kv", ctypes.c_uint32), ("bos_token_id", ctypes.c_uint32),
                ("eos_token_id", ctypes.c_uint32), ("padding_token_id", ctypes.c_uint32),
                ("add_bos_token", ctypes.c_bool), ("add_eos_token", ctypes.c_bool),
                ("tokens", ctypes.POINTER(ArrayToken))]


class Weights(ctypes.Structure):
    _fields_ = [("tok_embed_weights", TensorP), ("blocks", ctypes.POINTER(ArrayBlockWeights)),
                ("output_norm_weight", TensorP), ("output_weight", TensorP), ("kvcache", ctypes.c_void_p)]


class ModelStruct(ctypes.Structure):
    _fields_ = [("meta", Meta), ("weights", Weights), ("priv", ctypes.c_void_p)]


class LlamaConfig(ctypes.Structure):
    _fields_ = [("block_count", ctypes.c_uint32), ("embedding_length", ctypes.c_uint32),
                ("head_count", ctypes.c_uint32), ("feed_forward_length", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("context_length", ctypes.c_uint32),
                ("layer_norm_rms_epsilon", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
                ("weight_std", ctypes.c_float)]


class MatmulParams(ctypes.Structure):
    _fields_ = [("scale", ctypes.c_float), ("act", ctypes.c_int32)]


class RmsnormParams(ctypes.Structure):
    _fields_ = [("power", ctypes.c_float), ("eps", ctypes.c_float)]


class RopeParams(ctypes.Structure):
    _fields_ = [("offset", ctypes.c_uint32), ("base", ctypes.c_float), ("neox_style", ctypes.c_bool)]


class SoftmaxParams(ctypes.Structure):
    _fields_ = [("seq_mask", ctypes.c_int32), ("offsets", ctypes.c_uint32)]


class UpdateRowsParams(ctypes.Structure):
    _fields_ = [("offset_rows", ctypes.c_uint32)]


OPS = ["copy", "bin", "embedding", "rmsnorm", "matmul", "rope", "softmax", "ffn_up_and_gate", "update_rows",
       "arg_max"]

_lib = None


def lib():
    """The loaded libvkllm; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (make -C vkllm.c_amd)")
        L = ctypes.CDLL(LIB_PATH)
        E = ctypes.c_int
        vp = ctypes.c_void_p
        u32 = ctypes.c_uint32
        sig = {
            "vkllm_err_s": (ctypes.c_char_p, [E]),
            "vkllm_dtype_s": (ctypes.c_char_p, [E]),
            "vkllm_op_s": (ctypes.c_char_p, [E]),
            "vkllm_context_new": (E, [u32, ctypes.POINTER(ctypes.POINTER(Context))]),
            "vkllm_context_free": (None, [ctypes.POINTER(Context)]),
            "vkllm_tensor_new": (E, [vp, ctypes.c_char_p, ctypes.POINTER(u32), E, E, ctypes.POINTER(TensorP), u32,
                                     vp, ctypes.c_size_t, ctypes.c_bool, ctypes.POINTER(TensorP)]),
            "vkllm_tensor_free": (None, [vp, TensorP]),
            "vkllm_tensor_invalid_cache": (E, [vp, TensorP]),
            "vkllm_tensor_flush_cache": (E, [vp, TensorP]),
            "vkllm_tensor_new_staging": (E, [vp, TensorP, ctypes.POINTER(TensorP)]),
            "vkllm_tensor_reshape": (E, [vp, TensorP, ctypes.POINTER(u32)]),
            "vkllm_tensor_permute": (E, [vp, TensorP, ctypes.POINTER(u32)]),
            "vkllm_tensor_copy_ref": (E, [vp, TensorP, ctypes.POINTER(TensorP)]),
            "vkllm_tensor_slice0": (E, [vp, TensorP, ctypes.POINTER(u32), ctypes.POINTER(TensorP)]),
            "vkllm_tensor_s": (E, [vp, TensorP, ctypes.c_char_p, ctypes.c_size_t]),
            "vkllm_commands_new": (E, [vp, ctypes.POINTER(vp)]),
            "vkllm_commands_free": (None, [vp, vp]),
            "vkllm_commands_begin": (E, [vp, vp]),
            "vkllm_commands_end": (E, [vp, vp]),
            "vkllm_commands_upload": (E, [vp, vp, TensorP, vp, ctypes.c_size_t]),
            "vkllm_commands_download": (E, [vp, vp, TensorP, vp, ctypes.c_size_t]),
            "vkllm_commands_submit": (E, [vp, vp]),
            "vkllm_commands_wait_exec": (E, [vp, vp]),
            "vkllm_commands_sync_tensor": (None, [vp, vp, TensorP, u32, u32]),
            "vkllm_graph_new": (E, [vp, ctypes.POINTER(ctypes.POINTER(Graph))]),
            "vkllm_graph_add_input": (E, [vp, ctypes.POINTER(Graph), TensorP]),
            "vkllm_graph_add_node": (E, [vp, ctypes.POINTER(Graph), TensorP]),
            "vkllm_graph_set_output": (E, [vp, ctypes.POINTER(Graph), TensorP]),
            "vkllm_graph_init": (E, [vp, ctypes.POINTER(Graph)]),
            "vkllm_graph_run": (E, [vp, ctypes.POINTER(Graph)]),
            "vkllm_graph_post_run": (E, [vp, ctypes.POINTER(Graph)]),
            "vkllm_graph_free": (E, [vp, ctypes.POINTER(Graph)]),
            "vkllm_pipeline_query_exec_time": (E, [vp, vp, ctypes.POINTER(ctypes.c_uint64)]),
            "vkllm_models_llama2_load": (E, [vp, ctypes.POINTER(ModelStruct), ctypes.c_char_p]),
            "vkllm_models_llama2_free": (E, [vp, ctypes.POINTER(ModelStruct)]),
            "vkllm_models_llama2_build_graph": (E, [vp, ctypes.POINTER(ModelStruct), TensorP, ctypes.POINTER(Graph),
                                                    u32]),
            "vkllm_models_llama2_tokenize": (E, [ctypes.POINTER(ModelStruct), ctypes.c_char_p,
                                                 ctypes.POINTER(ctypes.POINTER(ArrayTokenId))]),
            "vkllm_models_llama2_init_random": (E, [vp, ctypes.POINTER(ModelStruct), ctypes.POINTER(LlamaConfig),
                                                    ctypes.c_uint64]),
            "vkllm_hip_set_exec_mode": (E, [vp, E]),
            "vkllm_hip_get_exec_mode": (E, [vp]),
            "vkllm_hip_set_graph_replay": (E, [vp, E]),
            "vkllm_hip_set_timing": (E, [vp, E]),
            "vkllm_hip_synchronize": (E, [vp]),
            "vkllm_hip_context_stream": (E, [vp, ctypes.POINTER(vp)]),
            "vkllm_hip_time_ops": (E, [vp, ctypes.POINTER(TensorP), u32, u32, ctypes.POINTER(ctypes.c_uint64)]),
            "vkllm_hip_probe_stream_read": (E, [vp, ctypes.c_uint64, u32, ctypes.POINTER(ctypes.c_double),
                                                ctypes.POINTER(ctypes.c_double)]),
            "vkllm_hip_probe_launch_gap": (E, [vp, u32, u32, ctypes.POINTER(ctypes.c_double)]),
            "vkllm_hip_kernel_stats": (E, [vp, E, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64)]),
            "vkllm_hip_reset_kernel_stats": (E, [vp]),
            "vkllm_hip_kernel_family_count": (E, []),
            "vkllm_hip_model_time_kernel": (E, [vp, ctypes.POINTER(ModelStruct), ctypes.c_char_p, u32,
                                                ctypes.POINTER(ctypes.c_uint64)]),
            "vkllm_hip_device_arch": (ctypes.c_char_p, [vp]),
            "vkllm_hip_model_last_logits": (E, [vp, ctypes.POINTER(ModelStruct), vp, u32]),
            "vkllm_hip_token_loop": (E, [vp, ctypes.POINTER(ModelStruct), vp, u32, u32, u32, vp, vp, vp]),
            "vkllm_hip_gemm": (E, [vp, E, vp, vp, vp, u32, u32, u32, u32, u32, vp, ctypes.c_uint64]),
            "vkllm_hip_gemm_noalloc": (E, [vp, E, vp, vp, vp, u32, u32, u32, u32, u32, ctypes.c_uint64]),
            "vkllm_hip_gemm_streamed": (E, [vp, E, vp, vp, vp, u32, u32, u32, u32, u32]),
            "vkllm_hip_abi_layout": (E, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_uint64), E]),
            "vkllm_hashmap_new": (E, [ctypes.POINTER(vp), ctypes.c_size_t]),
            "vkllm_hashmap_free": (None, [vp]),
            "vkllm_hashmap_insert": (E, [vp, ctypes.c_char_p, ctypes.c_uint64]),
            "vkllm_hashmap_get": (ctypes.c_bool, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
            "vkllm_hashmap_contains": (ctypes.c_bool, [vp, ctypes.c_char_p]),
            "vkllm_hashmap_remove": (E, [vp, ctypes.c_char_p]),
            "vkllm_hashmap_size": (ctypes.c_size_t, [vp]),
            "vkllm_hashmap_empty": (ctypes.c_bool, [vp]),
            "vkllm_hashmap_clear": (None, [vp]),
        }
        for op in OPS:
            for phase in ("init", "run", "post_run"):
                sig[f"vkllm_op_{op}_{phase}"] = (E, [vp, vp, TensorP])
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def err_s(code):
    try:
        return lib().vkllm_err_s(code).decode()
    except Exception:  # library missing: still print something useful
        return str(code)


def check(fn, code):
    if code != ERR_OK:
        raise VkllmError(fn, code)


def abi_layout():
    L = lib()
    n = L.vkllm_hip_abi_layout(None, None, 0)
    names = (ctypes.c_char_p * n)()
    vals = (ctypes.c_uint64 * n)()
    L.vkllm_hip_abi_layout(names, vals, n)
    return {names[i].decode(): vals[i] for i in range(n)}


def abi_check():
    """Mismatches between these ctypes mirrors and the library's struct layout (empty when they agree)."""
    lay = abi_layout()
    mine = {
        "sizeof(vkllm_tensor)": ctypes.sizeof(Tensor),
        "vkllm_tensor.dtype": Tensor.dtype.offset,
        "vkllm_tensor.shapes": Tensor.shapes.offset,
        "vkllm_tensor.strides": Tensor.strides.offset,
        "vkllm_tensor.bytes": Tensor.bytes.offset,
        "vkllm_tensor.data.dev": Tensor.data.offset + TensorData.dev.offset,
        "vkllm_tensor.data.host": Tensor.data.offset + TensorData.host.offset,
        "vkllm_tensor.data.mapped": Tensor.data.offset + TensorData.mapped.offset,
        "vkllm_tensor.op": Tensor.op.offset,
        "vkllm_tensor.pipeline": Tensor.pipeline.offset,
        "vkllm_tensor.srcs": Tensor.srcs.offset,
        "vkllm_tensor.params": ctypes.sizeof(Tensor),
        "sizeof(vkllm_graph)": ctypes.sizeof(Graph),
        "vkllm_graph.output_node": Graph.output_node.offset,
        "vkllm_graph.commands": Graph.commands.offset,
        "sizeof(vkllm_models_llama2)": ctypes.sizeof(ModelStruct),
        "vkllm_models_llama2.weights": ModelStruct.weights.offset,
        "sizeof(vkllm_context)": ctypes.sizeof(Context),
        "vkllm_context.stats": Context.stats.offset,
        "sizeof(vkllm_pipeline)": ctypes.sizeof(Pipeline),
    }
    return {k: (v, lay.get(k)) for k, v in mine.items() if lay.get(k) != v}


# --------------------------------------------------------------------------------------------------------------
class Ctx:
    """A vkllm_context plus one commands object for op-level work."""

    def __init__(self, dev=0):
        L = lib()
        p = ctypes.POINTER(Context)()
        check("vkllm_context_new", L.vkllm_context_new(dev, ctypes.byref(p)))
        self.p = p
        self.vp = ctypes.cast(p, ctypes.c_void_p)
        c = ctypes.c_void_p()
        check("vkllm_commands_new", L.vkllm_commands_new(self.vp, ctypes.byref(c)))
        self.cmds = c

    def close(self):
        if getattr(self, "p", None):
            L = lib()
            L.vkllm_commands_free(self.vp, self.cmds)
            L.vkllm_context_free(self.p)
            self.p = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def stats(self):
        return self.p.contents.stats

    def arch(self):
        return lib().vkllm_hip_device_arch(self.vp).decode()

    def set_exec_mode(self, mode):
        check("vkllm_hip_set_exec_mode", lib().vkllm_hip_set_exec_mode(self.vp, mode))

    def set_graph_replay(self, on):
        check("vkllm_hip_set_graph_replay", lib().vkllm_hip_set_graph_replay(self.vp, int(on)))

    def set_timing(self, on):
        check("vkllm_hip_set_timing", lib().vkllm_hip_set_timing(self.vp, int(on)))

    def sync(self):
        check("vkllm_hip_synchronize", lib().vkllm_hip_synchronize(self.vp))

    def kernel_stats(self):
        """{kernel family name: (timed launches, summed nanoseconds)} for the families launched while timing."""
        out = {}
        name, n, ns = ctypes.c_char_p(), ctypes.c_uint64(), ctypes.c_uint64()
        for i in range(lib().vkllm_hip_kernel_family_count()):
            check("vkllm_hip_kernel_stats",
                  lib().vkllm_hip_kernel_stats(self.vp, i, ctypes.byref(name), ctypes.byref(n), ctypes.byref(ns)))
            if n.value:
                out[name.value.decode()] = (n.value, ns.value)
        return out

    def time_ops(self, tensors, reps):
        """Nanoseconds of `reps` back-to-back runs of the ops of `tensors` (cycled) between one event pair."""
        arr = (TensorP * len(tensors))(*tensors)
        ns = ctypes.c_uint64()
        check("vkllm_hip_time_ops", lib().vkllm_hip_time_ops(self.vp, arr, len(tensors), reps, ctypes.byref(ns)))
        return ns.value

    def probe_stream_read(self, window_bytes, reps):
        """(median, best) GB/s of a kernel that only streams window_bytes from HBM (vkllm_hip_probe_stream_read)."""
        med, best = ctypes.c_double(), ctypes.c_double()
        check("vkllm_hip_probe_stream_read", lib().vkllm_hip_probe_stream_read(self.vp, window_bytes, reps,
                                                                                ctypes.byref(med), ctypes.byref(best)))
        return med.value, best.value

    def probe_launch_gap(self, launches, blocks):
        """Microseconds per launch of a graph-replayed chain of empty kernels (vkllm_hip_probe_launch_gap)."""
        us = ctypes.c_double()
        check("vkllm_hip_probe_launch_gap", lib().vkllm_hip_probe_launch_gap(self.vp, launches, blocks,
                                                                              ctypes.byref(us)))
        return us.value

    def reset_kernel_stats(self):
        check("vkllm_hip_reset_kernel_stats", lib().vkllm_hip_reset_kernel_stats(self.vp))

    # ---- tensors ----
    def tensor(self, shapes, dtype, name="t", op=OP_NONE, srcs=(), params=None, mapped=False):
        """vkllm_tensor_new; params is a ctypes object or None."""
        L = lib()
        sh = (ctypes.c_uint32 * 4)(*shapes)
        arr = (TensorP * max(1, len(srcs)))(*srcs)
        out = TensorP()
        pp = ctypes.cast(ctypes.byref(params), ctypes.c_void_p) if params is not None else None
        pb = ctypes.sizeof(params) if params is not None else 0
        rc = L.vkllm_tensor_new(self.vp, name.encode(), sh, dtype, op, arr, len(srcs), pp, pb, mapped,
                                ctypes.byref(out))
        check("vkllm_tensor_new", rc)
        return out

    def free(self, t):
        lib().vkllm_tensor_free(self.vp, t)

    def upload(self, t, arr):
        arr = np.ascontiguousarray(arr)
        check("vkllm_commands_upload", lib().vkllm_commands_upload(self.vp, self.cmds, t, arr.ctypes.data,
                                                                    arr.nbytes))

    def download_raw(self, t, nbytes=None):
        n = t.contents.bytes if nbytes is None else nbytes
        buf = np.zeros(n, dtype=np.uint8)
        check("vkllm_commands_download", lib().vkllm_commands_download(self.vp, self.cmds, t, buf.ctypes.data, n))
        return buf

    def download(self, t):
        """The tensor's elements as an array of its shape (honours its byte strides)."""
        tc = t.contents
        buf = self.download_raw(t)
        return strided_view(buf, tc)

    def run_op(self, op, t):
        """init + run + post_run of one op on the commands object, then submit/wait (reference op-test flow)."""
        L = lib()
        check("vkllm_commands_begin", L.vkllm_commands_begin(self.vp, self.cmds))
        rc = getattr(L, f"vkllm_op_{op}_init")(self.vp, self.cmds, t)
        if rc == ERR_OK:
            rc = getattr(L, f"vkllm_op_{op}_run")(self.vp, self.cmds, t)
        if rc == ERR_OK:
            rc = getattr(L, f"vkllm_op_{op}_post_run")(self.vp, self.cmds, t)
        L.vkllm_commands_end(self.vp, self.cmds)
        L.vkllm_commands_submit(self.vp, self.cmds)
        w = L.vkllm_commands_wait_exec(self.vp, self.cmds)
        return rc if rc != ERR_OK else w

    def tensor_from(self, arr, name="t", mapped=False):
        arr = np.ascontiguousarray(arr)
        shapes = list(arr.shape)
        while len(shapes) < 4:
            shapes.insert(0, 1)
        t = self.tensor(shapes, DTYPE_OF[arr.dtype], name=name, mapped=mapped)
        self.upload(t, arr)
        return t


def strided_view(buf, tc):
    dt = NP_DTYPE[tc.dtype]
    es = np.dtype(dt).itemsize
    flat = buf.view(dt)
    shape = tuple(tc.shapes)
    strides = tuple(s for s in tc.strides)
    return np.lib.stride_tricks.as_strided(flat, shape=shape, strides=strides).copy()


def tensor_element_strides(t):
    tc = t.contents
    es = np.dtype(NP_DTYPE[tc.dtype]).itemsize
    return [s // es for s in tc.strides]


# --------------------------------------------------------------------------------------------------------------
class Model:
    """vkllm_models_llama2: from a GGUF file, or generated on the device from (config, seed)."""

    def __init__(self, ctx, path=None, config=None, seed=0):
        self.ctx = ctx
        self.m = ModelStruct()
        L = lib()
        if path is not None:
            check("vkllm_models_llama2_load", L.vkllm_models_llama2_load(ctx.vp, ctypes.byref(self.m), path.encode()))
        else:
            check("vkllm_models_llama2_init_random",
                  L.vkllm_models_llama2_init_random(ctx.vp, ctypes.byref(self.m), ctypes.byref(config), seed))

    def close(self):
        if self.m is not None:
            lib().vkllm_models_llama2_free(self.ctx.vp, ctypes.byref(self.m))
            self.m = None

    @property
    def meta(self):
        return self.m.meta

    def tokenize(self, text):
        ids = ctypes.POINTER(ArrayTokenId)()
        check("vkllm_models_llama2_tokenize",
              lib().vkllm_models_llama2_tokenize(ctypes.byref(self.m), text.encode(), ctypes.byref(ids)))
        a = ids.contents
        out = [a.data[i] for i in range(a.used_n)]
        # the array is malloc'd by the library's inline helpers; release it with libc
        libc = ctypes.CDLL(None)
        libc.free.argtypes = [ctypes.c_void_p]
        libc.free(ctypes.cast(a.data, ctypes.c_void_p))
        libc.free(ctypes.cast(ids, ctypes.c_void_p))
        return out

    def time_kernel(self, family, reps):
        """Average nanoseconds of `reps` back-to-back launches of a decode kernel (after a decode step)."""
        ns = ctypes.c_uint64()
        check("vkllm_hip_model_time_kernel", lib().vkllm_hip_model_time_kernel(
            self.ctx.vp, ctypes.byref(self.m), family.encode(), reps, ctypes.byref(ns)))
        return ns.value / reps

    def last_logits(self, rows):
        out = np.zeros((rows, self.meta.vocab_size), dtype=np.float16)
        check("vkllm_hip_model_last_logits",
              lib().vkllm_hip_model_last_logits(self.ctx.vp, ctypes.byref(self.m), out.ctypes.data, rows))
        return out

    def step(self, toks, offset):
        """One pass of the reference loop body (tests/vkllm_test_infer_gguf.c:183-270) for `toks` at `offset`:
        tensor_new(input_toks, mapped) -> graph_new -> build_graph -> graph_init -> upload -> graph_run ->
        post_run -> invalid_cache -> read the output ids -> graph_free. Returns the S arg-max ids."""
        L = lib()
        ctx = self.ctx
        toks = np.ascontiguousarray(toks, dtype=np.uint32)
        S = len(toks)
        inp = ctx.tensor([1, 1, 1, S], U32, name="input_toks", mapped=True)
        g = ctypes.POINTER(Graph)()
        check("vkllm_graph_new", L.vkllm_graph_new(ctx.vp, ctypes.byref(g)))
        rc = L.vkllm_models_llama2_build_graph(ctx.vp, ctypes.byref(self.m), inp, g, offset)
        if rc != ERR_OK:  # build_graph frees the graph (and the input it holds) on failure
            raise VkllmError("vkllm_models_llama2_build_graph", rc)
        try:
            check("vkllm_graph_init", L.vkllm_graph_init(ctx.vp, g))
            gc = g.contents
            check("vkllm_commands_upload", L.vkllm_commands_upload(ctx.vp, gc.commands, inp, toks.ctypes.data,
                                                                    toks.nbytes))
            check("vkllm_graph_run", L.vkllm_graph_run(ctx.vp, g))
            check("vkllm_graph_post_run", L.vkllm_graph_post_run(ctx.vp, g))
            out = gc.output_node
            check("vkllm_tensor_invalid_cache", L.vkllm_tensor_invalid_cache(ctx.vp, out))
            oc = out.contents
            ids = np.ctypeslib.as_array(ctypes.cast(oc.data.host, ctypes.POINTER(ctypes.c_uint32)), shape=(S,))
            return ids.copy()
        finally:
            L.vkllm_graph_free(ctx.vp, g)

    def loop(self, prompt, n_steps, offset=0):
        """The reference driver's loop run in C (vkllm_hip_token_loop): returns (ids [n_steps], per-step wall
        nanoseconds [n_steps], phase nanoseconds summed over steps 1.. [build, init+upload, run, free])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        ids = np.zeros(n_steps, np.uint32)
        step_ns = np.zeros(n_steps, np.uint64)
        phase_ns = np.zeros(4, np.uint64)
        check("vkllm_hip_token_loop", lib().vkllm_hip_token_loop(
            self.ctx.vp, ctypes.byref(self.m), prompt.ctypes.data, len(prompt), offset, n_steps, ids.ctypes.data,
            step_ns.ctypes.data, phase_ns.ctypes.data))
        return ids, step_ns, phase_ns

    def token_loop(self, prompt, n_steps, want_logits=False):
        """Prefill `prompt`, then feed back the arg max of the last row; n_steps ids (the first from prefill)."""
        out, logits = [], []
        toks = np.asarray(prompt, dtype=np.uint32)
        offset = 0
        for _ in range(n_steps):
            ids = self.step(toks, offset)
            if want_logits:
                logits.append(self.last_logits(len(toks))[-1])
            offset += len(toks)
            out.append(int(ids[-1]))
            toks = np.array([out[-1]], dtype=np.uint32)
        return np.array(out, dtype=np.uint32), (np.stack(logits) if want_logits else None)


def splitmix64(stream, n):
    """Counter-based SplitMix64 word n of `stream`: the generator behind every synthetic input of this library."""
    m = (1 << 64) - 1
    z = (stream + (n + 1) * 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def prompt_tokens(seed, n, vocab):
    """Uniform-random prompt: token i = splitmix64(seed, i) mod vocab."""
    return np.array([splitmix64(seed, i) % vocab for i in range(n)], dtype=np.uint32)


def llama_config(n_layer, dim, n_head, ffn, vocab=32000, ctx=256, eps=1e-5, theta=10000.0, std=0.02):
    return LlamaConfig(n_layer, dim, n_head, ffn, vocab, ctx, eps, theta, std)
