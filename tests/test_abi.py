"""The C ABI of libvkllm without a GPU: the library loads, exports every function that include/vkllm/*.h declares,
and its public struct layouts match the ctypes mirrors the tests and bench use (no compute calls)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include", "vkllm")


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        text = re.sub(r"#[^\n]*", " ", text)
        for m in re.finditer(r"\bextern\s+(?!\"C\")([^;{}()]*?)\b([A-Za-z_]\w*)\s*\(", text):
            names.add(m.group(2))
    return names


def test_headers_declare_the_api():
    names = declared_functions()
    for must in ("vkllm_context_new", "vkllm_graph_run", "vkllm_models_llama2_build_graph", "vkllm_op_matmul_run",
                 "vkllm_hip_gemm", "vkllm_hip_token_loop", "vkllm_hashmap_insert"):
        assert must in names
    assert len(names) > 80


def test_library_exports_every_declared_function(vk):
    L = vk.lib()
    missing = []
    for name in sorted(declared_functions()):
        try:
            getattr(L, name)
        except AttributeError:
            missing.append(name)
    assert not missing, f"declared in include/vkllm but not exported: {missing}"


def test_exports_are_c_symbols(vk):
    """Every declared function is an unmangled dynamic symbol (extern "C"), not only reachable through C++ names."""
    out = subprocess.run(["nm", "-D", "--defined-only", vk.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}
    missing = sorted(declared_functions() - exported)
    assert not missing, missing


def test_struct_layouts_match_the_ctypes_mirrors(vk):
    assert vk.abi_check() == {}


def test_error_strings_without_a_device(vk):
    assert vk.err_s(vk.ERR_OK) != ""
    assert vk.lib().vkllm_dtype_s(vk.F16) is not None
    assert isinstance(vk.lib().vkllm_hip_kernel_family_count(), int)
    assert vk.lib().vkllm_hip_kernel_family_count() > 0
