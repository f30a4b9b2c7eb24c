"""Shared fixtures. GPU tests carry @pytest.mark.gpu and use one HIP context per session."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "vkllm.c_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libvkllm")


@pytest.fixture(scope="session")
def oracle():
    import oracle_ffi

    oracle_ffi.lib()
    return oracle_ffi


@pytest.fixture(scope="session")
def vk():
    import pyvkllm

    pyvkllm.lib()
    return pyvkllm


@pytest.fixture(scope="session")
def ctx(vk):
    c = vk.Ctx(0)
    print(f"\n[gpu] device {c.arch()}", flush=True)
    yield c
    c.close()


@pytest.fixture(scope="session")
def tiny_gguf(tmp_path_factory, oracle):
    """The tiny LLaMA-2 workload's model: dim 288, 6 layers, 6 heads, FFN 768, vocab 32000, ctx 256, seed 0."""
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    oracle.write_gguf(path, oracle.make_cfg(**oracle.TINY), 0)
    return path
