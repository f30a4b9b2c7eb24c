"""bench.py on the CPU: the multi-GPU refusal of its command line, and its decode byte accounting (the numerator of
every HBM roofline fraction it prints) against the closed form of the workload's algorithmic bytes per token:
2 [L (4 d^2 + 3 d F) + V d] (fp16 weights) + 4 L d kv (K and V rows read) + 4 L d (the step's K and V rows written)
+ 2 d (the embedding row) + 4 d (2 L + 1) (fp32 norm weights). bench.py also counts the activation vectors, a few
hundredths of a percent at the 7B and 13B widths; a dropped weight matrix or cache term moves it by percents."""
import importlib.util
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BENCH = os.path.join(HERE, "..", "bench.py")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _closed_form(shape, kv):
    L, d, F, V = shape["n_layer"], shape["dim"], shape["ffn"], shape["vocab"]
    return 2 * (L * (4 * d * d + 3 * d * F) + V * d) + 4 * L * d * kv + 4 * L * d + 2 * d + 4 * d * (2 * L + 1)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("name,tol", [("7b", 5e-4), ("13b", 5e-4), ("tiny", 5e-3)])
@pytest.mark.parametrize("kv", [1, 129, 1024, 4096])
def test_decode_bytes_per_token(name, tol, kv):
    b = _bench()
    shape = b.CONFIGS[name]["shape"]
    got, want = b.step_bytes(shape, kv), _closed_form(shape, kv)
    assert want <= got <= want * (1 + tol), (name, kv, got, want)


def test_seven_b_bytes_at_the_quoted_cache_lengths():
    # 13.214 GB + 0.524 MB per cached position: 13.28 GB at kv 129, 13.75 at 1k, 14.29 at 2k, 15.36 at 4k
    b = _bench()
    for kv, gb in ((129, 13.28), (1024, 13.75), (2048, 14.29), (4096, 15.36)):
        assert abs(b.step_bytes(b.SHAPE_7B, kv) / 1e9 - gb) < 0.01, kv
