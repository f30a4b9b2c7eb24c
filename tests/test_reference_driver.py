"""The reference's own token-loop driver (tests/vkllm_test_infer_gguf.c) on this library: the source-level drop-in.

The driver is compiled unchanged from the reference tree against include/ (its "src/core/..." includes are
one-line forwarding headers) and linked with libvkllm.so, by the ref_driver recipe of oracle/Makefile into
oracle/_ref/. The CPU test compiles it into a temporary directory (skipped where the reference tree is absent);
the GPU test runs the binary build() left in oracle/_ref/ on the tiny LLaMA-2 workload's GGUF and requires the
oracle's greedy token stream (skipped where that binary was not built). Nothing from the reference is copied into
this repository.
"""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE = "/root/reference"
DRIVER_SRC = os.path.join(REFERENCE, "tests", "vkllm_test_infer_gguf.c")
DRIVER_BIN = os.path.join(ROOT, "oracle", "_ref", "vkllm_test_infer_gguf")
LIB_DIR = os.path.join(ROOT, "vkllm.c_amd", "build")


@pytest.mark.skipif(not os.path.exists(DRIVER_SRC), reason="the reference tree is not present")
@pytest.mark.parametrize("timing", [False, True], ids=["plain", "node_time_cost"])
def test_reference_driver_compiles_against_the_headers(tmp_path, timing):
    if not os.path.exists(os.path.join(LIB_DIR, "libvkllm.so")):
        pytest.skip("libvkllm.so is not built")
    subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle"), f"REF={REFERENCE}",
                           "_ref/inc/.stamp"])
    inc = os.path.join(ROOT, "oracle", "_ref", "inc")
    out = str(tmp_path / "driver")
    cmd = ["gcc", "-O2", "-std=gnu11", "-Wall", "-Werror", "-Wno-unused-function", "-Wno-unused-variable",
           "-Wno-unused-but-set-variable", "-Wno-unused-label", "-I", inc, "-I", os.path.join(ROOT, "include"),
           DRIVER_SRC, "-L", LIB_DIR, "-lvkllm", "-lm", "-o", out]
    if timing:
        cmd.insert(1, "-D_LOG_NODE_TIME_COST=1")
    subprocess.check_call(cmd)
    assert os.path.exists(out)


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(DRIVER_BIN), reason="oracle/_ref/vkllm_test_infer_gguf was not built")
def test_reference_driver_runs_the_oracle_token_stream(oracle, tiny_gguf):
    from test_oracle import parse_gguf

    n = 24
    print(f"[driver] {DRIVER_BIN} {tiny_gguf} {n}", flush=True)
    r = subprocess.run([DRIVER_BIN, tiny_gguf, str(n)], capture_output=True, text=True, timeout=120)
    # the driver's main returns its last vkllm_err_t: VKLLM_ERR_OK is 1 (tests/vkllm_test_infer_gguf.c:324)
    assert r.returncode == 1, r.stderr[-2000:]
    # the driver prints the prompt's ids on stderr ("input ids: ..."), the generated pieces on stdout
    m = re.search(r"input ids: ([0-9 ]+)", r.stderr)
    assert m, r.stderr[-2000:]
    prompt = np.array([int(t) for t in m.group(1).split()], np.uint32)
    ref = oracle.Model(tiny_gguf)
    try:
        want_ids, _ = ref.token_loop(prompt, n)
    finally:
        ref.close()
    _, kv, _, _, _ = parse_gguf(tiny_gguf)
    texts = kv["tokenizer.ggml.tokens"][1]
    want = "".join(texts[i] for i in want_ids)
    print(f"[driver] prompt {prompt.tolist()} -> {r.stdout[:120]!r}")
    assert r.stdout == want


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(DRIVER_BIN + "_timing"),
                    reason="oracle/_ref/vkllm_test_infer_gguf_timing was not built")
def test_reference_driver_node_time_cost_loop(tiny_gguf):
    """The driver built with _LOG_NODE_TIME_COST sums vkllm_pipeline_query_exec_time over the graph nodes that have a
    pipeline into context->stats (tests/vkllm_test_infer_gguf.c:205-225) and prints the per-node table at the end
    (:288-313, in whole milliseconds; it adds up the decode steps only). With VKLLM_TIMING=1 the fused nodes are in
    it; without timing none is. A decode step's arg max runs in the vocabulary product's launch, charged to "logits";
    with VKLLM_ARGMAX_EPI=0 it is a launch of its own, charged to "output"."""
    for argmax_epi in ("1", "0"):
        env = dict(os.environ, VKLLM_TIMING="1", VKLLM_ARGMAX_EPI=argmax_epi)
        r = subprocess.run([DRIVER_BIN + "_timing", tiny_gguf, "8"], capture_output=True, text=True, timeout=120,
                           env=env)
        assert r.returncode == 1, r.stderr[-2000:]
        nodes = set(re.findall(r"node (\S+) total cost", r.stderr))
        print(f"[driver] VKLLM_ARGMAX_EPI={argmax_epi}: {len(nodes)} nodes timed")
        for name in ("embedded", "block.0.attn.Q", "block.5.attn.scores", "block.3.attn.final_output",
                     "block.2.ffn.up", "block.4.ffn.down", "logits"):
            assert name in nodes, name
        assert ("output" in nodes) == (argmax_epi == "0")
    r = subprocess.run([DRIVER_BIN + "_timing", tiny_gguf, "4"], capture_output=True, text=True, timeout=120,
                       env={k: v for k, v in os.environ.items() if k != "VKLLM_TIMING"})
    assert r.returncode == 1
    assert re.findall(r"node (\S+) total cost", r.stderr) == []
