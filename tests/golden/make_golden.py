#!/usr/bin/env python3
"""Writes the committed fixtures of the tiny LLaMA-2 workload from the oracle (oracle/, the CPU restatement of the
reference's path). The reference ships no expected tokens or logits for this path and cannot run here, so these
fixtures are the oracle's own output: they pin the oracle against regressions and give the GPU tests a fixed target.

Workload (the tiny configuration): dim 288, 6 layers, 6 heads (head_dim 48), FFN 768, vocab 32000, ctx 256,
random-init GGUF from seed 0 (weights N(0, 0.02) rounded to fp16, norm weights 1.0), RMSNorm eps 1e-5, RoPE theta
1e4; prompt = 16 uniform-random ids from seed 1; 64 greedy steps (the prefill step, then 63 single-token steps).

Usage: python3 tests/golden/make_golden.py   (rewrites tests/golden/tiny_token_loop.json and tiny_gguf.json)
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))

N_STEPS = 64
PROBE_IDS = [0, 1, 2, 3, 100, 1000, 4095, 4096, 12345, 16000, 20000, 25000, 29999, 31000, 31998, 31999]


def token_loop_fixture(oracle, path):
    m = oracle.Model(path)
    try:
        prompt = oracle.prompt_tokens(1, 16, m.cfg.vocab)
        ids, logits = m.token_loop(prompt, N_STEPS, want_logits=True)
    finally:
        m.close()
    lf = logits.astype(np.float32)
    steps = []
    for t in range(N_STEPS):
        top = np.argsort(-lf[t], kind="stable")[:8]
        steps.append({
            "id": int(ids[t]),
            "top8": [[int(i), float(lf[t, i])] for i in top],
            "probe": [float(lf[t, i]) for i in PROBE_IDS],
        })
    return {
        "workload": "tiny LLaMA-2 (dim 288, 6 layers, 6 heads, FFN 768, vocab 32000, ctx 256), GGUF seed 0, "
                    "16-token prompt from seed 1, 64 greedy steps",
        "prompt": [int(x) for x in prompt],
        "ids": [int(x) for x in ids],
        "probe_ids": PROBE_IDS,
        "logits_fp16_sha256": hashlib.sha256(logits.astype(np.float16).tobytes()).hexdigest(),
        "steps": steps,
    }


def gguf_fixture(path):
    data = open(path, "rb").read()
    return {
        "workload": "tiny LLaMA-2 random-init GGUF written by the oracle from seed 0",
        "bytes": len(data),
        "sha256": hashlib.sha256(data).hexdigest(),
        "head_hex": data[:64].hex(),
    }


def main():
    import oracle_ffi as oracle

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        oracle.write_gguf(path, oracle.make_cfg(**oracle.TINY), 0)
        g = gguf_fixture(path)
        t = token_loop_fixture(oracle, path)
    with open(os.path.join(HERE, "tiny_gguf.json"), "w") as f:
        json.dump(g, f, indent=1)
        f.write("\n")
    with open(os.path.join(HERE, "tiny_token_loop.json"), "w") as f:
        json.dump(t, f, indent=1)
        f.write("\n")
    print(f"ids {t['ids'][:8]}... gguf {g['bytes']} bytes sha256 {g['sha256'][:16]}")


if __name__ == "__main__":
    main()
