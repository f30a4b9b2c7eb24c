"""The committed fixtures of the tiny LLaMA-2 workload (tests/golden/, written by tests/golden/make_golden.py from
the oracle): the oracle must reproduce them exactly, and the HIP token loop must produce the same greedy ids with
logits within 2e-2 at the recorded entries (each step's eight largest and sixteen fixed vocabulary ids)."""
import hashlib
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LOGIT_TOL = 2e-2


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_oracle_gguf_matches_fixture(tiny_gguf):
    want = _load("tiny_gguf.json")
    data = open(tiny_gguf, "rb").read()
    assert len(data) == want["bytes"]
    assert data[:64].hex() == want["head_hex"]
    assert hashlib.sha256(data).hexdigest() == want["sha256"]


def test_oracle_reproduces_tiny_token_loop(oracle, tiny_gguf):
    want = _load("tiny_token_loop.json")
    m = oracle.Model(tiny_gguf)
    try:
        prompt = oracle.prompt_tokens(1, 16, m.cfg.vocab)
        ids, logits = m.token_loop(prompt, len(want["ids"]), want_logits=True)
    finally:
        m.close()
    assert [int(x) for x in prompt] == want["prompt"]
    assert [int(x) for x in ids] == want["ids"]
    assert hashlib.sha256(logits.astype(np.float16).tobytes()).hexdigest() == want["logits_fp16_sha256"]


@pytest.mark.gpu
def test_hip_token_loop_matches_fixture(ctx, vk, tiny_gguf):
    want = _load("tiny_token_loop.json")
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        ids, logits = model.token_loop(np.array(want["prompt"], dtype=np.uint32), len(want["ids"]), want_logits=True)
    finally:
        model.close()
    assert [int(x) for x in ids] == want["ids"]
    lf = logits.astype(np.float32)
    worst = 0.0
    for t, st in enumerate(want["steps"]):
        for i, v in st["top8"]:
            worst = max(worst, abs(float(lf[t, i]) - v))
        for i, v in zip(want["probe_ids"], st["probe"]):
            worst = max(worst, abs(float(lf[t, i]) - v))
    print(f"max |dlogit| at the recorded entries {worst:.3g}")
    assert worst <= LOGIT_TOL
