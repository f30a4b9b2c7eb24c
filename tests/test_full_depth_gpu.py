"""The full-depth LLaMA-2-7B and -13B shapes against the oracle, at the depths and widths that bench.py times (7B: 32
layers, dim 4096, 32 heads of 128, FFN 11008; 13B: 40 layers, dim 5120, 40 heads of 128, FFN 13824; vocabulary
32000). The 7B case runs the 7B workload's own 128-token prompt (seed 1, the streamed short-prompt products with the
token-split QKV product) and 16 decode steps; the 13B case an 8-token prompt and 4 steps. Decode is teacher-forced:
every step is fed the oracle's id, so the logits of every step are compared on the same inputs. The prompt step also
runs on the tile GEMMs (VKLLM_PREFILL_TILED=0), another fp32 summation order of this library, to the same bar. The
C token loop that bench.py times (vkllm_hip_token_loop, tests/vkllm_test_infer_gguf.c:181-272) runs free.

Bar, logits. At full depth no fp32 summation order stays within the 2e-2 of the one- and two-layer tests: a sum in
another order lands on the neighbouring fp16 value now and then at one of the reference graph's rounding points, and
those one-ulp differences accumulate through the residual stream. The scale comes from the oracle alone: the same
model run twice on the CPU, once with double sums and once with sequential fp32 sums (oracle_set_accumulation; every
fp16 rounding point the same), gives the distance between two valid orders of the reference's graph at this depth.
The library's logits may be at most twice that distance from the double-sum oracle, in max and in rms, and at most
0.1 absolute. A dropped term, a wrong sign or a misplaced row moves logits of magnitude ~6 by far more.

Bar, ids. At every row (prompt rows and decode steps) whose oracle top-1/top-2 margin exceeds 2e-2 and on which the
two oracle orders agree, the library's arg max is the oracle's. The free-running C loop's ids equal the oracle's up
to the first step where that does not hold.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ABS_CAP = 0.1
MARGIN = 2e-2

# (shape, prompt tokens, decode steps)
CASES = {
    "7b": (dict(n_layer=32, dim=4096, n_head=32, ffn=11008, vocab=32000, ctx=160), 128, 16),
    "13b": (dict(n_layer=40, dim=5120, n_head=40, ffn=13824, vocab=32000, ctx=64), 8, 4),
}


def _oracle_run(oracle, cfg, prompt, n_steps, fp32_sequential, forced=None):
    """Prompt step, then n_steps single-token steps fed forced[i] (or the run's own previous id). Returns every
    row's logits [P + n_steps, V] and the ids fed to the decode steps [n_steps + 1] (its own arg maxes)."""
    oracle.set_accumulation(fp32_sequential)
    m = oracle.Model(cfg=cfg, seed=0)
    try:
        ids, lg, _ = m.step(prompt, 0, want_logits=True)
        rows, own = [lg], [int(ids[-1])]
        for i in range(n_steps):
            tok = forced[i] if forced is not None else own[-1]
            ids1, lg1, _ = m.step(np.array([tok], np.uint32), len(prompt) + i, want_logits=True)
            rows.append(lg1)
            own.append(int(ids1[0]))
    finally:
        m.close()
        oracle.set_accumulation(False)
    return np.concatenate(rows).astype(np.float32), own


def _gpu_forced(ctx, vk, shape, prompt, forced):
    vcfg = vk.llama_config(shape["n_layer"], shape["dim"], shape["n_head"], shape["ffn"], shape["vocab"],
                           shape["ctx"])
    model = vk.Model(ctx, config=vcfg, seed=0)
    try:
        model.step(prompt, 0)
        rows = [model.last_logits(len(prompt))]
        for i, tok in enumerate(forced):
            model.step(np.array([tok], np.uint32), len(prompt) + i)
            rows.append(model.last_logits(1))
        c_ids = model.loop(prompt, len(forced) + 1)[0]
    finally:
        model.close()
    return np.concatenate(rows).astype(np.float32), c_ids


@pytest.mark.timeout(900)  # the oracle runs the full depth twice on the host's cores
@pytest.mark.parametrize("name", sorted(CASES))
def test_full_depth(ctx, vk, oracle, monkeypatch, name):
    shape, prompt_len, n_steps = CASES[name]
    cfg = oracle.make_cfg(**shape)
    prompt = oracle.prompt_tokens(1, prompt_len, cfg.vocab)
    print(f"[{name}] oracle, double sums", flush=True)
    want, own = _oracle_run(oracle, cfg, prompt, n_steps, False)
    forced = own[:n_steps]  # the id each decode step is fed
    print(f"[{name}] oracle, sequential fp32 sums", flush=True)
    want32, _ = _oracle_run(oracle, cfg, prompt, n_steps, True, forced)
    d_orders = want32 - want
    spread, rms_spread = float(np.abs(d_orders).max()), float(np.sqrt(np.mean(d_orders ** 2)))
    print(f"[{name}] between the oracle's two orders: max {spread:.4f}, rms {rms_spread:.5f}", flush=True)
    assert spread > 0

    top2 = np.sort(want, axis=1)[:, -2:]
    decided = (top2[:, 1] - top2[:, 0] > MARGIN) & (want.argmax(1) == want32.argmax(1))
    print(f"[{name}] {int(decided.sum())} of {len(want)} rows decided by the oracle", flush=True)

    got, c_ids = _gpu_forced(ctx, vk, shape, prompt, forced)
    monkeypatch.setenv("VKLLM_PREFILL_TILED", "0")  # read when a model's first short prompt arrives
    alt, _ = _gpu_forced(ctx, vk, shape, prompt, forced[:0])
    monkeypatch.delenv("VKLLM_PREFILL_TILED")

    for what, g in (("streamed prompt products", got), ("tile-GEMM prompt products", alt)):
        d = g - want[:len(g)]
        err, rms_err = float(np.abs(d).max()), float(np.sqrt(np.mean(d ** 2)))
        print(f"[{name}] {what}: max|dlogit| {err:.4f} (rms {rms_err:.5f}) against bars {2 * spread:.4f} "
              f"(rms {2 * rms_spread:.5f})", flush=True)
        assert err <= ABS_CAP and err <= 2 * spread and rms_err <= 2 * rms_spread, what
        n = len(g)
        bad = np.nonzero(decided[:n] & (g.argmax(1) != want[:n].argmax(1)))[0]
        assert bad.size == 0, f"{what}: arg max differs from the oracle on decided rows {bad.tolist()}"

    # the free-running C loop: ids equal to the oracle's own stream up to its first undecided step
    steps_decided = decided[prompt_len - 1:]
    upto = int(np.argmin(steps_decided)) if not steps_decided.all() else len(steps_decided)
    print(f"[{name}] C loop ids {c_ids.tolist()}, oracle {own}; compared through step {upto}", flush=True)
    assert c_ids[:upto].tolist() == own[:upto]
