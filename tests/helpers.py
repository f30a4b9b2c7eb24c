"""Test helpers: deterministic inputs, fp16 ulp comparisons, oracle views of library tensors."""
import numpy as np


def rand(shape, dtype, lo=-1.0, hi=1.0, seed=0):
    r = np.random.default_rng(seed)
    return r.uniform(lo, hi, size=shape).astype(dtype)


def fp16_ulp(x):
    """Spacing of fp16 numbers at |x| (for x in the normal range; 2^-24 below it)."""
    a = np.abs(np.asarray(x, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.float32(2.0) ** (e - 10)


def ulp_diff(got, want):
    """|got - want| in units of fp16 ulps of `want` (fp16 arrays)."""
    g = got.astype(np.float32)
    w = want.astype(np.float32)
    return np.abs(g - w) / fp16_ulp(w)


def assert_fp16_close(got, want, max_ulp=1.0, frac_exact=None, what="", atol=0.0):
    """Every element within max_ulp fp16 ulps plus `atol` (the fp32 arithmetic's absolute error, which near zero
    exceeds an ulp of the result); optionally at least frac_exact of them bit-identical."""
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    w = want.astype(np.float32)
    d = np.maximum(np.abs(got.astype(np.float32) - w) - np.asarray(atol, dtype=np.float32), 0) / fp16_ulp(w)
    worst = float(d.max()) if d.size else 0.0
    assert worst <= max_ulp, f"{what}: max diff {worst:.2f} ulp > {max_ulp} (at {np.unravel_index(d.argmax(), d.shape)})"
    if frac_exact is not None and got.size:
        same = float(np.mean(got.view(np.uint16) == want.view(np.uint16))) if got.dtype == np.float16 else 1.0
        assert same >= frac_exact, f"{what}: only {same:.4f} bit-identical (< {frac_exact})"


U32 = 2.0 ** -24


def dot_atol(a, b, transposed=True, k_axis=-1):
    """Bound on fp32 accumulation error of a matmul: 16 units of fp32 roundoff times sum_k |a_k||b_k|."""
    a64 = np.abs(a.astype(np.float64))
    b64 = np.abs(b.astype(np.float64))
    bb = np.swapaxes(b64, -1, -2) if transposed else b64
    return (16 * U32 * np.matmul(a64, bb)).astype(np.float32)


def mse(got, want):
    return float(np.mean((got.astype(np.float64) - want.astype(np.float64)) ** 2))


def bitrev5(x):
    return int(f"{x:05b}"[::-1], 2)


def argmax_tie_rule(row):
    """The reference's arg max restated as a rule (src/shaders/vkllm_arg_max.comp:40-97): among the maximal
    elements take the one whose lane (index mod 32) has the smallest 5-bit bit-reversal, then the smallest index."""
    row = np.asarray(row, dtype=np.float32)
    m = row.max()
    cand = np.nonzero(row == m)[0]
    return int(min(cand, key=lambda i: (bitrev5(int(i) % 32), int(i))))


def assert_prefill_ids(ids, want_ids, want_logits, what=""):
    """Arg-max ids of a multi-row step against the oracle's. The last row (the token the loop feeds back) must match
    exactly. An earlier row may differ only at a near-tie: the oracle's logit for the id picked here is within one
    fp16 ulp of the oracle's largest logit of that row, so fp32 summation order alone decides between them.
    Returns the number of rows that differed at such ties."""
    ids, want_ids = list(map(int, ids)), list(map(int, want_ids))
    assert len(ids) == len(want_ids)
    assert ids[-1] == want_ids[-1], f"{what}: last row id {ids[-1]} != {want_ids[-1]}"
    ties = 0
    for r, (a, b) in enumerate(zip(ids, want_ids)):
        if a == b:
            continue
        row = want_logits[r].astype(np.float32)
        top = float(row[b])
        assert top - float(row[a]) <= float(fp16_ulp(np.float32(top))), \
            f"{what}: row {r} id {a} (oracle logit {row[a]}) vs {b} ({top}): not a near-tie"
        ties += 1
    if ties:
        print(f"{what}: {ties} of {len(ids)} rows took the other id of a one-ulp tie")
    return ties


def prompt_rows(ref, model, part, offset, what, tol=2e-2):
    """One prompt step of `part` at `offset` on the oracle and the library: every row's logits within tol, ids as
    assert_prefill_ids takes them. Returns the oracle's ids and the number of one-ulp ties."""
    print(f"[{what}] prompt rows {offset}..{offset + len(part) - 1}", flush=True)
    want_ids, want_logits, _ = ref.step(part, offset, want_logits=True)
    ids = model.step(part, offset)
    logits = model.last_logits(len(part)).astype(np.float32)
    err = float(np.max(np.abs(logits - want_logits.astype(np.float32))))
    print(f"[{what}] rows {offset}..{offset + len(part) - 1}: max|dlogit| {err:.3g}", flush=True)
    assert err <= tol
    ties = assert_prefill_ids(ids, want_ids, want_logits, f"{what} rows at {offset}")
    return want_ids, ties


def forced_decode(ref, model, first_tok, offset, n, what, tol=2e-2):
    """n single-token steps from position `offset`, each fed the oracle's previous id; returns the worst logit
    difference, the number of one-ulp ties and the oracle's last id (the next step's input)."""
    tok, worst, ties = int(first_tok), 0.0, 0
    for i in range(n):
        toks = np.array([tok], np.uint32)
        want_ids, want_logits, _ = ref.step(toks, offset + i, want_logits=True)
        ids = model.step(toks, offset + i)
        logits = model.last_logits(1).astype(np.float32)
        err = float(np.max(np.abs(logits - want_logits.astype(np.float32))))
        worst = max(worst, err)
        assert err <= tol, f"{what} position {offset + i}: max|dlogit| {err}"
        a, b = int(ids[0]), int(want_ids[0])
        if a != b:
            row = want_logits[0].astype(np.float32)
            assert row[b] - row[a] <= float(fp16_ulp(row[b])), f"{what} position {offset + i}: id {a} vs {b}"
            ties += 1
        tok = b
    print(f"[{what}] decode {offset}..{offset + n - 1}: max|dlogit| {worst:.3g}, {ties} one-ulp ties", flush=True)
    return worst, ties, tok
