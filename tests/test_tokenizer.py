"""vkllm_models_llama2_tokenize (src/models/vkllm_models_llama2.c:604-816): the best-score pair merge.

The CPU restatement (oracle/oracle_tokenizer.py) is pinned by answers derived by hand on small vocabularies: the
leftmost pair wins a tie, a text repeated in the vocabulary scores and returns as its first id, pieces outside the
vocabulary are dropped, characters of 2, 3 and 4 UTF-8 bytes are single pieces, an empty sentence has no ids. The
GPU tests load GGUF files with such vocabularies through vkllm_models_llama2_load and compare the library's ids with
the restatement: the hand cases, and random sentences on a vocabulary of every string of up to three characters of
a mixed-width alphabet, scored with many ties and with repeated texts, so merges run several steps deep.
"""
import itertools
import os

import numpy as np
import pytest

import gguf_util

SPECIALS = ["<unk>", "<s>", "</s>"]
# ids 3..: the hand vocabulary (texts, scores); "ab" appears twice, the second time with a higher score
HAND = [("▁", -10), ("a", -10), ("b", -10), ("c", -10), ("ab", -1), ("bc", -1), ("▁ab", -4), ("▁a", -5),
        ("日", -10), ("本", -10), ("日本", -1), ("▁日本", -2), ("é", -10), ("🙂", -10), ("ab", 5)]


def hand_vocab(bc_score=-1):
    texts = SPECIALS + [t for t, _ in HAND]
    scores = [0.0, 0.0, 0.0] + [float(s) for _, s in HAND]
    scores[texts.index("bc")] = float(bc_score)
    return texts, scores


def ids_of(texts, *pieces):
    return [texts.index(p) for p in pieces]


@pytest.fixture(scope="module")
def tok():
    import oracle_tokenizer

    return oracle_tokenizer


def test_leftmost_pair_wins_a_tie(tok):
    texts, scores = hand_vocab()
    # ▁abc: "ab" and "bc" both score -1; the leftmost merges, then "▁ab"; the rightmost would give ▁a + bc
    assert tok.tokenize(texts, scores, "abc") == [1] + ids_of(texts, "▁ab", "c")


def test_repeated_text_scores_and_returns_as_its_first_id(tok):
    texts, scores = hand_vocab(bc_score=0)
    # "ab" scores -1 (its first id), so "bc" (0) merges first: ▁a + bc. With the second "ab" (+5) it would be ▁ab + c
    assert tok.tokenize(texts, scores, "abc") == [1] + ids_of(texts, "▁a", "bc")
    # a final piece "ab" is the first id of that text
    assert tok.tokenize(texts, scores, "cab") == [1] + ids_of(texts, "▁", "c", "ab")
    assert texts.index("ab") == 7


def test_multibyte_characters_and_dropped_pieces(tok):
    texts, scores = hand_vocab()
    assert tok.tokenize(texts, scores, "日本") == [1] + ids_of(texts, "▁日本")
    assert tok.tokenize(texts, scores, "é🙂x") == [1] + ids_of(texts, "▁", "é", "🙂")  # 'x' has no id
    assert tok.tokenize(texts, scores, "b ab") == [1] + ids_of(texts, "▁", "b", "▁ab")
    assert tok.tokenize(texts, scores, " ") == [1] + ids_of(texts, "▁", "▁")


def test_empty_sentence_and_eos(tok):
    texts, scores = hand_vocab()
    assert tok.tokenize(texts, scores, "") == []
    assert tok.tokenize(texts, scores, "") == tok.tokenize(texts, scores, "", add_eos=True)
    assert tok.tokenize(texts, scores, "a", add_eos=True, add_bos=False) == ids_of(texts, "▁a") + [2]


def test_split_utf8_by_lead_byte(tok):
    assert tok.split_utf8("aé日🙂".encode()) == [b"a", "é".encode(), "日".encode(), "🙂".encode()]
    assert tok.split_utf8(b"\x80a") == [b"\x80", b"a"]  # a stray continuation byte is one piece
    assert tok.split_utf8("日".encode()[:2]) == ["日".encode()[:2]]  # cut short at the end


ALPHABET = ["a", "b", "c", "▁", "é", "日", "本", "🙂"]


def random_vocab(seed):
    """every string of 1-3 alphabet characters, scores from a few values (many ties), some texts repeated later with
    another score"""
    rng = np.random.default_rng(seed)
    texts = list(SPECIALS)
    for n in (1, 2, 3):
        texts += ["".join(p) for p in itertools.product(ALPHABET, repeat=n)]
    scores = [0.0, 0.0, 0.0] + [float(rng.integers(-6, 0)) for _ in texts[3:]]
    dup = rng.choice(np.arange(3, len(texts)), 40, replace=False)
    texts += [texts[i] for i in dup]
    scores += [float(rng.integers(-6, 3)) for _ in dup]
    # a few multi-character texts are missing, so some merges stop early
    for i in rng.choice(np.arange(3 + len(ALPHABET), len(texts)), 60, replace=False):
        texts[i] = texts[i] + "#"
    return texts, scores


def random_sentences(seed, n):
    rng = np.random.default_rng(seed)
    chars = ["a", "b", "c", " ", "é", "日", "本", "🙂", "x"]
    return ["".join(rng.choice(chars, rng.integers(1, 14))) for _ in range(n)]


@pytest.mark.gpu
@pytest.mark.parametrize("bc_score,add_eos", [(-1, False), (0, True)])
def test_library_tokenizer_hand_vocabulary(ctx, vk, tok, tmp_path, bc_score, add_eos):
    texts, scores = hand_vocab(bc_score)
    path = str(tmp_path / "hand.gguf")
    gguf_util.llama_model(path, texts, scores, add_eos=add_eos)
    model = vk.Model(ctx, path=path)
    try:
        for s in ["abc", "cab", "日本", "é🙂x", "b ab", " ", "", "abcabc ab 日本本", "xyz"]:
            want = tok.tokenize(texts, scores, s, add_eos=add_eos)
            assert model.tokenize(s) == want, s
    finally:
        model.close()


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1])
def test_library_tokenizer_random_vocabulary(ctx, vk, tok, tmp_path, seed):
    texts, scores = random_vocab(seed)
    path = str(tmp_path / f"rand{seed}.gguf")
    gguf_util.llama_model(path, texts, scores)
    model = vk.Model(ctx, path=path)
    deep = 0
    try:
        for s in random_sentences(seed + 10, 300):
            want = tok.tokenize(texts, scores, s)
            assert model.tokenize(s) == want, s
            deep += len(want) - 1 < len(s) // 2  # at least two characters per piece on average: merges chained
    finally:
        model.close()
    assert deep > 30


@pytest.mark.gpu
def test_library_tokenizer_tiny_workload_vocabulary(ctx, vk, tok, tiny_gguf):
    """the tiny workload's vocabulary and the reference driver's prompt (tests/vkllm_test_infer_gguf.c:160)"""
    from test_oracle import parse_gguf

    _, kv, _, _, _ = parse_gguf(tiny_gguf)
    texts, scores = kv["tokenizer.ggml.tokens"][1], kv["tokenizer.ggml.scores"][1]
    add_bos = kv.get("tokenizer.ggml.add_bos_token", (7, True))[1]
    add_eos = kv.get("tokenizer.ggml.add_eos_token", (7, True))[1]
    model = vk.Model(ctx, path=tiny_gguf)
    try:
        for s in ["Q: What is the largest animal? A:", "the blue whale is the largest animal", "a"]:
            assert model.tokenize(s) == tok.tokenize(texts, scores, s, add_bos=bool(add_bos), add_eos=bool(add_eos))
    finally:
        model.close()
