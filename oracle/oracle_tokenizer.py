"""CPU restatement of the reference's LLaMA-2 tokenizer. TEST INFRASTRUCTURE ONLY: imported by tests/ to check
vkllm_models_llama2_tokenize; the shipped library never loads it.

Follows vkllm_models_llama2_tokenize, src/models/vkllm_models_llama2.c:652-816, with its helpers
find_token_by_text (:604-614) and find_best_merge (:616-650):
  1. an empty sentence gives no ids at all (no BOS or EOS) (:661-665);
  2. "▁" is put in front and every ' ' becomes "▁" (:667-688);
  3. the bytes are split into UTF-8 characters by their lead byte: 110xxxxx two bytes, 1110xxxx three, 11110xxx four,
     any other byte (ASCII or a stray continuation byte) one (:702-741);
  4. while two or more pieces remain, the adjacent pair whose concatenation is a vocabulary text with the highest
     score is merged; the score of a text is the score of its first (lowest) id; a pair wins only with a strictly
     higher score, so among equal scores the leftmost pair merges; no such pair ends the merging (:744-774);
  5. BOS when add_bos_token, the first id of each piece's text (pieces outside the vocabulary are dropped), EOS when
     add_eos_token (:776-795).
A character cut short by the end of the sentence reads bytes past it in the reference (undefined there); here it is
the remaining bytes, as in the library.
"""
import math

SPACE = "▁".encode()


def split_utf8(b):
    """bytes -> list of byte strings, one per UTF-8 character by lead byte (src/models/vkllm_models_llama2.c:702-741)"""
    out, i = [], 0
    while i < len(b):
        c = b[i]
        n = 1
        if c >= 0x80:
            if c & 0xE0 == 0xC0:
                n = 2
            elif c & 0xF0 == 0xE0:
                n = 3
            elif c & 0xF8 == 0xF0:
                n = 4
        n = min(n, len(b) - i)
        out.append(b[i:i + n])
        i += n
    return out


def tokenize(texts, scores, sentence, bos_id=1, eos_id=2, add_bos=True, add_eos=False):
    """ids of `sentence` (str or bytes) for a vocabulary given as parallel lists of texts (str or bytes) and scores"""
    vocab = [t.encode() if isinstance(t, str) else bytes(t) for t in texts]
    first = {}
    for i, t in enumerate(vocab):
        first.setdefault(t, i)  # find_token_by_text scans from id 0
    s = sentence.encode() if isinstance(sentence, str) else bytes(sentence)
    if not s:
        return []
    pieces = split_utf8(SPACE + s.replace(b" ", SPACE))
    while len(pieces) > 1:
        best, at = -math.inf, -1
        for i in range(len(pieces) - 1):
            tid = first.get(pieces[i] + pieces[i + 1])
            if tid is not None and scores[tid] > best:
                best, at = scores[tid], i
        if at < 0:
            break
        pieces[at:at + 2] = [pieces[at] + pieces[at + 1]]
    ids = [bos_id] if add_bos else []
    ids += [first[p] for p in pieces if p in first]
    if add_eos:
        ids.append(eos_id)
    return ids
