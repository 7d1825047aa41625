"""Pins the oracle's serving-side functions (fill_engram_ids, mask_media) against the
brute-force expectation and the multimodal cases of the reference's own test
(test_vllm_ids.py:59-98, 135-160)."""
import random

import numpy as np
import pytest

import oracle

V, MAX_REQS, MAX_LEN = 1000, 8, 64


def make_step(chunks, histories, slots, width=3, rows=MAX_REQS, max_len=MAX_LEN):
    """Inputs of one serving step: chunks = [(request, first position, count)]. The history table
    holds real tokens before each chunk and 999 from the chunk on (never read)."""
    input_ids, positions, qsl = [], [], [0]
    for r, start, n in chunks:
        input_ids += histories[r][start:start + n]
        positions += list(range(start, start + n))
        qsl.append(qsl[-1] + n)
    num_tokens = len(input_ids)
    table = np.full((rows, max_len), 999, dtype=np.int32)
    for r, start, _ in chunks:
        table[slots[r], :start] = histories[r][:start]
    return dict(input_ids=np.array(input_ids + [5] * 3, np.int32),
                positions=np.array(positions + [0] * 3, np.int64),
                idx_mapping=np.array([slots[r] for r, _, _ in chunks], np.int32),
                query_start_loc=np.array(qsl, np.int32), all_token_ids=table,
                num_reqs=len(chunks), num_tokens=num_tokens, num_tokens_padded=num_tokens + 3,
                width=width)


def expected(chunks, histories, width=3):
    """test_vllm_ids.py:59-65: (token at p, p-1, ..., -1 before the sequence start)."""
    rows = []
    for r, start, n in chunks:
        h = histories[r]
        for p in range(start, start + n):
            rows.append([h[p - k] if p >= k else -1 for k in range(width)])
    return np.array(rows, np.int32)


def run_oracle(step):
    out = np.full((step["num_tokens"] + 10, step["width"]), 777, np.int32)
    oracle.fill_engram_ids(out, step["input_ids"], step["positions"], step["idx_mapping"],
                           step["query_start_loc"], step["all_token_ids"], step["num_reqs"],
                           step["num_tokens"], step["num_tokens_padded"])
    return out


def histories(seed=0):
    rnd = random.Random(seed)
    return {r: [rnd.randrange(5, V) for _ in range(MAX_LEN)] for r in range(4)}


SLOTS = {0: 5, 1: 2, 2: 7, 3: 0}
CASES = {  # test_vllm_ids.py:84-98
    "full prefill": [(0, 0, 20)],
    "chunked prefill, 2nd chunk": [(0, 20, 15)],
    "prefix-cache hit": [(1, 33, 4)],
    "decode steps": [(0, 40, 1), (1, 37, 1), (2, 2, 1)],
    "decode at position 0 and 1": [(3, 0, 1), (2, 1, 1)],
    "mixed prefill + decode": [(0, 41, 1), (1, 0, 9), (2, 10, 2), (3, 50, 1)],
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("width", [3, 4, 1])
def test_fill_matches_bruteforce(name, width):
    h = histories()
    step = make_step(CASES[name], h, SLOTS, width)
    out = run_oracle(step)
    n, padded = step["num_tokens"], step["num_tokens_padded"]
    assert np.array_equal(out[:n], expected(CASES[name], h, width))
    assert (out[n:padded] == -1).all() and (out[padded:] == 777).all()


def test_fill_zero_tokens_pads_only():
    out = np.full((6, 3), 777, np.int32)
    oracle.fill_engram_ids(out, np.zeros(0, np.int32), np.zeros(0), np.zeros(0, np.int32),
                           np.zeros(1, np.int32), np.zeros((1, 4), np.int32), 0, 0, 4)
    assert (out[:4] == -1).all() and (out[4:] == 777).all()


def test_mask_media_cases():
    # test_vllm_ids.py:135-160: text, 4 image placeholders, text
    h = histories()
    IMG = 900
    seq = h[0][:6] + [IMG] * 4 + h[0][6:14]
    step = make_step([(0, 0, len(seq))], {0: seq}, {0: 3})
    out = run_oracle(step)[:len(seq)]
    ids, keep = oracle.mask_media(out, [IMG, 901])
    assert not keep[6:10].any() and keep[:6].all() and keep[10:].all()
    assert (ids[6:10, 0] == -1).all() and ids[6, 1] == out[6, 1]  # text before the image stays
    # right after the image: the history is missing, as at a sequence start
    assert ids[10, 1] == -1 and ids[10, 2] == -1 and ids[11, 2] == -1
    assert np.array_equal(ids[:6], out[:6])
    plain, plain_keep = oracle.mask_media(out, [7777])
    assert np.array_equal(plain, out) and plain_keep.all()
