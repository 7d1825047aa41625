"""Pins the oracle's integer half (multipliers and n-gram hashing) against things other than
itself: published known answers, torch's own generator, exact big-integer arithmetic and the
invariants the reference's tests check (test_canon.py:42-56, test_vllm_ids.py:68-83)."""
import numpy as np
import pytest
import torch

import oracle

P = oracle.PRIME


def test_mt19937_known_answer():
    # C++11 [rand.predef]: the 10000th output of a default-constructed mt19937 is 4123659995
    assert int(oracle.mt19937(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("seed", [0, 1, 7, 290_203, 10007 * 5, 2**32 - 1])
@pytest.mark.parametrize("shape", [(16, 3), (24, 4), (4, 2), (3, 8)])
def test_mults_match_torch_generator(seed, shape):
    # the reference draws the multipliers with torch's CPU generator (module.py:94-99)
    gen = torch.Generator().manual_seed(seed)
    want = torch.randint(1, P, shape, generator=gen, device="cpu") | 1
    got = oracle.make_mults(seed, *shape)
    assert np.array_equal(want.numpy(), got)
    assert (got % 2 == 1).all() and (got >= 1).all() and (got <= P).all()


def _random_case(rng, B, T, vocab, orders_heads=((2, 2), (3, 2)), sizes=None, with_pos=True):
    orders = []
    for n, heads in orders_heads:
        orders += [n] * heads
    max_o = max(orders)
    sizes = sizes or {n: int(rng.integers(1, 5000)) for n, _ in orders_heads}
    rows = [sizes[n] for n in orders]
    mults = oracle.make_mults(int(rng.integers(0, 1000)), len(orders), max_o)
    canon = rng.integers(0, vocab, size=vocab)
    ids = rng.integers(-3, vocab + 3, size=(B, T))  # out-of-range ids are clamped
    pos = None
    if with_pos:
        pos = np.stack([np.concatenate([np.arange(a) for a in _doc_lengths(rng, T)]) for _ in range(B)])
    return ids, pos, canon, mults, orders, rows


def _doc_lengths(rng, T):
    out, left = [], T
    while left:
        n = int(min(left, rng.integers(1, 9)))
        out.append(n)
        left -= n
    return out


def _bigint_hash(ids, pos, canon, mults, orders, rows, pad):
    """Independent brute force in Python integers: token (b, t-i) enters when t-i >= 0 and
    (no positions or pos >= i), else the raw pad id; ids clamped into the vocab first."""
    B, T = ids.shape
    V = canon.size
    out = np.empty((len(orders), B, T), dtype=np.int64)
    for b in range(B):
        for t in range(T):
            toks = []
            for i in range(max(orders)):
                ok = t - i >= 0 and (i == 0 or pos is None or pos[b, t] >= i)
                toks.append(int(canon[min(max(int(ids[b, t - i]), 0), V - 1)]) if ok else pad)
            for k, n in enumerate(orders):
                out[k, b, t] = oracle.hash_bigint(toks, mults[k], n, rows[k])
    return out


@pytest.mark.parametrize("seed", range(6))
def test_hash_ids_equals_bigint_bruteforce(seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    ids, pos, canon, mults, orders, rows = _random_case(rng, 3, 23, 500, with_pos=seed % 2 == 0)
    pad = int(rng.integers(0, 500))
    got = oracle.hash_ids(ids, mults, orders, rows, canon, pad, position_ids=pos)
    assert np.array_equal(got, _bigint_hash(ids, pos, canon, mults, orders, rows, pad))


def test_hash_ids_4gram_mixed_sizes():
    # 4-grams with per-order sizes 257/401/97 (test_vllm_ids.py:118-132)
    rng = np.random.Generator(np.random.PCG64(11))
    ids, pos, canon, mults, orders, rows = _random_case(
        rng, 2, 30, 1000, orders_heads=((2, 2), (3, 2), (4, 2)), sizes={2: 257, 3: 401, 4: 97})
    got = oracle.hash_ids(ids, mults, orders, rows, canon, 0, position_ids=pos)
    assert np.array_equal(got, _bigint_hash(ids, pos, canon, mults, orders, rows, 0))
    for k, r in enumerate(rows):
        assert got[k].min() >= 0 and got[k].max() < r


def test_hash_rows_exceeding_prime_are_identity_mod():
    # a table with more rows than 2^31-1: the second modulo changes nothing
    mults = oracle.make_mults(3, 2, 2)
    ids = np.array([[5, 9, 123456]])
    big = oracle.hash_ids(ids, mults, [2, 2], [P + 5, 2**40], np.arange(200000), 0)
    ref = oracle.hash_ids(ids, mults, [2, 2], [P, P], np.arange(200000), 0)
    assert np.array_equal(big, ref)


def test_canon_merged_variants_hash_identically():
    # test_canon.py:47-56
    V = 1000
    mults = oracle.make_mults(0, 4, 3)
    orders, rows = [2, 2, 3, 3], [257] * 4
    canon = np.arange(V)
    canon[11], canon[501] = 10, 500
    a = np.array([[3, 10, 7, 500, 9, 10, 4]])
    b = np.array([[3, 11, 7, 501, 9, 11, 4]])
    c = np.array([[3, 12, 7, 500, 9, 10, 4]])
    ha, hb, hc = (oracle.hash_ids(x, mults, orders, rows, canon, 0) for x in (a, b, c))
    assert np.array_equal(ha, hb)
    assert not np.array_equal(ha, hc)


def test_identity_canon_is_original_hashing():
    # test_canon.py:42-45: with the identity map, hashing equals the map-free formula
    rng = np.random.Generator(np.random.PCG64(2))
    V = 1000
    ids = rng.integers(5, V, size=(3, 20))
    mults = oracle.make_mults(0, 4, 3)
    orders, rows = [2, 2, 3, 3], [257] * 4
    got = oracle.hash_ids(ids, mults, orders, rows, np.arange(V), 0)
    assert np.array_equal(got, _bigint_hash(ids, None, np.arange(V), mults, orders, rows, 0))


@pytest.mark.parametrize("packed", [False, True])
def test_hash_prev_equals_hash_ids(packed):
    # test_vllm_ids.py:68-83: the [N, max_order] predecessor matrix hashes like the sequence
    V = 1000
    rng = np.random.Generator(np.random.PCG64(5))
    ids = rng.integers(5, V, size=(1, 30))
    ids[0, 3], ids[0, 9] = 11, 501
    canon = np.arange(V)
    canon[11], canon[501] = 10, 500
    mults = oracle.make_mults(0, 4, 3)
    orders, rows = [2, 2, 3, 3], [257] * 4
    pos = np.concatenate([np.arange(12), np.arange(13), np.arange(5)])[None] if packed else None
    ref = oracle.hash_ids(ids, mults, orders, rows, canon, 0, position_ids=pos)
    p = pos[0] if packed else np.arange(30)
    mat = np.array([[ids[0, t], ids[0, t - 1] if p[t] >= 1 else -1, ids[0, t - 2] if p[t] >= 2 else -1]
                    for t in range(30)])
    got = oracle.hash_prev(mat, mults, orders, rows, canon, 0)
    assert np.array_equal(ref[:, 0, :], got)


def test_packed_document_hashes_like_standalone():
    # position resets keep n-grams inside a document: a document packed after another hashes
    # exactly as the same document at the start of its own row
    rng = np.random.Generator(np.random.PCG64(9))
    mults = oracle.make_mults(4, 6, 4)
    orders, rows = [2, 2, 3, 3, 4, 4], [1001, 1001, 997, 997, 4099, 4099]
    canon = rng.integers(0, 800, size=800)
    doc_a, doc_b = rng.integers(0, 800, size=17), rng.integers(0, 800, size=9)
    packed = np.concatenate([doc_a, doc_b])[None]
    pos = np.concatenate([np.arange(17), np.arange(9)])[None]
    both = oracle.hash_ids(packed, mults, orders, rows, canon, 7, position_ids=pos)
    alone = oracle.hash_ids(doc_b[None], mults, orders, rows, canon, 7)
    assert np.array_equal(both[:, :, 17:], alone)


def test_pad_id_is_raw_not_canon_mapped():
    # missing predecessors contribute the raw pad id (module.py:189, 218), never canon[pad]
    mults = oracle.make_mults(0, 1, 2)
    canon = np.arange(100)
    canon[7] = 3
    got = oracle.hash_ids(np.array([[42]]), mults, [2], [1 << 20], canon, 7)[0, 0, 0]
    want = ((42 * int(mults[0, 0]) + 7 * int(mults[0, 1])) % P) % (1 << 20)
    assert got == want


def test_negative_pad_and_canon_values_floor_modulo():
    # torch's integer % is floor modulo: negative sums still land in [0, rows)
    mults = oracle.make_mults(1, 2, 3)
    canon = -np.arange(1, 51)  # every canonical id negative
    ids = np.array([[1, 2, 3, 4, 5]])
    got = oracle.hash_ids(ids, mults, [3, 3], [97, 1000], canon, -5)
    want = _bigint_hash(ids, None, canon, mults, [3, 3], [97, 1000], -5)
    assert np.array_equal(got, want)
    assert got.min() >= 0


def test_golden_fixture():
    # regression fixture written by tests/golden/make_golden.py
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "hash_small.npz")
    f = np.load(path)
    got = oracle.hash_ids(f["ids"], f["mults"], list(f["orders"]), list(f["rows"]), f["canon"],
                          int(f["pad_id"]), position_ids=f["pos"])
    assert np.array_equal(got, f["idx"])
    prev = oracle.hash_prev(f["prev_ids"], f["mults"], list(f["orders"]), list(f["rows"]),
                            f["canon"], int(f["pad_id"]))
    assert np.array_equal(prev, f["prev_idx"])


@pytest.mark.parametrize("seed", range(4))
def test_torch_restatement_equals_c_oracle(seed):
    # the CPU baseline's torch-op hash gives the C oracle's row ids bit for bit (big-integer
    # brute force pins the C oracle above)
    rng = np.random.Generator(np.random.PCG64(100 + seed))
    ids, pos, canon, mults, orders, rows = _random_case(
        rng, 2, 41, 700, orders_heads=((2, 3), (3, 2), (4, 1)), with_pos=seed % 2 == 0)
    pad = int(rng.integers(0, 700))
    want = oracle.hash_ids(ids, mults, orders, rows, canon, pad, position_ids=pos)
    got = oracle.hash_ids_torch(ids, mults, orders, rows, canon, pad, position_ids=pos)
    assert np.array_equal(got.numpy(), want)


@pytest.mark.parametrize("seed", range(4))
def test_torch_hash_prev_equals_c_oracle(seed):
    # the decode baseline's torch-op hash_prev gives the C oracle's row ids bit for bit, with
    # missing predecessors (-1), out-of-range ids (clamped) and a negative pad id
    rng = np.random.Generator(np.random.PCG64(200 + seed))
    V = 700
    mults = oracle.make_mults(seed, 6, 4)
    orders, rows = [2, 2, 3, 3, 4, 4], [1009, 97, 257, 2**31 + 11, 4099, 65536]
    canon = rng.integers(-50, V, size=V)
    mat = rng.integers(-1, V + 40, size=(57, 5))
    mat[rng.random((57, 5)) < 0.2] = -1
    pad = int(rng.integers(-9, V))
    want = oracle.hash_prev(mat, mults, orders, rows, canon, pad)
    got = oracle.hash_prev_torch(mat, mults, orders, rows, canon, pad)
    assert np.array_equal(got.numpy(), want)


def test_lookup_torch_equals_lookup():
    # F.embedding + cat (the CPU baselines' lookup) == the numpy fancy-index lookup
    rng = np.random.Generator(np.random.PCG64(3))
    tables = [rng.standard_normal((r, 8)).astype(np.float32) for r in (31, 57, 12)]
    idx = [rng.integers(0, t.shape[0], size=40) for t in tables]
    got = oracle.lookup_torch([torch.from_numpy(t) for t in tables], idx)
    assert np.array_equal(got.numpy(), oracle.lookup(tables, idx))
