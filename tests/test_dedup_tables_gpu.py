"""The row lookup's key plan from per-table row ids (me_dedup_tables) against the oracle's dedup
of the token-major keys offset_k + idx[k][t] (torch.unique(return_inverse) + index_add_ order,
rows.py:81, 117-118): unique keys, inverse, local rows, the tables' bounds (searchsorted of
rows.py:123-129) and, through the plan, the fp32 gradient sums -- all bit-exact. Cases cover
both launches' paths: parts sorted in LDS, a part larger than LDS (one row taking every lookup
of its table), tables of one row, a row-id view with a stride, more tokens than the table path
takes (the generic key half), and tables too long for 32-bit rows."""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import ops, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(idx2d, table_rows, dim=4, seed=0):
    nt, n = idx2d.shape
    offs = np.concatenate([[0], np.cumsum(np.array(table_rows, dtype=np.int64))])
    keys = (idx2d.cpu().numpy() + offs[:-1, None]).T.reshape(-1)  # token-major
    g = torch.Generator().manual_seed(seed)
    grads = torch.randn(n * nt, dim, generator=g) * torch.logspace(-3, 1, n * nt).unsqueeze(1)
    u, i, acc = oracle.dedup(keys, grads.numpy())
    for inverse in (True, False):  # the row lookup's key plan leaves the inverse unwritten
        uniq, local, inv, count, plan, info = ops.dedup_tables(idx2d.to(DEV), table_rows, inverse=inverse)
        gsum = ops.dedup_sums(plan, count, grads.to(DEV))
        torch.cuda.synchronize()
        cnt = int(count.item())
        assert cnt == u.size
        assert np.array_equal(uniq[:cnt].cpu().numpy(), u)
        if inverse:
            assert np.array_equal(inv.cpu().numpy(), i)
        tbl = np.searchsorted(offs[:-1], u, side="right") - 1
        assert np.array_equal(local[:cnt].cpu().numpy(), u - offs[tbl])
        assert info.cpu().tolist() == [cnt] + np.searchsorted(u, offs).tolist()
        assert np.array_equal(gsum[:cnt].cpu().numpy().view(np.int32), acc.view(np.int32))


@pytest.mark.parametrize("n,rows", [(1, [1]), (37, [5, 100, 7]), (512, [1, 3, 1 << 20]),
                                    (1000, [257, 4099, 97, 65536]), (8192, [50_000, 1 << 22]),
                                    (16384, [1 << 21, 3000])])
def test_dedup_tables_random(n, rows):
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.randint(0, r, (n,), generator=g) for r in rows])
    if n > 100:
        idx[:, ::5] = idx[:, :1]  # one row repeated across every round and part
    _check(idx, rows, seed=n)


def test_dedup_tables_gemma_batch():
    # the 8192-token Gemma prefill batch's 24 tables (196,608 lookups, Zipf-hot order-2 rows)
    eng = synthetic.build_engram("gemma", DEV, seed=0)
    ids, pos, _ = synthetic.prefill_inputs(seed=0, device=DEV)
    idx = torch.stack(eng.hash_ids(ids, pos)).reshape(len(eng.tables), -1)
    _check(idx.cpu(), eng.table_rows, dim=64)
    del eng
    torch.cuda.empty_cache()


def test_dedup_tables_part_larger_than_lds():
    # every lookup of table 0 on one row (8192 in one part: the global-memory sort), table 1
    # split between two rows, table 2 random
    n = 8192
    g = torch.Generator().manual_seed(3)
    idx = torch.stack([torch.full((n,), 123_456, dtype=torch.long),
                       torch.randint(0, 2, (n,), generator=g) * 999_999,
                       torch.randint(0, 1 << 22, (n,), generator=g)])
    _check(idx, [1 << 22, 1 << 20, 1 << 22])


def test_dedup_tables_strided_view():
    n = 3000
    g = torch.Generator().manual_seed(5)
    big = torch.randint(0, 7000, (4, n + 77), generator=g)
    _check(big[:, 10:10 + n], [7000, 7001, 9000, 7000])


@pytest.mark.parametrize("n,rows", [(20_000, [4099, 1 << 22]), (300, [1 << 33, 5])])
def test_dedup_tables_generic_path(n, rows):
    # more tokens than the table path takes, and a table whose rows exceed 32 bits: the keys,
    # the generic key half and the bounds
    g = torch.Generator().manual_seed(n)
    idx = torch.stack([torch.randint(0, min(r, 1 << 40), (n,), generator=g) for r in rows])
    idx[:, ::7] = idx[:, 3:4]
    _check(idx, rows)


def test_dedup_tables_empty():
    uniq, local, inv, count, plan, info = ops.dedup_tables(torch.empty(3, 0, dtype=torch.long, device=DEV),
                                                           [5, 6, 7])
    assert info.cpu().tolist() == [0, 0, 0, 0, 0]


def test_dedup_tables_hot_buckets():
    # rows repeated 49 to 600 times among random ones: buckets far larger than their share of
    # the part, ranked in LDS (the part still fits)
    n, rows = 8192, 1 << 22
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, rows, (2, n), generator=g)
    perm = torch.randperm(n, generator=g)
    at = 0
    for reps, row in ((49, 7), (100, 300_001), (300, 900_000), (512, 1_500_000), (513, 2_900_000), (600, 4_000_000)):
        idx[0, perm[at:at + reps]] = row
        at += reps
    idx[1, perm[:300]] = 123  # a second table with one hot row
    _check(idx, [rows, rows])


def test_dedup_tables_calls_in_a_row():
    # plans of more and fewer parts back to back on one stream, each against the oracle
    g = torch.Generator().manual_seed(21)
    cases = [(4096, [1 << 22] * 6), (512, [1 << 20, 77]), (4096, [1 << 22] * 6), (2000, [5000, 1 << 21, 3])]
    for n, rows in cases:
        idx = torch.stack([torch.randint(0, r, (n,), generator=g) for r in rows])
        _check(idx, rows, dim=2)
