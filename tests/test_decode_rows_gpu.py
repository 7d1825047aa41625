"""hash_prev without gradients reads the rows in the same launch (me_hash_prev_gather) and the
id list it returns carries them; inject / lookup then read no rows again. The result must be
what the reference's hash_prev + inject give (micro_engram/module.py:207-261): the same ids bit
for bit, the same output as an inject on the same ids without the carried rows, and fresh rows
whenever the tables, the ids or the carried rows were written in between."""
import pytest
import torch

from micro_engram_fork_amd import MicroEngram, ops, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _engram(shard=False):
    torch.manual_seed(0)
    eng = MicroEngram(model_dim=64, table_size=211, engram_dim=8, num_heads=2, orders=(2, 3, 4),
                      vocab_size=1000, gate="scalar_sqrt", seed=5)
    synthetic.fill_dense(eng, seed=5, std=0.2)
    eng = eng.to(DEV).to(torch.bfloat16).eval()
    if shard:
        eng.shard_rows(0, 1, device=DEV, dtype=torch.bfloat16)
    return eng


def _inputs(seed=1, n=77):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(-1, 1000, (n, 4), generator=g)
    ids[:, 0] = ids[:, 0].clamp(min=0)
    h = torch.randn(n, 64, generator=g).bfloat16()
    return ids.to(DEV), h.to(DEV)


def _plain(idx):
    return [t.clone() for t in idx]  # the same ids, no rows with them


@pytest.mark.parametrize("shard", [False, True])
def test_hash_prev_rows_travel_with_the_ids(shard):
    eng = _engram(shard)
    ids, h = _inputs()
    canon, mults, ident = eng._hash_consts(ids.device)
    with torch.inference_mode():
        idx = eng.hash_prev(ids)
        assert idx.rows is not None
        want_ids = ops.hash_prev(ids, canon, mults, eng._table_orders, eng.table_rows, int(eng.pad_id), ident)
        assert torch.equal(torch.stack(list(idx)), want_ids)
        got = eng.inject(h, idx)
        want = eng.inject(h, _plain(idx))
        assert torch.equal(got, want) and not torch.equal(got, h)
        rows = eng.lookup(idx)
        assert all(torch.equal(a, b) for a, b in zip(rows, eng.lookup(_plain(idx))))


def test_carried_rows_are_dropped_after_writes():
    eng = _engram()
    ids, h = _inputs(2)
    with torch.inference_mode():
        idx = eng.hash_prev(ids)
        eng.lookup(idx)[1].mul_(0)  # the carried rows written through a view
        assert torch.equal(eng.inject(h, idx), eng.inject(h, _plain(idx)))
        idx = eng.hash_prev(ids)
    with torch.no_grad():
        for t in eng.tables:
            t.weight.add_(0.5)  # the tables written after the ids were hashed
    with torch.inference_mode():
        assert torch.equal(eng.inject(h, idx), eng.inject(h, _plain(idx)))
    with torch.no_grad():  # ids made outside inference mode keep a version counter
        idx = eng.hash_prev(ids)
        assert idx.rows is not None
        idx[0].fill_(3)  # the ids written: the rows of the new ids are read
        assert torch.equal(eng.inject(h, idx), eng.inject(h, _plain(idx)))
        idx = eng.hash_prev(ids)
        idx[1] = idx[1].clone()  # an element replaced: likewise
        assert torch.equal(eng.inject(h, idx), eng.inject(h, _plain(idx)))


def test_hash_prev_with_gradients_reads_no_rows():
    eng = _engram()
    ids, _ = _inputs(3)
    assert eng.hash_prev(ids).rows is None
