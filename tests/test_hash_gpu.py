"""Stages 1-2 on the GPU against the oracle: row ids bit-exact, gathered rows bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, ops, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _engram(orders=(2, 3), heads=2, sizes=None, table_size=257, dim=4, vocab=1000, seed=0,
            pad_id=0, canon=None, dtype=torch.float32, build_tables=True):
    eng = MicroEngram(model_dim=32, table_size=table_size, engram_dim=dim, num_heads=heads,
                      orders=orders, table_sizes=sizes, vocab_size=vocab, seed=seed, pad_id=pad_id,
                      canon=canon, gate="scalar_sqrt", build_tables=build_tables)
    return eng.to(device=DEV, dtype=dtype)


def _oracle_ids(eng, ids, pos=None):
    return oracle.hash_ids(ids.cpu().numpy(), eng.mults.cpu().numpy(), eng._table_orders,
                           eng.table_rows, eng.canon.cpu().numpy(), eng.pad_id,
                           position_ids=None if pos is None else pos.cpu().numpy())


def _stack(idx):
    return torch.stack(idx).cpu().numpy()


@pytest.mark.parametrize("ids_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("pos_kind", [None, "full", "row", "flat"])
def test_hash_ids_small(ids_dtype, pos_kind):
    rng = np.random.Generator(np.random.PCG64(1))
    canon = np.arange(1000)
    canon[rng.choice(1000, 80, replace=False)] = rng.integers(0, 1000, 80)
    eng = _engram(orders=(2, 3, 4), sizes={2: 257, 3: 401, 4: 97}, canon=canon, pad_id=5)
    B, T = 3, 37
    ids = torch.from_numpy(rng.integers(-4, 1004, size=(B, T))).to(ids_dtype)
    pos = None
    if pos_kind is not None:
        p = np.concatenate([np.arange(11), np.arange(20), np.arange(6)])
        if pos_kind == "full":
            pos = torch.from_numpy(np.stack([np.roll(p, b) for b in range(B)]))
        elif pos_kind == "row":
            pos = torch.from_numpy(p[None])
        else:
            pos = torch.from_numpy(p)
    got = _stack(eng.hash_ids(ids.to(DEV), None if pos is None else pos.to(DEV)))
    want = _oracle_ids(eng, ids, None if pos is None else (pos if pos.dim() == 2 else pos[None]))
    assert np.array_equal(got, want)


def test_hash_ids_edge_values():
    # rows above 2^31-1 (identity second modulo), negative canon values and pad id, one row of
    # one token, a table with one row
    canon = -np.arange(1, 101)
    eng = _engram(orders=(2, 3), heads=1, sizes={2: oracle.PRIME + 3, 3: 1}, canon=canon,
                  vocab=100, pad_id=-9, build_tables=False)
    for ids in (torch.tensor([[5]]), torch.randint(-5, 120, (2, 19))):
        got = _stack(eng.hash_ids(ids.to(DEV)))
        assert np.array_equal(got, _oracle_ids(eng, ids))


def test_hash_ids_empty():
    eng = _engram()
    got = eng.hash_ids(torch.zeros((2, 0), dtype=torch.long, device=DEV))
    assert len(got) == 4 and all(g.shape == (2, 0) for g in got)


@pytest.mark.parametrize("ids_dtype", [torch.int32, torch.int64])
def test_hash_prev_small(ids_dtype):
    rng = np.random.Generator(np.random.PCG64(3))
    eng = _engram(orders=(2, 3, 4), heads=3, sizes={2: 257, 3: 401, 4: 97}, pad_id=2)
    ids = rng.integers(-1, 1000, size=(41, 6))  # wider than max_order, like a padded buffer
    ids[::7, 0] = -1
    t = torch.from_numpy(ids).to(ids_dtype)
    want = oracle.hash_prev(ids[:, :4], eng.mults.cpu().numpy(), eng._table_orders, eng.table_rows,
                            eng.canon.cpu().numpy(), 2)
    got = _stack(eng.hash_prev(t.to(DEV)[:, :4]))  # a column slice: rows 6 apart
    assert np.array_equal(got, want)


def test_hash_prev_matches_hash_ids_packed():
    # test_vllm_ids.py:68-83 on the GPU
    rng = np.random.Generator(np.random.PCG64(4))
    eng = _engram(orders=(2, 3))
    ids = torch.from_numpy(rng.integers(5, 1000, size=(1, 30)))
    pos = torch.cat([torch.arange(12), torch.arange(13), torch.arange(5)]).unsqueeze(0)
    ref = eng.hash_ids(ids.to(DEV), pos.to(DEV))
    p = pos[0]
    mat = torch.tensor([[int(ids[0, t]), int(ids[0, t - 1]) if p[t] >= 1 else -1,
                         int(ids[0, t - 2]) if p[t] >= 2 else -1] for t in range(30)])
    got = eng.hash_prev(mat.to(DEV))
    assert all(torch.equal(a[0], b) for a, b in zip(ref, got))


@pytest.mark.parametrize("dtype,dim", [(torch.float32, 4), (torch.bfloat16, 64), (torch.float32, 64),
                                       (torch.bfloat16, 4), (torch.bfloat16, 3)])
def test_lookup_rows_bit_exact(dtype, dim):
    eng = _engram(dim=dim, dtype=dtype, sizes={2: 300, 3: 50})
    ids = torch.randint(0, 1000, (4, 33))
    idx = eng.hash_ids(ids.to(DEV))
    rows = eng.lookup(idx)
    tables = [t.weight.detach().cpu().float().numpy() for t in eng.tables]
    want = oracle.lookup(tables, [i.cpu().numpy() for i in idx])
    got = torch.cat([r.detach().reshape(-1, dim) for r in rows], dim=-1).float().cpu().numpy()
    assert np.array_equal(got, want)
    assert rows[0].shape == (4, 33, dim)


def test_lookup_out_of_range_rows_are_zero():
    # the masked serving lookup (micro_engram_vllm/tp.py:20-39 at TP=1): rows outside a table
    eng = _engram(dim=8, sizes={2: 10, 3: 20})
    idx = [torch.tensor([0, 9, 10, -1, 5], device=DEV)] * 2 + [torch.tensor([19, 20, 3, -7, 0], device=DEV)] * 2
    got = torch.cat(eng.lookup(idx), dim=-1).detach().cpu().numpy()
    tables = [t.weight.detach().cpu().numpy() for t in eng.tables]
    assert np.array_equal(got, oracle.lookup(tables, [i.cpu().numpy() for i in idx]))


def test_hash_gather_equals_hash_then_gather():
    eng = _engram(orders=(2, 3, 4), heads=4, dim=16, dtype=torch.bfloat16, sizes={2: 1000, 3: 3000, 4: 77})
    ids = torch.randint(0, 1000, (2, 50), device=DEV)
    pos = torch.cat([torch.arange(20), torch.arange(30)]).to(DEV)
    mem, idx = ops.hash_gather(ids, pos, eng.canon, eng.mults, eng._table_orders, eng.table_rows,
                               eng.pad_id, [t.weight.detach() for t in eng.tables], True)
    ref_idx = torch.stack(eng.hash_ids(ids, pos))
    assert torch.equal(idx, ref_idx)
    assert torch.equal(mem, torch.cat(eng.lookup(list(ref_idx.unbind(0))), dim=-1).reshape(100, -1))


@pytest.mark.parametrize("n", [1, 700, 1025, 2049, 4089, 4096, 16384, 16393])
def test_gathers_across_tokens_per_workgroup(n):
    # the launches give each workgroup 8 tokens (24 tables), fewer when that would leave under
    # 512 workgroups (n < 4089: 4, 2 or 1 per workgroup), and pace their row loads while they
    # are one round of 2048 workgroups (16384 tokens; 16393 is past it): every size is bit-exact
    # against the oracle, whole and ragged last workgroups included
    eng = _engram(orders=(2, 3, 4), heads=8, dim=64, dtype=torch.bfloat16, sizes={2: 4001, 3: 7919, 4: 6007},
                  canon=torch.randint(0, 1000, (1000,), generator=torch.Generator().manual_seed(n)))
    gen = torch.Generator().manual_seed(n)
    ids = torch.randint(-3, 1010, (1, n), generator=gen)
    pos = torch.arange(n).remainder(517)[None]
    tabs = [t.weight.detach() for t in eng.tables]
    tables_np = [t.float().cpu().numpy() for t in tabs]
    want_idx = _oracle_ids(eng, ids, pos)
    want_mem = oracle.lookup(tables_np, list(want_idx.reshape(len(tabs), -1)))
    mem, idx = ops.hash_gather(ids.to(DEV), pos.to(DEV), eng.canon, eng.mults, eng._table_orders,
                               eng.table_rows, eng.pad_id, tabs, True)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(mem.float().cpu().numpy(), want_mem)
    got = ops.gather(idx.reshape(len(tabs), -1), tabs)
    assert np.array_equal(got.float().cpu().numpy(), want_mem)
    prev = torch.randint(-1, 1010, (n, 4), dtype=torch.int32, generator=gen)
    prev[::5, 0] = -1
    want_prev = oracle.hash_prev(prev.numpy(), eng.mults.cpu().numpy(), eng._table_orders, eng.table_rows,
                                 eng.canon.cpu().numpy(), eng.pad_id)
    pmem, pidx = ops.hash_prev_gather(prev.to(DEV), eng.canon, eng.mults, eng._table_orders, eng.table_rows,
                                      eng.pad_id, tabs, True)
    assert np.array_equal(pidx.cpu().numpy(), want_prev)
    assert np.array_equal(pmem.float().cpu().numpy(), oracle.lookup(tables_np, list(want_prev)))


def test_prev_gather_equals_hash_prev_then_gather():
    eng = _engram(orders=(2, 3, 4), heads=2, dim=64, dtype=torch.bfloat16)
    ids = torch.randint(-1, 1000, (77, 4), dtype=torch.int32, device=DEV)
    mem, idx = ops.hash_prev_gather(ids, eng.canon, eng.mults, eng._table_orders, eng.table_rows,
                                    eng.pad_id, [t.weight.detach() for t in eng.tables], True)
    ref = eng.hash_prev(ids)
    assert torch.equal(idx, torch.stack(ref))
    assert torch.equal(mem, torch.cat(eng.lookup(ref), dim=-1))


def test_identity_canon_path_equals_explicit_map():
    # canon=None builds arange(vocab): the kernels' identity path (no canon read) must give the
    # ids of the explicit map, for every op that hashes, including clamped out-of-vocab ids
    eng = _engram(orders=(2, 3, 4), heads=2, dim=64, dtype=torch.bfloat16, vocab=1000)
    assert torch.equal(eng.canon.cpu(), torch.arange(1000))
    ids = torch.randint(-50, 1100, (3, 61), device=DEV)
    pos = torch.cat([torch.arange(30), torch.arange(31)]).to(DEV)
    prev = torch.randint(-1, 1100, (91, 4), dtype=torch.int32, device=DEV)
    tabs = [t.weight.detach() for t in eng.tables]
    args = (eng.canon, eng.mults, eng._table_orders, eng.table_rows, eng.pad_id)
    for ident in (True, False):
        a = ops.hash_ids(ids, pos, *args, ident)
        b = ops.hash_prev(prev, *args, ident)
        c = ops.hash_gather(ids, pos, *args, tabs, True, ident)
        d = ops.hash_prev_gather(prev, *args, tabs, True, ident)
        if ident:
            first = (a, b, c, d)
    assert torch.equal(first[0], a) and torch.equal(first[1], b)
    assert all(torch.equal(x, y) for x, y in zip(first[2] + first[3], c + d))
    assert np.array_equal(first[0].cpu().numpy(), _oracle_ids(eng, ids, pos[None]))
    # the module reads the map on every call: a write through .data (no version bump) is hashed
    eng.canon.data[ids[0, 5].clamp(0, 999)] = 17
    assert np.array_equal(_stack(eng.hash_ids(ids, pos)), _oracle_ids(eng, ids, pos[None]))
    want = oracle.hash_prev(prev.cpu().numpy(), eng.mults.cpu().numpy(), eng._table_orders, eng.table_rows,
                            eng.canon.cpu().numpy(), eng.pad_id)
    assert np.array_equal(_stack(eng.hash_prev(prev)), want)


# ---------------------------------------------------------------- full-size workloads
@pytest.fixture(scope="module")
def gemma():
    eng = synthetic.build_engram("gemma", DEV, seed=0)
    yield eng
    del eng
    torch.cuda.empty_cache()


def test_gemma_prefill_ids_bit_exact(gemma):
    ids, pos, _ = synthetic.prefill_inputs(seed=0)
    with torch.no_grad():
        mem, idx = ops.hash_gather(ids.to(DEV), pos.to(DEV), gemma.canon, gemma.mults,
                                   gemma._table_orders, gemma.table_rows, gemma.pad_id,
                                   [t.weight for t in gemma.tables], True)
    want = _oracle_ids(gemma, ids, pos)
    assert np.array_equal(idx.cpu().numpy(), want)
    # rows: every table's rows of a token sample, fetched by index on the device
    sample = torch.from_numpy(np.random.Generator(np.random.PCG64(0)).choice(8192, 512, replace=False))
    got = mem[sample.to(DEV)].cpu()
    parts = [t.weight[idx[k, 0][sample.to(DEV)]].cpu() for k, t in enumerate(gemma.tables)]
    assert torch.equal(got, torch.cat(parts, dim=-1))
    # the gathered buffer as a whole: its checksum equals the sum of the gathered rows' sums
    table_sums = [t.weight.float().sum(dim=1) for t in gemma.tables]
    want_sum = sum(table_sums[k][idx[k, 0]].double().sum() for k in range(len(gemma.tables)))
    assert torch.allclose(mem.float().sum(dtype=torch.float64), want_sum, rtol=1e-9, atol=1e-6)


def test_serving_decode_ids_bit_exact(gemma):
    ids, _ = synthetic.decode_inputs(seed=1)
    got = _stack(gemma.hash_prev(ids.to(DEV)))
    want = oracle.hash_prev(ids.numpy(), gemma.mults.cpu().numpy(), gemma._table_orders,
                            gemma.table_rows, gemma.canon.cpu().numpy(), gemma.pad_id)
    assert np.array_equal(got, want)


def test_two_engram_canon_ids_bit_exact():
    rng = np.random.Generator(np.random.PCG64(29))
    canon = synthetic.canon_map(rng, synthetic.GEMMA_VOCAB)
    assert np.array_equal(canon[canon], canon)
    ids, pos, _ = synthetic.prefill_inputs(seed=3, batch=8, dim=8)
    for seed in (0, synthetic.LAYER29_SEED):
        eng = MicroEngram(model_dim=8, engram_dim=64, num_heads=8, orders=synthetic.GEMMA_ORDERS,
                          table_size=synthetic.GEMMA_SIZES[2], table_sizes=synthetic.GEMMA_SIZES,
                          vocab_size=synthetic.GEMMA_VOCAB, seed=seed, canon=canon,
                          build_tables=False, gate="scalar_sqrt").to(DEV)
        got = _stack(eng.hash_ids(ids.to(DEV), pos.to(DEV)))
        assert np.array_equal(got, _oracle_ids(eng, ids, pos))
