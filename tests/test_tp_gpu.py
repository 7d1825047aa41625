"""The serving plugin's wiring on the GPU (micro_engram_vllm/model.py:165-201, tp.py): an engram
built without tables, given empty row shards, filled by load_rows, with tp_lookup installed as
row_lookup_fn, then hash_prev + inject as EngramGemma4DecoderLayer.forward calls them
(model.py:45-50). torch's embedding is made to raise, so the rows can only come from the HIP
gather; the result is compared with the oracle."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from micro_engram_fork_amd import MicroEngram, engram_from_spec, synthetic
from micro_engram_fork_amd.tp import load_rows, tp_lookup

pytestmark = pytest.mark.gpu
DEV = "cuda"
D, V = 256, 3000
SPEC = {"layer": 0, "table_size": 1009, "table_sizes": {2: 1009, 3: 701, 4: 503}, "engram_dim": 16,
        "num_heads": 4, "orders": [2, 3, 4], "gate": "scalar_sqrt", "seed": 5, "pad_id": 0}


def _trained_source(dtype):
    src = engram_from_spec(SPEC, D, V)
    synthetic.fill_dense(src, seed=9, std=0.1)
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        for t in src.tables:
            t.weight.copy_(torch.randn(t.weight.shape, generator=g) * 0.1)
    return src.to(dtype=dtype)


def _served(dtype):
    eng = engram_from_spec(SPEC, D, V, build_tables=False)
    eng.to(device=DEV, dtype=dtype)
    eng.shard_rows(0, 1, device=DEV, dtype=dtype, requires_grad=False, empty=True)
    eng.row_lookup_fn = tp_lookup(lambda x: x)
    return eng


def _no_torch_embedding(monkeypatch):
    def refuse(*args, **kwargs):
        raise AssertionError("torch embedding called: the lookup must run in the HIP gather")

    monkeypatch.setattr(F, "embedding", refuse)
    monkeypatch.setattr(torch.nn.functional, "embedding", refuse)


def _ids_matrix(n, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, V, (n, 4), generator=g, dtype=torch.int32)
    hist = torch.randint(0, 4, (n,), generator=g)
    for c in range(1, 4):
        ids[hist < c, c] = -1  # shorter histories: missing predecessors
    return ids


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_plugin_wiring_runs_on_hip_gather(monkeypatch, dtype):
    src = _trained_source(dtype)
    eng = _served(dtype)
    loaded = load_rows(eng, src.state_dict(), "test engram")
    assert loaded == set(range(len(eng.row_shards)))
    _no_torch_embedding(monkeypatch)
    ids = _ids_matrix(300, 1)
    g = torch.Generator().manual_seed(2)
    hidden = torch.randn(300, D, generator=g).to(dtype)
    keep = torch.rand(300, generator=g) > 0.1
    with torch.inference_mode():
        idx = eng.hash_prev(ids.to(DEV))
        parts = eng.lookup(idx)
        out = eng.inject(hidden.to(DEV), idx, keep.to(DEV))
    torch.cuda.synchronize()
    monkeypatch.undo()  # the oracle below uses torch's embedding itself
    want_idx = oracle.hash_prev(ids.numpy(), src.mults.numpy(), src._table_orders, src.table_rows,
                                src.canon.numpy(), 0)
    assert np.array_equal(torch.stack(idx).cpu().numpy(), want_idx)
    tables = [t.weight.detach() for t in src.tables]
    mem = oracle.lookup_torch(tables, list(want_idx))
    for k, part in enumerate(parts):  # tp_lookup's per-table rows, bit for bit
        assert part.shape == (300, 16)
        assert torch.equal(part.cpu(), mem[:, k * 16:(k + 1) * 16])
    ref = oracle.inject(hidden, mem, src.key.weight.detach(), src.value.weight.detach(),
                        "scalar_sqrt", src.q_scale.detach(), src.k_scale.detach(), keep=keep)
    assert torch.equal(out.cpu()[~keep], hidden[~keep])
    from test_gate_gpu import assert_close_out  # the gate tests' stated per-dtype tolerance

    assert_close_out(out, ref, hidden, dtype)


def test_tp_lookup_zero_rows_outside_the_table():
    # tp.py:28-33: ids outside [start, start + n) give zero rows
    eng = _served(torch.float32)
    src = _trained_source(torch.float32)
    load_rows(eng, src.state_dict(), "test engram")
    idx = [torch.tensor([0, 5, -1, eng.table_rows[k], 10**9], device=DEV) for k in range(len(eng.row_shards))]
    with torch.inference_mode():
        parts = eng.row_lookup_fn(eng, idx)
    for k, part in enumerate(parts):
        w = src.tables[k].weight.detach()
        assert torch.equal(part[0].cpu(), w[0]) and torch.equal(part[1].cpu(), w[5])
        assert not part[2:].any()


def test_tp_lookup_refuses_several_ranks():
    eng = engram_from_spec(SPEC, D, V, build_tables=False).to(DEV)
    eng.shard_rows(1, 2, device=DEV, requires_grad=False, empty=True)
    eng.row_lookup_fn = tp_lookup(lambda x: x)
    idx = eng.hash_prev(_ids_matrix(8, 0).to(DEV))
    with pytest.raises(NotImplementedError, match="tensor-parallel"):
        eng.lookup(idx)


def test_load_rows_checks():
    eng = _served(torch.float32)
    src = _trained_source(torch.float32)
    sd = src.state_dict()
    with pytest.raises(ValueError, match="no rows given"):
        load_rows(eng, {k: v for k, v in sd.items() if k != "tables.3.weight"}, "partial")
    part = {k: v for k, v in sd.items() if k.startswith("tables.")}
    assert load_rows(eng, part, "tables only", complete=False) == set(range(12))
    bad = dict(sd)
    bad["tables.0.weight"] = bad["tables.0.weight"][:-1]
    with pytest.raises(ValueError, match="table 0"):
        load_rows(eng, bad, "short table")
    wrong_seed = dict(sd)
    wrong_seed["mults"] = sd["mults"] + 2
    with pytest.raises(ValueError, match="multipliers"):
        load_rows(eng, wrong_seed, "wrong seed")
