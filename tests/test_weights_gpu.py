"""Trained engrams through the on-disk formats on the GPU: an engram loaded from each format
gives the same forward, bit for bit, as the one that was saved (same HIP kernels on the same
tensors), and matches the oracle; a row-table checkpoint resumes training exactly (the step
after loading equals the step the saving run takes next)."""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, ops, rows as me_rows
from micro_engram_fork_amd import weights as W

pytestmark = pytest.mark.gpu
DEV = "cuda"
D, H, E, V = 256, 4, 16, 5000


def _trained(dtype, seed=11, canon=None):
    g = torch.Generator().manual_seed(seed)
    eng = MicroEngram(model_dim=D, table_size=1009, engram_dim=E, num_heads=H, orders=(2, 3, 4),
                      vocab_size=V, gate="scalar_sqrt", seed=seed, canon=canon, table_sizes={4: 503})
    with torch.no_grad():
        for t in eng.tables:
            t.weight.copy_(torch.randn(t.weight.shape, generator=g) * 0.1)
        eng.key.weight.copy_(torch.randn(eng.key.weight.shape, generator=g) * 0.05)
        eng.value.weight.copy_(torch.randn(eng.value.weight.shape, generator=g) * 0.05)
        # deltas on a 2^-10 grid: 1 + delta is exact in fp32, so the file's scale gives the
        # module's delta back bit for bit and the forwards can be compared exactly
        eng.q_scale.copy_(torch.round(torch.randn(D, generator=g) * 0.05 * 1024) / 1024)
        eng.k_scale.copy_(torch.round(torch.randn(D, generator=g) * 0.05 * 1024) / 1024)
    return eng.to(dtype=dtype)


def _inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, V, (2, 150), generator=g)
    pos = torch.cat([torch.arange(60), torch.arange(90)]).unsqueeze(0).expand(2, -1)
    hidden = torch.randn(2, 150, D, generator=g)
    return ids, pos, hidden


@pytest.mark.parametrize("fmt,name", [("pt", "micro_engram.pt"), ("safetensors", "e.safetensors"),
                                      ("safetensors_dir", "assembled"), ("dcp", "pytorch_model_fsdp_0")])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_loaded_engram_forward_bit_exact(tmp_path, fmt, name, dtype):
    canon = np.arange(V)
    canon[np.arange(100, 400, 3)] = 7
    eng = _trained(dtype, canon=canon)
    layer = 29
    path = W.save_engram_weights(eng, str(tmp_path / name), layer=layer, fmt=fmt)
    spec = {"layer": layer, "table_size": 1009, "table_sizes": {2: 1009, 3: 1009, 4: 503}, "engram_dim": E,
            "num_heads": H, "orders": [2, 3, 4], "gate": "scalar_sqrt", "seed": 11, "pad_id": 0,
            "weights": name}
    (tmp_path / W.CONFIG_NAME).write_text(__import__("json").dumps({"engrams": [spec]}))
    got = W.load_engram(str(tmp_path), layer, D, V, device=DEV, dtype=dtype)
    assert torch.equal(got.canon.cpu(), eng.canon.cpu())  # the saved map came back
    ids, pos, hidden = _inputs()
    eng = eng.to(DEV)
    with torch.inference_mode():
        want = eng(hidden.to(DEV, dtype), ids.to(DEV), pos.to(DEV))
        out = got(hidden.to(DEV, dtype), ids.to(DEV), pos.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"{fmt}: loaded engram's forward differs"
    if dtype == torch.float32:
        # and the loaded engram is the oracle's engram (module.py:183-265 restated)
        idx = oracle.hash_ids(ids.numpy(), got.mults.cpu().numpy(), got._table_orders, got.table_rows,
                              got.canon.cpu().numpy(), 0, position_ids=pos.numpy())
        tables = [t.weight.detach().cpu().numpy() for t in got.tables]
        mem = torch.from_numpy(oracle.lookup(tables, list(idx.reshape(len(tables), -1))))
        ref = oracle.inject(hidden.reshape(-1, D), mem, got.key.weight.detach().cpu(),
                            got.value.weight.detach().cpu(), "scalar_sqrt", got.q_scale.detach().cpu(),
                            got.k_scale.detach().cpu()).reshape(out.shape)
        rms = hidden.pow(2).mean(-1, keepdim=True).sqrt()
        assert bool(((out.cpu() - ref).abs() <= 1e-5 * rms).all())


def _step_grads(eng, seed):
    """One forward/backward of the row-sharded engram: sparse row gradients on every shard."""
    ids, pos, hidden = _inputs(seed)
    out = eng(hidden.to(DEV, torch.bfloat16), ids.to(DEV), pos.to(DEV))
    out.float().pow(2).sum().backward()


def _row_engram():
    eng = _trained(torch.bfloat16, seed=5)
    eng.shard_rows(0, 1, device=DEV)
    eng.to(DEV)
    return eng


def test_row_tables_resume_is_exact(tmp_path):
    # run A: two steps, save, a third step. Run B: load A's checkpoint after two steps, take
    # the third step with the same gradients: tables and optimizer state equal A's.
    a = _row_engram()
    rt_a = me_rows.RowTables([("model.layers.2.micro_engram.", a)], lr=5e-3, lazy=True, rowwise=True,
                             sparse_grads=True, seed=123)
    for s in range(2):
        _step_grads(a, s)
        rt_a.step(5e-3)
    folder, ofolder = str(tmp_path / me_rows.ROWS_DIR), str(tmp_path / me_rows.ROWS_OPTIM_DIR)
    rt_a.save(folder, ofolder)
    b = _row_engram()
    with torch.no_grad():
        for p in b.row_shards:
            p.zero_()
    rt_b = me_rows.RowTables([("model.layers.2.micro_engram.", b)], lr=5e-3, lazy=True, rowwise=True,
                             sparse_grads=True, seed=123)
    n, ok = rt_b.load(folder, ofolder)
    assert n == len(a.row_shards) and ok
    for eng, rt in ((a, rt_a), (b, rt_b)):
        _step_grads(eng, 2)
        rt.step(5e-3)
    torch.cuda.synchronize()
    for pa, pb in zip(a.row_shards, b.row_shards):
        assert torch.equal(pa, pb)
        sa, sb = rt_a.optimizer.state[pa], rt_b.optimizer.state[pb]
        assert torch.equal(sa["exp_avg"], sb["exp_avg"]) and torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"])
        assert float(sa["step"]) == float(sb["step"]) == 3.0
