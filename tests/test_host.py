"""Host logic on the CPU: the C-ABI library loads and exports its header's entry points, and the
MicroEngram surface keeps the reference's names, buffers and state-dict conventions."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, _lib, check_loaded, resolve_order_sizes
from micro_engram_fork_amd.module import default_seed

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(me_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_lib.lib_path())
    declared = _header_symbols()
    assert declared, "no declarations found in include/"
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python binding covers every declared entry point, with a signature
    assert declared <= set(_lib.exported_symbols())


def test_library_version_and_error_path():
    lib = _lib.load()
    assert lib.me_version() >= 1
    # a bad argument is refused before any GPU call, with a message
    with pytest.raises(_lib.EngramLibError, match="n_tables"):
        _lib.call("me_hash_prev", None, _lib.ME_I64, 0, 4, 4, None, 10, None, 4, 0, None, None, 0,
                  None, None)


def test_resolve_order_sizes():
    assert resolve_order_sizes(100, (3, 2)) == {2: 100, 3: 100}
    assert resolve_order_sizes(100, (2, 3), {"4": 50, 3: 0}) == {2: 100, 4: 50}
    with pytest.raises(ValueError):
        resolve_order_sizes(0, (2, 3))


def test_module_surface_and_layout():
    eng = MicroEngram(model_dim=16, table_size=257, engram_dim=4, num_heads=2, orders=(3, 2),
                      vocab_size=1000, gate="scalar_sqrt", table_sizes={4: 97})
    assert eng.orders == (2, 3, 4)
    assert eng._table_orders == [2, 2, 3, 3, 4, 4]
    assert eng.table_rows == [257, 257, 257, 257, 97, 97]
    assert eng.table_size is None
    sd = eng.state_dict()
    assert {"key.weight", "value.weight", "q_scale", "k_scale", "mults", "canon",
            "tables.0.weight", "tables.5.weight"} <= set(sd)
    assert torch.equal(eng.value.weight, torch.zeros(16, 24))
    assert torch.equal(eng.canon, torch.arange(1000))
    # multipliers equal the oracle's restatement of torch's generator
    assert np.array_equal(eng.mults.numpy(), oracle.make_mults(0, 6, 4))


def test_scales_stored_as_delta():
    # test_gate.py:132-143, 162-170
    eng = MicroEngram(model_dim=8, table_size=17, engram_dim=4, num_heads=1, vocab_size=50,
                      gate="scalar_sqrt")
    assert torch.equal(eng.state_dict()["q_scale"], torch.ones(8))
    old = eng.state_dict()
    old["q_scale"] = 1 + 0.3 * torch.rand(8)
    new = MicroEngram(model_dim=8, table_size=17, engram_dim=4, num_heads=1, vocab_size=50,
                      gate="scalar_sqrt")
    new.load_state_dict(old)
    assert torch.allclose(new.q_scale, old["q_scale"] - 1)
    assert torch.allclose(new.state_dict()["q_scale"], old["q_scale"])
    rt = new.to(torch.bfloat16)
    with torch.no_grad():
        rt.q_scale.copy_(torch.linspace(-0.01, 0.01, 8))
    back = MicroEngram(model_dim=8, table_size=17, engram_dim=4, num_heads=1, vocab_size=50,
                       gate="scalar_sqrt").to(torch.bfloat16)
    back.load_state_dict(rt.state_dict())
    assert torch.equal(back.q_scale, rt.q_scale)
    qs, _ = rt.norm_scales()
    assert qs.dtype == torch.float32


def test_check_loaded_refuses_wrong_seed():
    a = MicroEngram(model_dim=8, table_size=17, engram_dim=4, num_heads=1, vocab_size=50, seed=1)
    b = MicroEngram(model_dim=8, table_size=17, engram_dim=4, num_heads=1, vocab_size=50, seed=2)
    with pytest.raises(ValueError, match="seed is wrong"):
        check_loaded(b, a.state_dict(), "test")
    check_loaded(a, {k: v for k, v in a.state_dict().items() if k != "mults"}, "test")


def test_seed_rule():
    assert default_seed(0) == 0 and default_seed(29) == 290_203


def test_cpu_tensors_raise():
    eng = MicroEngram(model_dim=32, table_size=257, engram_dim=4, num_heads=2, vocab_size=1000)
    with pytest.raises(RuntimeError, match="only on the GPU"):
        eng.hash_ids(torch.zeros((1, 4), dtype=torch.long))
    with torch.no_grad(), pytest.raises(RuntimeError, match="only on the GPU"):
        eng(torch.zeros(1, 4, 32), torch.zeros((1, 4), dtype=torch.long))


def test_bad_gate_and_canon_rejected():
    with pytest.raises(ValueError):
        MicroEngram(model_dim=8, gate="bogus")
    with pytest.raises(ValueError):
        MicroEngram(model_dim=8, table_size=17, vocab_size=50, canon=torch.arange(49))


def test_module_always_passes_the_canon_map():
    # the module's hashing reads the canon buffer on every call (no identity shortcut), so a map
    # written in place, through .data (no version bump) or by load_state_dict is what it hashes
    eng = MicroEngram(64, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3), vocab_size=50)
    canon, _mults, ident = eng._hash_consts(eng.canon.device)
    assert ident is False and canon is eng.canon
    eng.canon.data[3] = 7
    canon, _mults, ident = eng._hash_consts(eng.canon.device)
    assert ident is False and int(canon[3]) == 7


def test_gate_stats_fold_in_order_of_records():
    # the recorded gates are reduced lazily (every 32 records and when read): the sums must be
    # those of every record since the last read, over more records than one fold holds
    eng = MicroEngram(model_dim=16, table_size=31, engram_dim=4, num_heads=1, orders=(2,), vocab_size=50)
    gen = torch.Generator().manual_seed(5)
    alphas = [torch.rand(17 + k, generator=gen) for k in range(75)]
    alphas[3][0] = 0.995
    for a in alphas:
        eng._record_gate(a)
    mean, sat = eng.pop_gate_stats()
    allv = torch.cat(alphas).double()
    assert mean == pytest.approx(float(allv.mean()), rel=1e-6)
    assert sat == pytest.approx(float((allv > 0.99).double().mean()), rel=1e-6)
    assert eng.pop_gate_stats() is None
    eng._record_gate(torch.tensor([1.0, 0.0]))
    assert eng.pop_gate_stats() == (0.5, 0.5)


def test_canon_in_state_dict_like_reference():
    # the reference's test_canon.py:58-66: the map is in the state dict, an old checkpoint
    # without it still loads (only canon missing), and the map round-trips into what the
    # module hashes with
    make = lambda canon=None: MicroEngram(model_dim=16, table_size=257, engram_dim=4, num_heads=2,
                                          vocab_size=1000, canon=canon)
    canon = torch.arange(1000)
    canon[[5, 17, 600]] = 4
    eng = make(canon)
    assert "canon" in eng.state_dict()
    old = {k: v for k, v in make().state_dict().items() if k != "canon"}
    res = make().load_state_dict(old, strict=False)
    assert list(res.missing_keys) == ["canon"] and not res.unexpected_keys
    e2 = make()
    e2.load_state_dict(eng.state_dict())
    assert torch.equal(e2.canon, canon)
    assert torch.equal(e2._hash_consts(e2.canon.device)[0], canon)


def test_ops_route_fake_tensors_to_the_registered_ops():
    # eager calls run the implementations directly; fake tensors (shape propagation, as under
    # torch.compile) must reach the registered ops and their fake functions instead
    from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode
    from micro_engram_fork_amd import ops

    assert hasattr(ops.gather, "op") and hasattr(ops.gate_residual_rows, "op")
    with FakeTensorMode():
        ids = torch.empty(32, 4, dtype=torch.int32, device="cuda")
        canon = torch.empty(500, dtype=torch.int64, device="cuda")
        mults = torch.empty(4, 3, dtype=torch.int64, device="cuda")
        idx = ops.hash_prev(ids, canon, mults, [2, 2, 3, 3], [97, 97, 89, 89], 0, True)
        assert isinstance(idx, FakeTensor) and tuple(idx.shape) == (4, 32)
        tables = [torch.empty(97, 8, dtype=torch.bfloat16, device="cuda") for _ in range(4)]
        mem = ops.gather(idx, tables)
        assert isinstance(mem, FakeTensor) and tuple(mem.shape) == (32, 32)
        hidden = torch.empty(32, 64, dtype=torch.bfloat16, device="cuda")
        wk = torch.empty(64, 32, dtype=torch.bfloat16, device="cuda")
        kv = ops.kv_proj(mem, wk, wk)
        assert tuple(kv.shape) == (32, 128)
        outs = ops.gate_residual_rows(hidden, mem, wk, wk, None, None, 0, None, True)
        assert tuple(outs[0].shape) == (32, 64) and tuple(outs[1].shape) == (32,)
        outs = ops.gate_residual(hidden, mem, wk, wk, None, None, 0, None, True)
        assert isinstance(outs[0], FakeTensor) and tuple(outs[0].shape) == (32, 64)
