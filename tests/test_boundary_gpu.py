"""The drop-in boundary on the GPU.

* The vLLM decoder layer's calls (hash_prev + inject, micro_engram_vllm/model.py:45-50) compile
  as ONE graph (torch.compile(fullgraph=True)) and the compiled step equals the eager one bit
  for bit, for the plain engram and for the plugin's tp_lookup wiring (tp.py:17-39), on both
  gate paths.
* `lookup` is the seam inject and forward read the rows through (module.py:146-154, 233): the
  reference's own test replaces it on the instance to drop the 4-gram lookups
  (test_zero_order.py:84-88); the output must equal an engram whose 4-gram tables are zero,
  and the oracle's inject of the rows with the 4-gram part zeroed.
* `lookup` on plain tables carries the tables' gradients, as nn.Embedding does (module.py:154):
  the gradient of every table equals CPU index_add_ of the rows' gradients, bit for bit.
"""
import copy

import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, synthetic
from micro_engram_fork_amd.tp import tp_lookup

from test_gate_gpu import assert_close_out

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(params=["fused", "rows"])
def gate_path(request, monkeypatch):
    limit = 0 if request.param == "fused" else 1 << 30
    monkeypatch.setattr(MicroEngram, "few_tokens_max", limit)
    monkeypatch.setattr(MicroEngram, "few_tokens_max_fp32", limit)
    monkeypatch.setattr(MicroEngram, "few_tokens_kv_bytes", 0 if limit == 0 else 1 << 62)
    return request.param


def _make(dtype, d=64, dim=8, heads=2, orders=(2, 3, 4), seed=0):
    eng = MicroEngram(model_dim=d, table_size=257, engram_dim=dim, num_heads=heads, orders=orders,
                      table_sizes={2: 257, 3: 241, 4: 229}, vocab_size=1000, gate="scalar_sqrt",
                      seed=seed)
    synthetic.fill_dense(eng, seed=seed, std=0.2)
    g = torch.Generator().manual_seed(seed + 5)
    with torch.no_grad():
        for t in eng.tables:
            t.weight.copy_(torch.randn(t.weight.shape, generator=g) * 0.3)
    return eng.to(device=DEV, dtype=dtype).eval()


@pytest.mark.parametrize("wiring", ["plain", "tp_lookup"])
def test_decode_layer_compiles_as_one_graph_like_eager(gate_path, wiring):
    eng = _make(torch.bfloat16)
    if wiring == "tp_lookup":
        eng.shard_rows(0, 1, device=DEV, dtype=torch.bfloat16, requires_grad=False)
        eng.row_lookup_fn = tp_lookup(lambda x: x)
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(-1, 1000, (48, 4), generator=gen, dtype=torch.int32).to(DEV)
    hidden = torch.randn(48, 64, generator=gen).to(device=DEV, dtype=torch.bfloat16)
    keep = (torch.arange(48) % 5 != 0).to(DEV)

    def layer(h, ids, keep):
        return eng.inject(h, eng.hash_prev(ids), keep)

    torch._dynamo.reset()
    with torch.no_grad():
        want = layer(hidden, ids, keep)
        compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
        got = compiled(hidden, ids, keep)
        again = compiled(hidden, ids, keep)
    torch._dynamo.reset()
    assert torch.equal(got, want) and torch.equal(again, want)
    assert not torch.equal(want, hidden)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_replaced_lookup_drops_the_four_gram_rows(gate_path, dtype):
    eng = _make(dtype)
    gen = torch.Generator().manual_seed(2)
    ids = torch.randint(1, 1000, (2, 20), generator=gen).to(DEV)
    h = torch.randn(2, 20, 64, generator=gen).to(device=DEV, dtype=dtype)
    zeroed = copy.deepcopy(eng)
    with torch.no_grad():
        for k, n in enumerate(zeroed._table_orders):
            if n == 4:
                zeroed.tables[k].weight.zero_()
        idx = eng.hash_ids(ids)
        mem = eng.lookup(idx)
        for k, n in enumerate(eng._table_orders):
            if n == 4:
                mem[k] = torch.zeros_like(mem[k])
        eng.lookup = lambda _i, m=mem: m  # the original engram, 4-gram lookups removed
        got = eng(h, ids)
        want = zeroed(h, ids)
    assert torch.equal(got, want)
    # against the oracle: the rows of the unmodified tables with the 4-gram part zeroed
    cpu_mem = torch.cat([m.float().cpu().reshape(-1, m.shape[-1]) for m in mem], dim=-1)
    ref = oracle.inject(h.cpu().reshape(-1, 64), cpu_mem.to(dtype), eng.key.weight.detach().cpu(),
                        eng.value.weight.detach().cpu(), "scalar_sqrt",
                        eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu())
    assert_close_out(got, ref.reshape(got.shape), h, dtype)
    assert not torch.equal(got, h)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_plain_lookup_carries_table_gradients(dtype):
    eng = _make(dtype)
    gen = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 60, (3, 50), generator=gen).to(DEV)  # few ids: repeated rows
    idx = eng.hash_ids(ids)
    rows = eng.lookup(idx)
    assert all(r.requires_grad and tuple(r.shape) == (3, 50, 8) for r in rows)
    weights = [torch.randn(3, 50, 8, generator=gen) for _ in rows]
    loss = sum((r.float() * w.to(DEV)).sum() for r, w in zip(rows, weights))
    loss.backward()
    for k, (t, w) in enumerate(zip(eng.tables, weights)):
        # the rows' gradient is w in the rows' dtype (the backward of .float())
        want = torch.zeros(t.weight.shape, dtype=torch.float32).index_add_(
            0, idx[k].reshape(-1).cpu(), w.to(dtype).float().reshape(-1, 8))
        assert torch.equal(t.weight.grad.cpu(), want.to(dtype)), k
    with torch.no_grad():
        assert not any(r.requires_grad for r in eng.lookup(idx))


def test_replaced_lookup_keeps_the_gradients():
    # inject through a replaced lookup that calls the class's own: every gradient equals the
    # one of the unreplaced engram, bit for bit
    def grads(replace):
        eng = _make(torch.float32).train()
        if replace:
            eng.lookup = lambda i, e=eng: MicroEngram.lookup(e, i)
        gen = torch.Generator().manual_seed(8)
        ids = torch.randint(0, 300, (2, 40), generator=gen).to(DEV)
        h = torch.randn(2, 40, 64, generator=gen).to(DEV).requires_grad_(True)
        out = eng(h, ids)
        out.backward(torch.randn(out.shape, generator=gen).to(DEV))
        named = {n: p.grad.clone() for n, p in eng.named_parameters()}
        named["hidden"] = h.grad.clone()
        return named

    a, b = grads(False), grads(True)
    assert a.keys() == b.keys()
    for name in a:
        assert torch.equal(a[name], b[name]), name
