"""Backward of the engram (stages 2-3) on the GPU against torch autograd of the oracle's CPU
restatement of MicroEngram.inject (module.py:228-261) with nn.Embedding-style lookups: the
gradients of hidden, of the key / value weights, of the q/k scale deltas and of the tables.

Tolerances (per gradient tensor, relative to the reference's largest entry):
  fp32  max |gpu - ref| <= 1e-4 * max |ref|   (fp32 GEMM and reduction orders differ)
  bf16  max |gpu - ref| <= 4e-2 * max |ref| and ||gpu - ref|| <= 1e-2 ||ref||: the products
        K, V and the gradients dK, dV are rounded to bf16 on both sides, and one-ulp flips of
        those roundings between the two accumulation orders move individual entries
The step-0 properties of test_gate.py:24-44 are exact.
"""
import pytest
import torch
import torch.nn.functional as F

import oracle
from micro_engram_fork_amd import MicroEngram, synthetic
from micro_engram_fork_amd.rows import RowTables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _make(dtype, gate, d, dim, heads, orders=(2, 3, 4), seed=0, std=0.2):
    eng = MicroEngram(model_dim=d, table_size=257, engram_dim=dim, num_heads=heads, orders=orders,
                      table_sizes={2: 131, 3: 257, 4: 97}, vocab_size=1000, gate=gate, seed=seed)
    synthetic.fill_dense(eng, seed=seed, std=std)
    return eng.to(device=DEV, dtype=dtype)


def _reference_grads(eng, hidden, ids, grad_out, keep=None):
    """torch autograd on the CPU of the oracle's inject over nn.Embedding lookups."""
    idx = [i.cpu() for i in eng.hash_ids(ids)]
    leaf = lambda t: t.detach().cpu().clone().requires_grad_(True)
    tables = [leaf(t.weight) for t in eng.tables]
    wk, wv = leaf(eng.key.weight), leaf(eng.value.weight)
    sqrt = eng.gate == "scalar_sqrt"
    dq = leaf(eng.q_scale) if sqrt else None
    dk = leaf(eng.k_scale) if sqrt else None
    h = leaf(hidden)
    d = hidden.shape[-1]
    mem = torch.cat([F.embedding(i.reshape(-1), t) for i, t in zip(idx, tables)], dim=-1)
    out = oracle.inject(h.reshape(-1, d), mem, wk, wv, eng.gate, dq, dk,
                        keep=None if keep is None else keep.cpu().reshape(-1))
    out.backward(grad_out.cpu().reshape(-1, d).to(out.dtype))
    grads = {"hidden": h.grad, "key": wk.grad, "value": wv.grad}
    if sqrt:
        grads["q_scale"], grads["k_scale"] = dq.grad, dk.grad
    for k, t in enumerate(tables):
        grads[f"table{k}"] = t.grad
    return out.detach(), grads


def _conditioned(eng, hidden, ids, grad_out, keep=None):
    """grad_out with the rows of tokens whose scalar_sqrt score is near 0 zeroed: there
    d sqrt|s0| / d s0 = 1 / (2 sqrt|s0|) amplifies the fp32 rounding of s0 itself (a sum of
    O(sqrt d) magnitude), so no two evaluation orders agree on those tokens' gradients. With
    |s| = sqrt|s0| >= 0.1 the amplification stays below ~1e-4 relative."""
    if eng.gate != "scalar_sqrt":
        return grad_out
    idx = [i.cpu() for i in eng.hash_ids(ids)]
    d = hidden.shape[-1]
    mem = torch.cat([F.embedding(i.reshape(-1), t.weight.detach().cpu()) for i, t in zip(idx, eng.tables)], -1)
    _, alpha = oracle.inject(hidden.cpu().reshape(-1, d), mem, eng.key.weight.detach().cpu(),
                             eng.value.weight.detach().cpu(), eng.gate, eng.q_scale.detach().cpu(),
                             eng.k_scale.detach().cpu(), return_alpha=True)
    s = torch.log(alpha / (1 - alpha))
    ok = (s.abs() >= 0.1).to(grad_out.dtype).to(grad_out.device)
    return grad_out * ok.reshape(*grad_out.shape[:-1], 1)


def _gpu_grads(eng, hidden, ids, grad_out, keep=None):
    eng.zero_grad(set_to_none=True)
    h = hidden.detach().clone().requires_grad_(True)
    if keep is None:
        out = eng(h, ids)
    else:
        out = eng.inject(h, eng.hash_ids(ids), keep=keep)
    out.backward(grad_out)
    grads = {"hidden": h.grad, "key": eng.key.weight.grad, "value": eng.value.weight.grad}
    if eng.gate == "scalar_sqrt":
        grads["q_scale"], grads["k_scale"] = eng.q_scale.grad, eng.k_scale.grad
    for k, t in enumerate(eng.tables):
        grads[f"table{k}"] = t.weight.grad
    return out.detach(), grads


def _assert_grads_close(got, want, dtype):
    assert set(got) == set(want)
    for name in want:
        g, w = got[name].float().cpu(), want[name].float()
        assert g.shape == w.shape, name
        scale = float(w.abs().max())
        err = (g - w).abs()
        if dtype == torch.float32:
            assert float(err.max()) <= 1e-4 * scale + 1e-12, (name, float(err.max()), scale)
        else:
            assert float(err.max()) <= 4e-2 * scale + 1e-12, (name, float(err.max()), scale)
            assert float((g - w).norm()) <= 1e-2 * float(w.norm()) + 1e-12, (name, float((g - w).norm()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", ["scalar_sqrt", "scalar"])
@pytest.mark.parametrize("n,d,dim,heads", [(300, 264, 8, 3), (600, 520, 16, 4)])
def test_backward_matches_autograd(dtype, gate, n, d, dim, heads):
    torch.manual_seed(n + d)
    eng = _make(dtype, gate, d, dim, heads).train()
    ids = torch.randint(0, 1000, (1, n), device=DEV)
    hidden = (torch.randn(1, n, d) * 3).to(dtype).to(DEV)
    grad_out = _conditioned(eng, hidden, ids, torch.randn(1, n, d).to(dtype).to(DEV))
    out, got = _gpu_grads(eng, hidden, ids, grad_out)
    ref_out, want = _reference_grads(eng, hidden, ids, grad_out)
    _assert_grads_close(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_with_keep(dtype):
    torch.manual_seed(3)
    eng = _make(dtype, "scalar_sqrt", 136, 8, 2).train()
    n = 260
    ids = torch.randint(0, 1000, (1, n), device=DEV)
    hidden = torch.randn(1, n, 136).to(dtype).to(DEV)
    grad_out = _conditioned(eng, hidden, ids, torch.randn(1, n, 136).to(dtype).to(DEV))
    keep = torch.rand(n, device=DEV) > 0.4
    _, got = _gpu_grads(eng, hidden, ids, grad_out, keep=keep)
    _, want = _reference_grads(eng, hidden, ids, grad_out, keep=keep)
    _assert_grads_close(got, want, dtype)
    # tokens without memory pass the output gradient straight through
    assert torch.equal(got["hidden"][0][~keep], grad_out[0][~keep])


def test_step0_gradients():
    # test_gate.py:24-44: with the zero-init value layer the output is hidden, only the value
    # layer gets a gradient; once it is non-zero, the tables learn too
    for dtype in (torch.float32, torch.bfloat16):
        eng = MicroEngram(model_dim=32, table_size=257, engram_dim=4, num_heads=2, vocab_size=1000,
                          gate="scalar_sqrt").to(device=DEV, dtype=dtype).train()
        ids = torch.randint(5, 1000, (2, 12), device=DEV)
        hidden = (torch.randn(2, 12, 32) * 50).to(dtype).to(DEV).requires_grad_(True)
        out = eng(hidden, ids)
        assert torch.equal(out, hidden)
        g = torch.randn_like(out)
        out.backward(g)
        assert torch.equal(hidden.grad, g)
        assert eng.value.weight.grad.abs().sum() > 0
        assert not eng.key.weight.grad.any() and not eng.q_scale.grad.any()
        assert all(not t.weight.grad.any() for t in eng.tables)
        eng.zero_grad()
        with torch.no_grad():
            eng.value.weight.normal_(std=0.02)
        eng(hidden.detach(), ids).pow(2).sum().backward()
        assert eng.tables[0].weight.grad.abs().sum() > 0
        assert eng.q_scale.grad.abs().sum() > 0 and eng.k_scale.grad.abs().sum() > 0


def test_sparse_row_gradients_equal_dense():
    # row shards at world size 1 with sparse gradients (rows.py:137-147): the coalesced
    # (rows, fp32 sums) equal the dense table gradient's non-zero rows
    torch.manual_seed(9)
    dense = _make(torch.float32, "scalar_sqrt", 64, 8, 2).train()
    sparse = _make(torch.float32, "scalar_sqrt", 64, 8, 2).train()
    sparse.load_state_dict(dense.state_dict())
    sparse.shard_rows(0, 1)
    rt = RowTables([("e", sparse)], lazy=True, rowwise=True, sparse_grads=True)
    ids = torch.randint(0, 1000, (2, 100), device=DEV)
    hidden = torch.randn(2, 100, 64, device=DEV)
    g = torch.randn(2, 100, 64, device=DEV)
    dense(hidden, ids).backward(g)
    sparse(hidden, ids).backward(g)
    for t, shard in zip(dense.tables, sparse.row_shards):
        rows, sums = shard.sparse_grad
        want = t.weight.grad
        nz = want.abs().sum(-1).nonzero().reshape(-1)
        assert torch.equal(torch.sort(rows).values, rows)
        assert set(nz.tolist()) <= set(rows.tolist())
        assert torch.equal(sums, want[rows])
    assert torch.equal(dense.key.weight.grad, sparse.key.weight.grad)
    rt.zero_grad()


def test_backward_gemma_prefill_full():
    # the training step's backward at the headline shape: 8192 tokens, model dim 5376, 24 bf16
    # tables of the Gemma-scale sizes (dense table gradients here; the sparse row path is
    # checked against these by test_sparse_row_gradients_equal_dense), every gradient against
    # torch autograd of the oracle on the CPU
    eng = synthetic.build_engram("gemma", DEV, seed=7).train()
    ids, pos, hidden = synthetic.prefill_inputs(seed=5, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(9)
    grad_out = torch.randn(hidden.shape, generator=gen, device=DEV).to(torch.bfloat16)
    idx = eng.hash_ids(ids, pos)
    d = hidden.shape[-1]
    # tokens whose score is near 0 get no output gradient (see _conditioned)
    mem = torch.cat([t.weight.detach()[i.reshape(-1)] for i, t in zip(idx, eng.tables)], -1).cpu()
    _, alpha = oracle.inject(hidden.cpu().reshape(-1, d), mem, eng.key.weight.detach().cpu(),
                             eng.value.weight.detach().cpu(), eng.gate, eng.q_scale.detach().cpu(),
                             eng.k_scale.detach().cpu(), return_alpha=True)
    ok = (torch.log(alpha / (1 - alpha)).abs() >= 0.1).to(grad_out.dtype).to(DEV)
    grad_out = grad_out * ok.reshape(*grad_out.shape[:-1], 1)

    eng.zero_grad(set_to_none=True)
    h = hidden.detach().clone().requires_grad_(True)
    eng.inject(h, idx).backward(grad_out)
    got = {"hidden": h.grad, "key": eng.key.weight.grad, "value": eng.value.weight.grad,
           "q_scale": eng.q_scale.grad, "k_scale": eng.k_scale.grad}
    got.update({f"table{k}": t.weight.grad for k, t in enumerate(eng.tables)})

    leaf = lambda t: t.detach().cpu().clone().requires_grad_(True)
    tables = [leaf(t.weight) for t in eng.tables]
    wk, wv, dq, dk, hc = leaf(eng.key.weight), leaf(eng.value.weight), leaf(eng.q_scale), leaf(eng.k_scale), leaf(hidden)
    mem = torch.cat([F.embedding(i.cpu().reshape(-1), t) for i, t in zip(idx, tables)], dim=-1)
    out = oracle.inject(hc.reshape(-1, d), mem, wk, wv, eng.gate, dq, dk)
    out.backward(grad_out.cpu().reshape(-1, d).to(out.dtype))
    want = {"hidden": hc.grad, "key": wk.grad, "value": wv.grad, "q_scale": dq.grad, "k_scale": dk.grad}
    want.update({f"table{k}": t.grad for k, t in enumerate(tables)})
    _assert_grads_close(got, want, torch.bfloat16)
    del want, tables, mem, out, hc

    # the same batch through row shards with sparse gradients (the key plan made in the forward,
    # the segment sums in the backward): each table's (rows, fp32 sums) are its dense gradient's
    # non-zero rows, and the other gradients are the dense path's, bit for bit
    key_grad, hidden_grad = got["key"].clone(), got["hidden"].clone()
    eng.zero_grad(set_to_none=True)
    shards = eng.shard_rows(0, 1, device=DEV)
    rt = RowTables([("e", eng)], lazy=True, rowwise=True, sparse_grads=True)
    h2 = hidden.detach().clone().requires_grad_(True)
    eng.inject(h2, idx).backward(grad_out)
    for k, shard in enumerate(shards):
        rows, sums = shard.sparse_grad
        dense = got[f"table{k}"]
        assert torch.equal(sums.to(dense.dtype), dense[rows])
        assert bool(torch.isin(dense.abs().sum(-1).nonzero().reshape(-1), rows).all())
    assert torch.equal(eng.key.weight.grad, key_grad)
    assert torch.equal(h2.grad, hidden_grad)
    rt.zero_grad()
    del eng, got, shards
    torch.cuda.empty_cache()


def test_empty_batch_zeroes_the_scale_gradients_in_a_graph():
    # no tokens: the scale-delta gradients are zero, written by a fill kernel (so a captured
    # backward records no memset node); checked eagerly and on every replay of a captured call
    from micro_engram_fork_amd import _lib
    from micro_engram_fork_amd._lib import ME_BF16, ME_F32, ME_GATE_SCALAR_SQRT

    d = 1000
    gq = torch.full((d,), 7.0, device=DEV)
    gk = torch.full((d,), 7.0, device=DEV)
    dummy = torch.zeros(64, dtype=torch.bfloat16, device=DEV)
    deltas = torch.zeros(d, device=DEV)

    def call():
        p = dummy.data_ptr()
        _lib.call("me_gate_backward", p, ME_BF16, 0, d, p, 16, p, p, ME_BF16, deltas.data_ptr(),
                  deltas.data_ptr(), ME_F32, ME_GATE_SCALAR_SQRT, None, p, None, p, p, p,
                  gq.data_ptr(), gk.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)

    call()
    torch.cuda.synchronize()
    assert not gq.any() and not gk.any()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.synchronize()
    for _ in range(3):
        gq.fill_(7.0)
        gk.fill_(-3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert not gq.any() and not gk.any()


def _ulp_bf16(x):
    x = x.abs().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(x)) - 7)


def _check_backward_at_forward_stats(eng, x, mem, g, dtype, rows=None, keep=None):
    """The HIP gate backward against the float64 closed form evaluated at the GPU forward's own
    row statistics (oracle.inject_backward(stats=...)), on every token in `rows` (all by
    default) -- including those with scalar_sqrt scores near 0, whose gradients the end-to-end
    tests leave out. Per element: |gpu - ref| <= rounding of the stored value + a multiple of
    the magnitudes the products are made of (bf16: K and V are bf16-rounded on the GPU)."""
    from micro_engram_fork_amd import ops
    from micro_engram_fork_amd._lib import ME_GATE_SCALAR_SQRT

    wk, wv = eng.key.weight.detach(), eng.value.weight.detach()
    dq, dk = eng.q_scale.detach(), eng.k_scale.detach()
    out, alpha, stats = ops.gate_residual(x, mem, wk, wv, dq, dk, ME_GATE_SCALAR_SQRT, keep, True, True)
    gh, gK, gV, gq, gk = ops.gate_backward(g, x, mem, wk, wv, dq, dk, ME_GATE_SCALAR_SQRT, keep, stats)
    sel = torch.arange(x.shape[0]) if rows is None else rows
    c = lambda t: t.detach().cpu()[sel]
    ref = oracle.inject_backward(c(g), c(x), c(mem), wk.cpu(), wv.cpu(), "scalar_sqrt", dq.cpu(),
                                 dk.cpu(), keep=None if keep is None else c(keep), stats=c(stats),
                                 with_terms=True)
    t_dx, t_dk, t_p = ref[5]
    rel = 2.0 ** -6 if dtype == torch.bfloat16 else 1e-5
    store = _ulp_bf16 if dtype == torch.bfloat16 else (lambda v: 1e-6 * v.abs())
    for name, got, want, term in (("hidden", gh, ref[0], t_dx), ("dK", gK, ref[1], t_dk),
                                  ("dV", gV, ref[2], torch.zeros_like(ref[2]))):
        got = got.detach().cpu()[sel].double()
        bound = store(want) + rel * term + 1e-30
        bad = (got - want).abs() > bound
        assert not bool(bad.any()), (name, int(bad.sum()), float((got - want).abs().max()))
    if rows is None:  # the scale gradients sum over every token
        ks, qs = 1 + dk.cpu().double(), 1 + dq.cpu().double()
        for name, got, want, scale in (("q_scale", gq, ref[3], ks), ("k_scale", gk, ref[4], qs)):
            err = (got.detach().cpu().double() - want).abs()
            assert bool((err <= 4 * rel * scale.abs() * t_p + 1e-12).all()), (name, float(err.max()))
    s = torch.log(alpha / (1 - alpha)).cpu()[sel]
    return int((s.abs() < 0.1).sum())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,d,dim,heads", [(300, 264, 8, 3), (1000, 520, 16, 4)])
def test_backward_at_the_forwards_stats_on_every_token(dtype, n, d, dim, heads):
    # no output gradient is zeroed: tokens with |s| < 0.1 are compared like the others
    torch.manual_seed(n + d + 1)
    eng = _make(dtype, "scalar_sqrt", d, dim, heads)
    ids = torch.randint(0, 1000, (1, n), device=DEV)
    x = (torch.randn(n, d) * 3).to(dtype).to(DEV)
    g = torch.randn(n, d).to(dtype).to(DEV)
    keep = torch.rand(n, device=DEV) > 0.2
    mem = eng.hashed_memory(ids)
    near_zero = _check_backward_at_forward_stats(eng, x, mem, g, dtype, keep=keep)
    _check_backward_at_forward_stats(eng, x, mem, g, dtype)
    if n >= 1000:
        assert near_zero > 0  # the case the end-to-end tests leave out is covered


def test_backward_at_the_forwards_stats_gemma_prefill():
    # the headline shape (8192 tokens, model dim 5376, 24 bf16 tables): every token with
    # |s| < 0.1 plus 256 others, against the float64 closed form at the GPU forward's stats
    eng = synthetic.build_engram("gemma", DEV, seed=7)
    ids, pos, hidden = synthetic.prefill_inputs(seed=5, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(9)
    x = hidden.reshape(-1, hidden.shape[-1])
    g = torch.randn(x.shape, generator=gen, device=DEV).to(torch.bfloat16)
    mem = eng.hashed_memory(ids, pos)
    from micro_engram_fork_amd import ops
    from micro_engram_fork_amd._lib import ME_GATE_SCALAR_SQRT

    _, alpha = ops.gate_residual(x, mem, eng.key.weight.detach(), eng.value.weight.detach(),
                                 eng.q_scale.detach(), eng.k_scale.detach(), ME_GATE_SCALAR_SQRT,
                                 None, True)
    s = torch.log(alpha / (1 - alpha)).cpu()
    low = torch.nonzero(s.abs() < 0.1).reshape(-1)
    others = torch.randperm(x.shape[0], generator=torch.Generator().manual_seed(3))[:256]
    rows = torch.unique(torch.cat([low, others]))
    near_zero = _check_backward_at_forward_stats(eng, x, mem, g, torch.bfloat16, rows=rows)
    assert near_zero == low.numel() > 0
    del eng
    torch.cuda.empty_cache()
