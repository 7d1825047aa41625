"""Engrams of any model dim and memory width (the reference's nn.Linear path takes any,
micro_engram/module.py:52-54, 76-79): shapes the MFMA kernels do not take (model dim not a
multiple of 8, memory rows not a multiple of 16 bytes) run library GEMMs for K and V and the
HIP row kernels (me_gate_rows with one column per lane, me_gate_rows_backward) for the gate,
the residual add and their backward. Checked against the oracle like the MFMA path:

  forward   test_gate_gpu's bounds (fp32 1e-5 rms(hidden); bf16 1 ulp + 2^-6 |ref - hidden|)
  backward  torch autograd of the oracle (test_gate_backward_gpu's bounds), and the float64
            closed form at the GPU forward's statistics on every token
"""
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, ops, synthetic
from micro_engram_fork_amd._lib import ME_GATE_SCALAR_SQRT

from test_gate_gpu import assert_close_out
from test_gate_backward_gpu import (_assert_grads_close, _conditioned, _gpu_grads,
                                    _reference_grads, _ulp_bf16)

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (model dim, engram dim, heads): model dim 37 / 100 / 36 (not multiples of 8), engram dims 3 and
# 5 (rows of 6 / 10 bf16 bytes); the last has MFMA-sized memory rows and an odd model dim
SHAPES = [(37, 3, 2), (100, 5, 3), (36, 8, 2)]


def _make(dtype, gate, d, dim, heads, seed=0):
    eng = MicroEngram(model_dim=d, table_size=257, engram_dim=dim, num_heads=heads, orders=(2, 3, 4),
                      table_sizes={2: 131, 3: 257, 4: 97}, vocab_size=1000, gate=gate, seed=seed)
    synthetic.fill_dense(eng, seed=seed, std=0.2)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for t in eng.tables:
            t.weight.copy_(torch.randn(t.weight.shape, generator=g) * 0.3)
    return eng.to(device=DEV, dtype=dtype)


def _oracle_forward(eng, hidden, ids, keep=None):
    idx = [i.cpu() for i in eng.hash_ids(ids)]
    mem = torch.cat([torch.nn.functional.embedding(i.reshape(-1), t.weight.detach().cpu())
                     for i, t in zip(idx, eng.tables)], dim=-1)
    sqrt = eng.gate == "scalar_sqrt"
    d = hidden.shape[-1]
    return oracle.inject(hidden.cpu().reshape(-1, d), mem, eng.key.weight.detach().cpu(),
                         eng.value.weight.detach().cpu(), eng.gate,
                         eng.q_scale.detach().cpu() if sqrt else None,
                         eng.k_scale.detach().cpu() if sqrt else None,
                         keep=None if keep is None else keep.cpu().reshape(-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", ["scalar_sqrt", "scalar"])
@pytest.mark.parametrize("d,dim,heads", SHAPES)
def test_forward_any_width(dtype, gate, d, dim, heads):
    eng = _make(dtype, gate, d, dim, heads).eval()
    assert not ops.fits_mfma(d, dim * heads * 3, dtype)
    gen = torch.Generator().manual_seed(d)
    ids = torch.randint(0, 1000, (2, 70), generator=gen).to(DEV)
    hidden = (torch.randn(2, 70, d, generator=gen) * 2).to(dtype).to(DEV)
    keep = (torch.rand(140, generator=gen) > 0.25).to(DEV)
    with torch.no_grad():
        out = eng(hidden, ids)
        out_keep = eng.inject(hidden, eng.hash_ids(ids), keep=keep)
    assert_close_out(out, _oracle_forward(eng, hidden, ids).reshape(out.shape), hidden, dtype)
    ref_keep = _oracle_forward(eng, hidden, ids, keep).reshape(out.shape)
    assert_close_out(out_keep, ref_keep, hidden, dtype)
    dropped = ~keep.reshape(2, 70)
    assert torch.equal(out_keep[dropped], hidden[dropped])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", ["scalar_sqrt", "scalar"])
@pytest.mark.parametrize("d,dim,heads", SHAPES)
def test_backward_any_width(dtype, gate, d, dim, heads):
    torch.manual_seed(d + dim)
    eng = _make(dtype, gate, d, dim, heads).train()
    ids = torch.randint(0, 1000, (1, 300), device=DEV)
    hidden = (torch.randn(1, 300, d) * 3).to(dtype).to(DEV)
    grad_out = _conditioned(eng, hidden, ids, torch.randn(1, 300, d).to(dtype).to(DEV))
    _, got = _gpu_grads(eng, hidden, ids, grad_out)
    _, want = _reference_grads(eng, hidden, ids, grad_out)
    _assert_grads_close(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d,dim,heads", SHAPES)
def test_row_backward_at_the_forwards_stats(dtype, d, dim, heads):
    # every token, |s| < 0.1 included, against the float64 closed form at the GPU forward's
    # statistics; K and V from the library GEMM, rounded to the engram dtype as nn.Linear does
    eng = _make(dtype, "scalar_sqrt", d, dim, heads)
    gen = torch.Generator().manual_seed(7 + d)
    n = 500
    ids = torch.randint(0, 1000, (1, n), generator=gen).to(DEV)
    x = (torch.randn(n, d, generator=gen) * 2).to(dtype).to(DEV)
    g = torch.randn(n, d, generator=gen).to(dtype).to(DEV)
    keep = (torch.rand(n, generator=gen) > 0.2).to(DEV)
    mem = eng.hashed_memory(ids)
    wk, wv = eng.key.weight.detach(), eng.value.weight.detach()
    dq, dk = eng.q_scale.detach(), eng.k_scale.detach()
    K, V = torch.nn.functional.linear(mem, wk), torch.nn.functional.linear(mem, wv)
    out, alpha, stats = ops.gate_rows(x, K, V, dq, dk, ME_GATE_SCALAR_SQRT, keep, True, True)
    gh, gK, gV, gq, gk = ops.gate_rows_backward(g, x, K, V, dq, dk, ME_GATE_SCALAR_SQRT, keep, stats)
    c = lambda t: t.detach().cpu()
    ref = oracle.inject_backward(c(g), c(x), c(mem), c(wk), c(wv), "scalar_sqrt", c(dq), c(dk),
                                 keep=c(keep), stats=c(stats), with_terms=True)
    t_dx, t_dk, t_p = ref[5]
    rel = 2.0 ** -6 if dtype == torch.bfloat16 else 1e-5
    store = _ulp_bf16 if dtype == torch.bfloat16 else (lambda v: 1e-6 * v.abs())
    for name, got, want, term in (("hidden", gh, ref[0], t_dx), ("dK", gK, ref[1], t_dk),
                                  ("dV", gV, ref[2], torch.zeros_like(ref[2]))):
        err = (c(got).double() - want).abs()
        bad = err > store(want) + rel * term + 1e-30
        assert not bool(bad.any()), (name, int(bad.sum()), float(err.max()))
    for name, got, want, scale in (("q_scale", gq, ref[3], 1 + c(dk).double()),
                                   ("k_scale", gk, ref[4], 1 + c(dq).double())):
        err = (c(got).double() - want).abs()
        assert bool((err <= 4 * rel * scale.abs() * t_p + 1e-12).all()), (name, float(err.max()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_row_kernels_narrow_and_wide_agree(dtype):
    # an MFMA-sized shape through the row kernels twice: 16-byte accesses (8 columns per lane)
    # and, from operands offset to break the 16-byte alignment, one column per lane -- the same
    # sums in another order, so within the forward's bounds of each other; and the same shape
    # through the MFMA path (me_gate_residual) within the bounds too
    n, d, m = 200, 64, 48
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(n, d, generator=gen).to(dtype).to(DEV)
    mem = (torch.randn(n, m, generator=gen) * 0.5).to(dtype).to(DEV)
    wk = (torch.randn(d, m, generator=gen) * 0.2).to(dtype).to(DEV)
    wv = (torch.randn(d, m, generator=gen) * 0.2).to(dtype).to(DEV)
    dq = (torch.randn(d, generator=gen) * 0.1).to(DEV)
    dk = (torch.randn(d, generator=gen) * 0.1).to(DEV)
    K, V = torch.nn.functional.linear(mem, wk), torch.nn.functional.linear(mem, wv)
    wide = ops.gate_rows(x, K, V, dq, dk, ME_GATE_SCALAR_SQRT, None, False)[0]

    def shifted(t):  # the same values one element past a 16-byte boundary
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=DEV)
        view = buf[1:].view(t.shape)
        view.copy_(t)
        return view

    narrow = ops.gate_rows(shifted(x), shifted(K), shifted(V), dq, dk, ME_GATE_SCALAR_SQRT, None, False)[0]
    mfma = ops.gate_residual(x, mem, wk, wv, dq, dk, ME_GATE_SCALAR_SQRT, None, False)[0]
    assert_close_out(narrow, wide, x, dtype)
    assert_close_out(mfma, wide, x, dtype)
    assert not torch.equal(wide, x)


def test_row_backward_empty_batch():
    d = 37
    z = torch.zeros(0, d, dtype=torch.bfloat16, device=DEV)
    dq = torch.randn(d, device=DEV)
    dk = torch.randn(d, device=DEV)
    outs = ops.gate_rows_backward(z, z, z, z, dq, dk, ME_GATE_SCALAR_SQRT, None,
                                  torch.zeros(0, 4, device=DEV))
    assert outs[0].shape == (0, d) and not outs[3].any() and not outs[4].any()
