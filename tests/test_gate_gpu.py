"""Stage 3 (key/value projection + scalar gates + residual) and the whole forward on the GPU
against the oracle's torch-CPU restatement of MicroEngram.inject (module.py:228-261).

Tolerances (stated per dtype, checked per element):
  fp32  |gpu - ref| <= 1e-5 * rms(hidden row)
  bf16  |gpu - ref| <= 1 bf16 ulp of the output + 2^-6 * |ref - hidden| : one rounding step of
        the residual add plus the effect of a one-ulp flip in the bf16 K/V products;
        and per row max|gpu - ref| <= 1e-2 * ||hidden row||_2
  gate  |alpha_gpu - alpha_ref| <= 1e-5 (fp32) / 2e-3 (bf16)
"""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, ops, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True, params=["fused", "rows"])
def gate_path(request, monkeypatch):
    """Every test of this file runs on both gate paths of MicroEngram: the fused two-pass kernel
    (me_gate_residual) and, for few tokens, the hand-written projection (me_kv_proj) + row
    kernel (me_gate_rows)."""
    limit = 0 if request.param == "fused" else 1 << 30
    monkeypatch.setattr(MicroEngram, "few_tokens_max", limit)
    monkeypatch.setattr(MicroEngram, "few_tokens_max_fp32", limit)
    monkeypatch.setattr(MicroEngram, "few_tokens_kv_bytes", 0 if limit == 0 else 1 << 62)
    return request.param


def _bf16_ulp(x):
    x = x.abs().float().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(x)) - 7)


def assert_close_out(got, ref, hidden, dtype):
    got, ref, hidden = got.float().cpu(), ref.float().cpu(), hidden.float().cpu()
    got, ref, hidden = (t.reshape(-1, t.shape[-1]) for t in (got, ref, hidden))
    err = (got - ref).abs()
    if dtype == torch.float32:
        rms = hidden.pow(2).mean(-1, keepdim=True).sqrt()
        bad = err > 1e-5 * rms + 1e-30
    else:
        bound = _bf16_ulp(torch.maximum(got.abs(), ref.abs())) + 2.0 ** -6 * (ref - hidden).abs()
        bad = err > bound
        row_norm = hidden.norm(dim=-1)
        assert (err.max(dim=-1).values <= 1e-2 * row_norm).all()
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance, max err {float(err.max()):.3g}"


def _make(dtype, gate="scalar_sqrt", d=32, dim=4, heads=2, orders=(2, 3), sizes=None, seed=0):
    eng = MicroEngram(model_dim=d, table_size=257, engram_dim=dim, num_heads=heads, orders=orders,
                      table_sizes=sizes, vocab_size=1000, gate=gate, seed=seed)
    synthetic.fill_dense(eng, seed=seed, std=0.2)
    return eng.to(device=DEV, dtype=dtype).eval()


def _oracle_forward(eng, hidden, ids, pos=None, keep=None):
    idx = oracle.hash_ids(ids.cpu().numpy(), eng.mults.cpu().numpy(), eng._table_orders,
                          eng.table_rows, eng.canon.cpu().numpy(), eng.pad_id,
                          position_ids=None if pos is None else pos.cpu().numpy())
    tables = [t.weight.detach().cpu().float().numpy() for t in eng.tables]
    mem = torch.from_numpy(oracle.lookup(tables, list(idx.reshape(idx.shape[0], -1))))
    mem = mem.to(eng.key.weight.dtype)
    sqrt = eng.gate == "scalar_sqrt"
    d = hidden.shape[-1]
    return oracle.inject(hidden.cpu().reshape(-1, d), mem, eng.key.weight.detach().cpu(),
                         eng.value.weight.detach().cpu(), eng.gate,
                         eng.q_scale.detach().cpu() if sqrt else None,
                         eng.k_scale.detach().cpu() if sqrt else None,
                         keep=None if keep is None else keep.cpu().reshape(-1), return_alpha=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gate", ["scalar_sqrt", "scalar"])
def test_forward_small(dtype, gate):
    torch.manual_seed(0)
    eng = _make(dtype, gate)
    ids = torch.randint(5, 1000, (2, 12), device=DEV)
    hidden = (torch.randn(2, 12, 32) * 50).to(dtype).to(DEV)
    with torch.no_grad():
        out = eng(hidden, ids)
    ref, _ = _oracle_forward(eng, hidden, ids)
    assert out.dtype == dtype and out.shape == hidden.shape
    assert_close_out(out, ref.reshape(out.shape), hidden, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gate_alpha_matches(dtype):
    torch.manual_seed(1)
    eng = _make(dtype, d=64, dim=8, heads=2, orders=(2, 3, 4))
    ids = torch.randint(0, 1000, (1, 300), device=DEV)
    hidden = torch.randn(1, 300, 64).to(dtype).to(DEV)
    idx = eng.hash_ids(ids)
    mem = torch.cat(eng.lookup(idx), dim=-1).reshape(300, -1)
    with torch.no_grad():
        out, alpha = ops.gate_residual(hidden, mem, eng.key.weight, eng.value.weight, eng.q_scale,
                                       eng.k_scale, 1, None, True)
    ref, ref_alpha = _oracle_forward(eng, hidden, ids)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    assert (alpha.cpu() - ref_alpha).abs().max() <= tol
    assert_close_out(out, ref.reshape(out.shape), hidden, dtype)


def test_step0_is_exact_noop():
    # value weight zero (a fresh engram): output == input exactly (test_gate.py:24-27)
    for dtype in (torch.float32, torch.bfloat16):
        eng = MicroEngram(model_dim=32, table_size=257, engram_dim=4, num_heads=2, vocab_size=1000,
                          gate="scalar_sqrt").to(device=DEV, dtype=dtype)
        hidden = (torch.randn(2, 12, 32) * 50).to(dtype).to(DEV)
        with torch.no_grad():
            out = eng(hidden, torch.randint(5, 1000, (2, 12), device=DEV))
        assert torch.equal(out, hidden)


def test_keep_mask():
    # keep=False rows unchanged, keep=True rows as without the mask (test_gate.py:122-130)
    eng = _make(torch.float32)
    ids = torch.randint(5, 1000, (2, 12), device=DEV)
    hidden = (torch.randn(2, 12, 32) * 50).to(DEV)
    keep = torch.tensor([[True] * 6 + [False] * 6] * 2, device=DEV)
    with torch.no_grad():
        idx = eng.hash_ids(ids)
        masked, full = eng.inject(hidden, idx, keep), eng.inject(hidden, idx)
    assert torch.equal(masked[:, 6:], hidden[:, 6:])
    assert torch.equal(masked[:, :6], full[:, :6])


def test_inject_does_not_modify_hidden():
    eng = _make(torch.bfloat16)
    hidden = torch.randn(5, 32, device=DEV).to(torch.bfloat16)
    before = hidden.clone()
    with torch.no_grad():
        eng.inject(hidden, eng.hash_prev(torch.randint(-1, 1000, (5, 3), device=DEV)))
    assert torch.equal(hidden, before)


def test_gate_stats_recorded_in_training_mode():
    eng = _make(torch.float32).train()
    with torch.no_grad():
        eng(torch.randn(1, 40, 32, device=DEV), torch.randint(0, 1000, (1, 40), device=DEV))
    mean, sat = eng.pop_gate_stats()
    assert 0.0 < mean < 1.0 and 0.0 <= sat <= 1.0
    eng.eval()
    with torch.no_grad():
        eng(torch.randn(1, 40, 32, device=DEV), torch.randint(0, 1000, (1, 40), device=DEV))
    assert eng.pop_gate_stats() is None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_grad_path_forward_equals_fused(dtype):
    # with gradients the forward hashes, gathers through the differentiable row lookup and
    # keeps the gate's row sums; its output is the fused inference forward's, bit for bit
    eng = _make(dtype, d=64, dim=8, heads=2, orders=(2, 3, 4)).train()
    eng.few_tokens_max = eng.few_tokens_max_fp32 = 0  # the fused kernel, as the gradient path
    ids = torch.randint(0, 1000, (2, 70), device=DEV)
    hidden = torch.randn(2, 70, 64).to(dtype).to(DEV)
    with torch.no_grad():
        fused = eng(hidden, ids)
    out = eng(hidden.clone().requires_grad_(True), ids)
    assert out.requires_grad and torch.equal(out.detach(), fused)


def test_golden_inject_fixture():
    import os

    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "inject_small.npz"))
    t = {k: torch.from_numpy(f[k]).to(DEV) for k in f.files}
    with torch.no_grad():
        out, alpha = ops.gate_residual(t["hidden"], t["mem"], t["wk"], t["wv"], t["dq"], t["dk"], 1,
                                       None, True)
    assert (alpha.cpu() - torch.from_numpy(f["alpha"])).abs().max() <= 1e-5
    assert_close_out(out, torch.from_numpy(f["out"]), t["hidden"], torch.float32)


@pytest.mark.parametrize("n,d,dim,heads", [(300, 264, 8, 3), (513, 1024, 16, 2), (7, 4096, 64, 8),
                                            (600, 776, 64, 8), (1100, 520, 32, 5), (260, 448, 64, 1),
                                            (50, 232, 32, 2), (40, 5632, 32, 2)])
def test_ragged_shapes_bf16(n, d, dim, heads):
    # token counts and model dims that are not multiples of the tiles; K from 2 to 24 128-byte
    # slabs. Whole slabs, at least three, take the 224-column kernel (M = 192: three slabs, d = 448
    # two whole column tiles, d = 232 a second tile of 8 columns, d = 5632 26 column tiles, past
    # the 24 whose gate sums the value pass loads late, the last of 32 columns); partial slabs the
    # 256 x 256 one (M = 72, 96, 480)
    torch.manual_seed(n)
    eng = _make(torch.bfloat16, d=d, dim=dim, heads=heads, orders=(2, 3, 4))
    ids = torch.randint(0, 1000, (1, n), device=DEV)
    hidden = torch.randn(1, n, d).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        out = eng(hidden, ids)
    ref, _ = _oracle_forward(eng, hidden, ids)
    assert_close_out(out, ref.reshape(out.shape), hidden, torch.bfloat16)


def test_tiny_forward_fp32_full():
    eng = synthetic.build_engram("tiny", DEV, seed=0).eval()
    ids, pos, hidden = synthetic.tiny_inputs(seed=0, device=DEV)
    with torch.no_grad():
        out = eng(hidden, ids, pos)
    ref, _ = _oracle_forward(eng, hidden, ids, pos)
    assert_close_out(out, ref.reshape(out.shape), hidden, torch.float32)


def test_gemma_prefill_forward_full():
    # the headline workload end to end: all 8192 tokens of a Gemma-scale prefill batch (fused
    # hash + gather, then the 256 x 224 gate passes) against the oracle's inject on the same rows
    eng = synthetic.build_engram("gemma", DEV, seed=0).eval()
    ids, pos, hidden = synthetic.prefill_inputs(seed=0, device=DEV)
    with torch.no_grad():
        out = eng(hidden, ids, pos)
        idx = torch.stack(eng.hash_ids(ids, pos)).reshape(len(eng.tables), -1)
        mem = torch.cat([t.weight[idx[k]] for k, t in enumerate(eng.tables)], dim=-1).cpu()
    h = hidden.reshape(-1, hidden.shape[-1]).cpu()
    ref = oracle.inject(h, mem, eng.key.weight.detach().cpu(), eng.value.weight.detach().cpu(),
                        "scalar_sqrt", eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu())
    assert_close_out(out.reshape(-1, out.shape[-1]), ref, h, torch.bfloat16)
    del eng
    torch.cuda.empty_cache()


def test_projection_rounds_to_nearest_even():
    # hidden = 0 makes the scalar gate exactly 0.5 (s = 0), so out = 0.5 * bf16(W_V e) exactly:
    # the projection's fp32 -> bf16 rounding is observed directly, ties included
    d, M = 64, 16
    k = torch.arange(d, dtype=torch.float32) - 32           # t = k / 512: every rounding case
    t = (k / 512).to(torch.bfloat16)
    wv = torch.zeros(d, M, dtype=torch.bfloat16)
    wv[:, 0] = torch.where(k >= 0, 1.0, -1.0).to(torch.bfloat16)
    wv[:, 1] = t
    mem = torch.zeros(4, M, dtype=torch.bfloat16)
    mem[:, 0] = 1.0
    mem[:, 1] = 1.0
    hidden = torch.zeros(4, d, dtype=torch.bfloat16)
    wk = torch.ones(d, M, dtype=torch.bfloat16)
    with torch.no_grad():
        out, alpha = ops.gate_residual(hidden.to(DEV), mem.to(DEV), wk.to(DEV), wv.to(DEV), None, None,
                                       0, None, True)
    assert torch.equal(alpha.cpu(), torch.full((4,), 0.5))
    want = (wv[:, 0].float() + t.float()).to(torch.bfloat16)  # fp32 sum is exact; RNE to bf16
    assert torch.equal((out.cpu().float() * 2).to(torch.bfloat16), want.expand(4, d))


@pytest.mark.parametrize("hdt,tdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                     (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("gate", [0, 1])
@pytest.mark.parametrize("n,d,m", [(1, 64, 32), (37, 520, 96), (256, 1024, 256), (300, 5376, 1536)])
def test_rows_path_matches_fused_and_oracle(hdt, tdt, gate, n, d, m):
    # the few-token path (me_kv_proj, then me_gate_rows) against the oracle and the fused kernel
    # on the same operands, with a keep mask and the row stats of the backward
    g = torch.Generator().manual_seed(n * 7 + d)
    hidden = (torch.randn(n, d, generator=g) * 3).to(hdt)
    mem = (torch.randn(n, m, generator=g) * 0.5).to(tdt)
    wk = (torch.randn(d, m, generator=g) * 0.05).to(tdt)
    wv = (torch.randn(d, m, generator=g) * 0.05).to(tdt)
    dq = (torch.randn(d, generator=g) * 0.1).to(tdt) if gate == 1 else None
    dk = (torch.randn(d, generator=g) * 0.1).to(tdt) if gate == 1 else None
    keep = torch.rand(n, generator=g) > 0.2
    dev = [t.to(DEV) if t is not None else None for t in (hidden, mem, wk, wv, dq, dk, keep)]
    with torch.no_grad():
        rows = ops.gate_residual_rows(*dev[:6], gate, dev[6], True, True)
        fused = ops.gate_residual(*dev[:6], gate, dev[6], True, True)
    ref, alpha_ref = oracle.inject(hidden.float() if hdt == torch.float32 else hidden, mem, wk, wv,
                                   ["scalar", "scalar_sqrt"][gate], dq, dk, keep=keep, return_alpha=True)
    assert_close_out(rows[0], ref, hidden, hdt if tdt == hdt else torch.bfloat16)
    tol = 1e-5 if (hdt, tdt) == (torch.float32, torch.float32) else 2e-3
    assert (rows[1].cpu() - alpha_ref.float()).abs().max() <= tol
    assert (rows[1] - fused[1]).abs().max() <= tol
    # row stats: sum x^2 exact up to summation order, the gate as returned
    assert torch.allclose(rows[2][:, 0], fused[2][:, 0], rtol=1e-5)
    assert torch.equal(rows[2][:, 3], rows[1])
    assert torch.equal(rows[0][~dev[6]], dev[0][~dev[6]])  # keep = False: unchanged


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,d,m", [(1, 64, 32), (5, 24, 40), (128, 520, 96), (129, 256, 8),
                                   (256, 5376, 1536), (300, 1024, 1024), (1000, 1024, 1024),
                                   (2048, 1024, 1024)])
def test_kv_proj_matches_fp32_reference(dtype, n, d, m):
    """me_kv_proj against torch's fp32 products of the same operands, rounded to the dtype:
    [K | V] = round(mem W_K^T | mem W_V^T). Tolerance: the sums run in another order, so after
    rounding an element may differ by one step of the dtype (bf16) or by 2e-6 of the sum of
    |products| (fp32). Shapes cover one and several token tiles, model dims that are not a
    multiple of 16 (the K / V boundary inside a 16-column block), mem dims that are not a
    multiple of the k-step, and the serving decode shape. Where the sum cancels to near zero a
    few fp32 roundings are many bf16 steps of the tiny result, hence the absolute term of 1e-6 of
    the sum of |products| (a bound on fp32 accumulation error over these lengths)."""
    g = torch.Generator().manual_seed(n + d + m)
    mem = (torch.randn(n, m, generator=g) * 0.5).to(dtype)
    wk = (torch.randn(d, m, generator=g) * 0.05).to(dtype)
    wv = (torch.randn(d, m, generator=g) * 0.05).to(dtype)
    got = ops.kv_proj(mem.to(DEV), wk.to(DEV), wv.to(DEV)).cpu()
    exact = torch.cat([mem.double() @ wk.double().T, mem.double() @ wv.double().T], dim=1)
    scale = torch.cat([mem.double().abs() @ wk.double().abs().T, mem.double().abs() @ wv.double().abs().T], 1)
    assert got.shape == (n, 2 * d) and got.dtype == dtype
    if dtype == torch.bfloat16:
        want = exact.to(torch.bfloat16)
        err = (got.double() - want.double()).abs()
        bound = _bf16_ulp(torch.maximum(got.abs().float(), want.abs().float())).double() + 1e-6 * scale
        assert bool((err <= bound).all()), float((err - bound).max())
        assert float((got != want).float().mean()) < 0.02
    else:
        assert bool(((got.double() - exact).abs() <= 2e-6 * scale + 1e-30).all())


def test_serving_decode_step_full():
    # the serving decode workload: 256 sequences x 1 token (0-3 history tokens, -1 = none) on the
    # Gemma-scale tables, hash_prev + inject as the vLLM layer calls them, against the oracle
    eng = synthetic.build_engram("gemma", DEV, seed=0).eval()
    ids, hidden = synthetic.decode_inputs(seed=2)
    with torch.no_grad():
        idx = eng.hash_prev(ids.to(DEV))
        out = eng.inject(hidden.to(DEV), idx)
    idx = torch.stack(idx)
    mem = torch.cat([t.weight[idx[k]] for k, t in enumerate(eng.tables)], dim=-1).cpu()
    ref = oracle.inject(hidden, mem, eng.key.weight.detach().cpu(), eng.value.weight.detach().cpu(),
                        "scalar_sqrt", eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu())
    assert_close_out(out, ref, hidden, torch.bfloat16)
    del eng
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_forward_after_optimizer_step_sees_new_weights(dtype):
    """A no-grad forward, a LazyAdamW step on the key / value weights (the optimizer writes
    through raw pointers), then a second forward: it must use the updated weights (both gate
    paths), and equal the oracle on them."""
    from micro_engram_fork_amd.optim import LazyAdamW

    torch.manual_seed(3)
    eng = _make(dtype, d=64, dim=8, heads=2)
    ids = torch.randint(5, 1000, (1, 40), device=DEV)
    hidden = torch.randn(1, 40, 64).to(dtype).to(DEV)
    with torch.no_grad():
        before = eng(hidden, ids)
    opt = LazyAdamW([eng.key.weight, eng.value.weight], lr=0.05, lazy=False, seed=1)
    eng.key.weight.grad = torch.randn_like(eng.key.weight)
    eng.value.weight.grad = torch.randn_like(eng.value.weight)
    opt.step()
    with torch.no_grad():
        after = eng(hidden, ids)
    assert not torch.equal(before, after)
    ref, _ = _oracle_forward(eng, hidden, ids)
    assert_close_out(after, ref.reshape(after.shape), hidden, dtype)
