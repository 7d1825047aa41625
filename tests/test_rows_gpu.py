"""Stage 4 on the GPU against the oracle: dedup bit-exact (unique keys, inverse, fp32 sums),
the squared norm, stochastic rounding and the sparse LazyAdamW step.

Tolerance of the Adam step: the GPU and the oracle draw identical rounding noise, so bf16
results are equal except where the fp32 value before rounding differs in its last bits (the
row mean of g^2 is summed in another order) and the noise sits right at the boundary: at most
1e-4 of the elements may differ, each by exactly one bf16 step; fp32 values within 2e-6
relative plus a few fp32 ulps of the pre-update magnitude; the row-wise second moment within
1e-6 relative. A bf16 element that an update cancels to near zero may differ by more steps,
within 2e-8 absolute (a few fp32 ulps of the ~0.02 operands).
"""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram, ops, rows as me_rows, synthetic
from micro_engram_fork_amd.optim import LazyAdamW, stochastic_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_dedup(keys, grads, key_bound):
    uniq, inv, gsum = me_rows.dedup_rows(keys.to(DEV), key_bound, None if grads is None else grads.to(DEV))
    g_np = grads.float().numpy() if grads is not None else np.zeros((keys.numel(), 1), np.float32)
    u, i, acc = oracle.dedup(keys.numpy(), g_np)
    assert np.array_equal(uniq.cpu().numpy(), u)
    assert np.array_equal(inv.cpu().numpy(), i)
    if grads is not None:
        assert np.array_equal(gsum.cpu().numpy().view(np.int32), acc.view(np.int32))


@pytest.mark.parametrize("n,bound,dim", [(1, 5, 4), (37, 3, 4), (2048, 100, 8), (2049, 100, 3),
                                         (10000, 1 << 20, 64), (5000, 1 << 40, 16)])
def test_dedup_bit_exact(n, bound, dim):
    g = torch.Generator().manual_seed(n)
    keys = torch.randint(0, bound, (n,), generator=g)
    if n > 100:
        keys[::3] = keys[0]  # one key repeated across blocks and passes
    grads = torch.randn(n, dim, generator=g) * torch.logspace(-4, 2, n).unsqueeze(1)
    _check_dedup(keys, grads, bound)


@pytest.mark.parametrize("case", ["all_equal", "clustered", "hot_keys", "large_random", "tiny"])
def test_dedup_bucket_paths_bit_exact(case):
    # keys that fit a bucket composite take the bucket dedup: buckets sorted in LDS, buckets too
    # large for LDS (repeats, or keys far denser than key_bound suggests) sorted in global
    # memory first; every case against the oracle's unique / inverse / ordered fp32 sums
    g = torch.Generator().manual_seed(7)
    if case == "all_equal":
        n, bound = 5000, 1000
        keys = torch.full((n,), 417, dtype=torch.long)
    elif case == "clustered":
        n, bound = 10000, 10**9
        keys = torch.randint(0, 3000, (n,), generator=g)
    elif case == "hot_keys":
        n, bound = 60000, 1 << 24
        keys = torch.randint(0, bound, (n,), generator=g)
        hot = torch.randint(0, bound, (5,), generator=g)
        keys[torch.randperm(n, generator=g)[:20000]] = hot[torch.randint(0, 5, (20000,), generator=g)]
    elif case == "large_random":
        n, bound = 300000, 79_691_776
        keys = torch.randint(0, bound, (n,), generator=g)
    else:
        n, bound = 3, 2
        keys = torch.tensor([1, 0, 1])
    grads = torch.randn(n, 16, generator=g) * torch.logspace(-3, 3, n).unsqueeze(1)
    _check_dedup(keys, grads, bound)


def test_dedup_bf16_grads_and_keys_only():
    g = torch.Generator().manual_seed(1)
    keys = torch.randint(0, 300, (4000,), generator=g)
    _check_dedup(keys, (torch.randn(4000, 32, generator=g)).bfloat16(), 300)
    _check_dedup(keys, None, 300)


def test_dedup_empty():
    uniq, inv, gsum = me_rows.dedup_rows(torch.zeros(0, dtype=torch.long, device=DEV), 10,
                                         torch.zeros(0, 4, device=DEV))
    assert uniq.numel() == 0 and inv.numel() == 0 and gsum.shape == (0, 4)


@pytest.mark.parametrize("n,bound,dim,dtype", [(196608, 79_691_776, 64, torch.float32),
                                               (5000, 1 << 40, 16, torch.float32),
                                               (4000, 300, 6, torch.bfloat16), (1, 5, 4, torch.float32)])
def test_dedup_split_halves_bit_exact(n, bound, dim, dtype):
    # the key half (unique keys, inverse, segment plan) run before the gradients exist, then the
    # sums from the plan: the same unique keys, inverse and fp32 sums as the oracle's one call;
    # bucket path (the workload's key range), radix path (40-bit keys), unaligned widths
    g = torch.Generator().manual_seed(n + dim)
    keys = torch.randint(0, bound, (n,), generator=g)
    if n > 100:
        keys[::5] = keys[1]
    grads = (torch.randn(n, dim, generator=g) * torch.logspace(-3, 2, n).unsqueeze(1)).to(dtype)
    uniq, inv, count, plan = ops.dedup_keys(keys.to(DEV), bound)
    gsum = ops.dedup_sums(plan, count, grads.to(DEV))
    c = int(count.item())
    u, i, acc = oracle.dedup(keys.numpy(), grads.float().numpy())
    assert c == len(u)
    assert np.array_equal(uniq[:c].cpu().numpy(), u)
    assert np.array_equal(inv.cpu().numpy(), i)
    assert np.array_equal(gsum[:c].cpu().numpy().view(np.int32), acc.view(np.int32))


def test_dedup_split_halves_empty():
    uniq, inv, count, plan = ops.dedup_keys(torch.zeros(0, dtype=torch.long, device=DEV), 10)
    gsum = ops.dedup_sums(plan, count, torch.zeros(0, 4, device=DEV))
    assert int(count.item()) == 0 and uniq.numel() == 0 and gsum.shape == (0, 4)


def test_add_sparse_grad_merges_like_reference():
    # rows.py:137-147: earlier entries first, then unique + index_add_
    p = torch.zeros(50, 8, device=DEV)
    g = torch.Generator().manual_seed(2)
    r1, g1 = torch.randint(0, 50, (30,), generator=g), torch.randn(30, 8, generator=g)
    r2, g2 = torch.randint(0, 50, (40,), generator=g), torch.randn(40, 8, generator=g)
    me_rows.add_sparse_grad(p, r1.to(DEV), g1.to(DEV))
    me_rows.add_sparse_grad(p, r2.to(DEV), g2.to(DEV))
    u1, _, a1 = oracle.dedup(r1.numpy(), g1.numpy())
    u, _, a = oracle.dedup(np.concatenate([u1, r2.numpy()]), np.concatenate([a1, g2.numpy()]))
    assert np.array_equal(p.sparse_grad[0].cpu().numpy(), u)
    assert np.array_equal(p.sparse_grad[1].cpu().numpy().view(np.int32), a.view(np.int32))


@pytest.mark.parametrize("n,skip", [(123457, 0), (5, 0), (12_000_003, 3)])
def test_sumsq(n, skip):
    # short, tiny and a clip-sized run starting off a 16-byte boundary; two calls agree bit for bit
    x = torch.randn(n + skip, device=DEV)[skip:]
    got = float(ops.sumsq(x))
    want = float((x.double() ** 2).sum())
    assert abs(got - want) <= 1e-5 * want
    assert float(ops.sumsq(x)) == got


def test_stochastic_bf16_matches_oracle_noise():
    x = torch.randn(10000) * 3
    seed, step, stream = 99, 4, 7
    got = stochastic_bf16(x.to(DEV), seed=seed, step=step, stream_id=stream).cpu()
    rows = np.arange(3)  # element i -> (row i // 4096, col i % 4096)
    noise = oracle.sr_noise(seed, step, stream, rows, 4096, 0).reshape(-1)[:10000]
    want = oracle.stochastic_bf16(x, torch.from_numpy(noise))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    special = torch.tensor([float("inf"), -float("inf"), 0.0, -0.0], device=DEV)
    assert torch.equal(stochastic_bf16(special, seed=1).float().cpu(), special.cpu())


def test_stochastic_bf16_unbiased():
    # test_optim.py:115-120
    for x in (1.00149, -1.00149):
        out = stochastic_bf16(torch.full((100_000,), x, device=DEV), seed=5).float()
        assert abs(float(out.mean()) - x) < 2e-5


def _adam_case(dtype, rowwise, R=300, D=64, n=120, steps=3, wd=0.0, sr=True, seed=123, lazy=True,
               zero_rows=True):
    g = torch.Generator().manual_seed(R + D)
    init = (torch.randn(R, D, generator=g) * 0.02).to(dtype)
    p_gpu = init.clone().to(DEV)
    m_gpu = torch.zeros_like(p_gpu)
    v_gpu = torch.zeros(R, device=DEV) if rowwise else torch.zeros_like(p_gpu)
    p_ref, m_ref = init.clone(), torch.zeros_like(init)
    v_ref = torch.zeros(R) if rowwise else torch.zeros_like(init)
    for step in range(1, steps + 1):
        rows = torch.randperm(R, generator=g)[:n].sort().values
        grads = torch.randn(n, D, generator=g) * 1e-3
        if zero_rows:
            grads[::7] = 0  # untouched rows inside the list
        ops.sparse_adam([p_gpu], [m_gpu], [v_gpu], [rows.to(DEV)], [grads.to(DEV)], [step], [3],
                        lr=5e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd, rowwise=rowwise,
                        lazy=lazy, stochastic_rounding=sr, seed=seed)

        def noise(r, which, step=step):
            return torch.from_numpy(oracle.sr_noise(seed, step, 3, r.numpy(), D, which))

        oracle.sparse_adam_step(p_ref, m_ref, v_ref, rows, grads, step, 5e-3, (0.9, 0.999), 1e-8, wd,
                                stochastic_rounding=sr, noise=noise)
    return (p_gpu.cpu(), m_gpu.cpu(), v_gpu.cpu()), (p_ref, m_ref, v_ref)


def _assert_bf16_close(got, want, frac=1e-4, atol=2e-8):
    # a result that an update cancels to ~1e-8 inherits the fp32 rounding of the ~0.02 operands
    # (ulp 2e-9), many bf16 steps at that magnitude: such elements pass on the absolute bound
    diff = got.view(torch.int16).int() - want.view(torch.int16).int()
    far = (diff.abs() > 1) & ((got.float() - want.float()).abs() > atol)
    assert not far.any(), f"{int(far.sum())} bf16 results differ by more than one step and {atol}"
    assert (diff != 0).float().mean() <= frac


@pytest.mark.parametrize("rowwise", [True, False])
@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_sparse_adam_bf16_matches_oracle(rowwise, wd):
    (p, m, v), (pr, mr, vr) = _adam_case(torch.bfloat16, rowwise, wd=wd)
    _assert_bf16_close(p, pr)
    _assert_bf16_close(m, mr)
    if rowwise:
        assert torch.allclose(v, vr, rtol=1e-6, atol=0)
    else:
        _assert_bf16_close(v, vr)


@pytest.mark.parametrize("D", [4, 8, 12, 128, 512])
@pytest.mark.parametrize("rowwise", [True, False])
def test_sparse_adam_kernel_shapes_match_oracle(D, rowwise):
    # 8 columns per lane (D = 8, 128, 512: 1, 16, 64 lanes per row), 4 per lane (D = 4), one
    # wave per row (D = 12)
    (p, m, v), (pr, mr, vr) = _adam_case(torch.bfloat16, rowwise, D=D, R=97, n=40)
    _assert_bf16_close(p, pr, frac=1e-2)
    _assert_bf16_close(m, mr, frac=1e-2)
    if rowwise:
        assert torch.allclose(v, vr, rtol=1e-6, atol=0)
    else:
        _assert_bf16_close(v, vr, frac=1e-2)


@pytest.mark.parametrize("D", [1024, 1536])
@pytest.mark.parametrize("rowwise", [True, False])
@pytest.mark.parametrize("lazy", [True, False])
def test_sparse_adam_wide_rows_match_oracle(D, rowwise, lazy):
    # rows wider than one 64-lane pass (the dense key / value weights: 1,536 columns), one wave
    # per row over 512-column blocks; lazy=False (the dense AdamW of the trainer) with every
    # listed row touched, as the oracle's lazy step then updates the same rows
    (p, m, v), (pr, mr, vr) = _adam_case(torch.bfloat16, rowwise, D=D, R=53, n=30, lazy=lazy,
                                         zero_rows=lazy)
    _assert_bf16_close(p, pr, frac=1e-2)
    _assert_bf16_close(m, mr, frac=1e-2)
    if rowwise:
        assert torch.allclose(v, vr, rtol=1e-6, atol=0)
    else:
        _assert_bf16_close(v, vr, frac=1e-2)


def _assert_fp32_close(got, want, rtol, atol):
    err = (got - want).abs() - rtol * want.abs()
    assert float(err.max()) <= atol, f"max excess {float(err.max()):.3e} over rtol {rtol} + atol {atol}"


def test_sparse_adam_fp32_matches_oracle():
    # weights ~0.02 carry an fp32 rounding of ulp(0.05) ~ 4e-9 per step; one that an update
    # cancels toward zero keeps that as absolute error, hence atol = 3 steps x 4 ulps of 0.05
    (p, m, v), (pr, mr, vr) = _adam_case(torch.float32, True, sr=True)
    _assert_fp32_close(p, pr, 2e-6, 5e-8)
    _assert_fp32_close(m, mr, 2e-6, 1e-10)  # m ~1e-4: a few ulps of 1e-4
    _assert_fp32_close(v, vr, 1e-6, 0.0)


def test_lazy_adamw_api_and_invariants():
    # test_optim.py:56-88 through the optimizer class: state names, untouched rows exact
    torch.manual_seed(0)
    R, C = 16, 8
    init = torch.randn(R, C)
    p = torch.nn.Parameter(init.clone().to(DEV))
    opt = LazyAdamW([p], lr=1e-2, lazy=True, rowwise=True, seed=1)
    for i in range(5):
        gr = torch.randn(R, C)
        gr[4:] = 0
        if i > 0:
            gr[0] = 0
        p.grad = gr.to(DEV)
        opt.step()
    st = opt.state[p]
    assert set(st) == {"step", "exp_avg", "exp_avg_sq"} and float(st["step"]) == 5
    assert st["exp_avg_sq"].shape == (R,) and st["exp_avg_sq"].dtype == torch.float32
    assert torch.equal(p.detach()[4:].cpu(), init[4:])
    assert torch.equal(st["exp_avg"][4:].cpu(), torch.zeros(R - 4, C))


def test_rowwise_equals_adamw_uniform_rows():
    # test_optim.py:74-80 through LazyAdamW (non-lazy rowwise, fp32)
    torch.manual_seed(1)
    R, C = 16, 8
    init = torch.randn(R, C)
    row_scale = torch.rand(R, 1) + 0.5
    grads = [row_scale * torch.sign(torch.randn(R, C)) * (i + 1) for i in range(5)]
    a = torch.nn.Parameter(init.clone())
    ta = torch.optim.AdamW([a], lr=1e-2, weight_decay=0.1, foreach=False)
    b = torch.nn.Parameter(init.clone().to(DEV))
    tb = LazyAdamW([b], lr=1e-2, weight_decay=0.1, lazy=False, rowwise=True)
    for gr in grads:
        a.grad, b.grad = gr.clone(), gr.clone().to(DEV)
        ta.step()
        tb.step()
    assert torch.allclose(a.detach(), b.detach().cpu(), atol=1e-6)


def test_bf16_stochastic_rounding_tracks_fp32():
    # test_optim.py:121-136: at a low learning rate bf16 + SR moves like fp32, plain rounding not
    moved = {}
    for name, dtype, sr in (("fp32", torch.float32, True), ("plain", torch.bfloat16, False),
                            ("sr", torch.bfloat16, True)):
        w = torch.nn.Parameter(torch.full((2000, 8), 0.03, dtype=dtype, device=DEV))
        opt = LazyAdamW([{"params": [w], "lazy": True, "rowwise": True}], lr=2.5e-5, stochastic_rounding=sr,
                        seed=7)
        for _ in range(300):
            w.grad = torch.ones_like(w)
            opt.step()
        moved[name] = float((0.03 - w.float()).mean())
    assert abs(moved["plain"] / moved["fp32"] - 1) > 0.2
    assert abs(moved["sr"] / moved["fp32"] - 1) < 0.03


def test_row_lookup_two_backwards_accumulate():
    # gradient accumulation: each backward sums its own duplicate lookups first (rows.py:117-118),
    # the first leaves each table's part as its sparse gradient and the second merges its part
    # into it like add_sparse_grad (rows.py:125-129, 137-147)
    eng = MicroEngram(model_dim=16, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3),
                      vocab_size=500, seed=4)
    shards = eng.shard_rows(0, 1, device=DEV)
    for s in shards:
        s._sparse_rows = True
    passes = []
    for _ in range(2):
        ids = torch.randint(0, 500, (2, 40), device=DEV)
        idx = eng.hash_ids(ids)
        out = me_rows.row_lookup(eng, idx)
        grads = [torch.randn_like(o) for o in out]
        torch.autograd.backward(out, grads)
        passes.append((idx, grads))
    for k, s in enumerate(shards):
        (i1, g1), (i2, g2) = passes[0], passes[1]
        u1, _, a1 = oracle.dedup(i1[k].reshape(-1).cpu().numpy(), g1[k].reshape(-1, 8).cpu().numpy())
        u2, _, a2 = oracle.dedup(i2[k].reshape(-1).cpu().numpy(), g2[k].reshape(-1, 8).cpu().numpy())
        u, _, acc = oracle.dedup(np.concatenate([u1, u2]), np.concatenate([a1, a2]))
        assert np.array_equal(s.sparse_grad[0].cpu().numpy(), u)
        assert np.array_equal(s.sparse_grad[1].cpu().numpy().view(np.int32), acc.view(np.int32))


def test_row_lookup_backward_sparse_grads():
    eng = MicroEngram(model_dim=16, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3),
                      vocab_size=500, seed=3)
    shards = eng.shard_rows(0, 1, device=DEV)
    for s in shards:
        s._sparse_rows = True
    ids = torch.randint(0, 500, (2, 40), device=DEV)
    idx = eng.hash_ids(ids)
    out = me_rows.row_lookup(eng, idx)
    grads = [torch.randn_like(o) for o in out]
    torch.autograd.backward(out, grads)
    for k, s in enumerate(shards):
        u, _, acc = oracle.dedup(idx[k].reshape(-1).cpu().numpy(), grads[k].reshape(-1, 8).cpu().numpy())
        assert np.array_equal(s.sparse_grad[0].cpu().numpy(), u)
        assert np.array_equal(s.sparse_grad[1].cpu().numpy().view(np.int32), acc.view(np.int32))


def test_row_lookup_retained_graph_second_backward():
    # the first backward uses the forward's key plan, a second one over the retained graph runs
    # the whole dedup again and merges into the sparse gradient (rows.py:125-129, 137-147)
    eng = MicroEngram(model_dim=16, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3),
                      vocab_size=500, seed=5)
    shards = eng.shard_rows(0, 1, device=DEV)
    for s in shards:
        s._sparse_rows = True
    ids = torch.randint(0, 500, (2, 40), device=DEV)
    idx = eng.hash_ids(ids)
    out = me_rows.row_lookup(eng, idx)
    grads = [torch.randn_like(o) for o in out]
    torch.autograd.backward(out, grads, retain_graph=True)
    torch.autograd.backward(out, grads)
    for k, s in enumerate(shards):
        u1, _, a1 = oracle.dedup(idx[k].reshape(-1).cpu().numpy(), grads[k].reshape(-1, 8).cpu().numpy())
        u, _, acc = oracle.dedup(np.concatenate([u1, u1]), np.concatenate([a1, a1]))
        assert np.array_equal(s.sparse_grad[0].cpu().numpy(), u)
        assert np.array_equal(s.sparse_grad[1].cpu().numpy().view(np.int32), acc.view(np.int32))


def test_key_plan_after_gate_matches_plan_at_lookup():
    # inject with gradients issues the dedup's key plan after the gate (key_plans_after); the
    # same lookup outside that block makes it at once: same sparse gradients, bit for bit, and
    # equal to the oracle's dedup of the ids with the memory gradient
    eng = MicroEngram(model_dim=32, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3),
                      vocab_size=500, seed=6).to(DEV)
    shards = eng.shard_rows(0, 1, device=DEV)
    for s in shards:
        s._sparse_rows = True
    ids = torch.randint(0, 500, (2, 48), device=DEV)
    idx = eng.hash_ids(ids)
    hidden = torch.randn(2, 48, 32, device=DEV)
    gout = torch.randn(2, 48, 32, device=DEV)
    got = []
    for deferred in (True, False):
        for s in shards:
            s.sparse_grad = None
        h = hidden.clone().requires_grad_(True)
        if deferred:
            out = eng.inject(h, idx)
        else:
            mem = eng._mem_grad(idx)
            mem.retain_grad()
            out = eng._gate(h, mem, None)
        out.backward(gout)
        got.append([(s.sparse_grad[0].clone(), s.sparse_grad[1].clone()) for s in shards])
    for (ua, ga), (ub, gb) in zip(*got):
        assert torch.equal(ua, ub)
        assert torch.equal(ga.view(torch.int32), gb.view(torch.int32))
    D = 8
    for k, s in enumerate(shards):
        g = mem.grad[:, k * D:(k + 1) * D].cpu().numpy()
        u, _, acc = oracle.dedup(idx[k].reshape(-1).cpu().numpy(), g)
        assert np.array_equal(got[1][k][0].cpu().numpy(), u)
        assert np.array_equal(got[1][k][1].cpu().numpy().view(np.int32), acc.view(np.int32))


def test_two_chained_engrams_one_backward():
    # two engrams in one graph (the second reads the first's output): each forward leaves its
    # key plan and its tables' bounds (copied to host memory behind an event) after its gate,
    # and the one backward reads both, the second engram's first; the sparse gradients equal
    # those of the same graph with the plans made at the lookups, and the oracle's dedup of
    # each memory gradient
    engs = [MicroEngram(model_dim=32, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3),
                        vocab_size=500, seed=s).to(DEV) for s in (7, 8)]
    shards = [e.shard_rows(0, 1, device=DEV) for e in engs]
    for sh in shards:
        for s in sh:
            s._sparse_rows = True
    ids = torch.randint(0, 500, (2, 48), device=DEV)
    idxs = [e.hash_ids(ids) for e in engs]
    hidden = torch.randn(2, 48, 32, device=DEV)
    gout = torch.randn(2, 48, 32, device=DEV)
    got = []
    for deferred in (True, False):
        for sh in shards:
            for s in sh:
                s.sparse_grad = None
        x = hidden.clone().requires_grad_(True)
        mems = []
        for e, idx in zip(engs, idxs):
            if deferred:
                x = e.inject(x, idx)
            else:
                mem = e._mem_grad(idx)
                mem.retain_grad()
                mems.append(mem)
                x = e._gate(x, mem, None)
        x.backward(gout)
        got.append([[(s.sparse_grad[0].clone(), s.sparse_grad[1].clone()) for s in sh] for sh in shards])
    D = 8
    for e_i, (sh, mem) in enumerate(zip(shards, mems)):
        for k in range(len(sh)):
            (ua, ga), (ub, gb) = got[0][e_i][k], got[1][e_i][k]
            assert torch.equal(ua, ub) and torch.equal(ga.view(torch.int32), gb.view(torch.int32))
            u, _, acc = oracle.dedup(idxs[e_i][k].reshape(-1).cpu().numpy(),
                                     mem.grad[:, k * D:(k + 1) * D].cpu().numpy())
            assert np.array_equal(ub.cpu().numpy(), u)
            assert np.array_equal(gb.cpu().numpy().view(np.int32), acc.view(np.int32))


def _clip_engram(dtype, sparse):
    eng = MicroEngram(model_dim=16, table_size=64, engram_dim=8, num_heads=2, orders=(2,), vocab_size=50,
                      seed=4)
    shards = eng.shard_rows(0, 1, device=DEV, dtype=dtype)
    rt = me_rows.RowTables([("x.", eng)], lr=5e-3, lazy=True, rowwise=True, sparse_grads=sparse,
                           stochastic_rounding=True, seed=77)
    return eng, shards, rt


def _oracle_step(init, rows, g, step, table, seed=77):
    p_ref = init.clone()
    m_ref = torch.zeros_like(p_ref)
    v_ref = torch.zeros(p_ref.shape[0])

    def noise(r, which):
        return torch.from_numpy(oracle.sr_noise(seed, step, table, r.numpy(), init.shape[1], which))

    oracle.sparse_adam_step(p_ref, m_ref, v_ref, rows, g, step, 5e-3, stochastic_rounding=True, noise=noise)
    return p_ref, m_ref, v_ref


def test_row_tables_clip_sparse_in_place_then_step():
    """RowTables.clip with coef < 1 (rows.py:208-233): the fp32 sparse sums are scaled in place
    by the fp32 coefficient -- bit-equal to the oracle's scaling given the same norm, the norm
    itself within 1e-6 of the oracle's (another summation order) -- and the next step equals the
    oracle's clip followed by sparse_adam_step with the same rounding noise."""
    eng, shards, rt = _clip_engram(torch.bfloat16, sparse=True)
    init = [s.detach().cpu().clone() for s in shards]
    g = torch.Generator().manual_seed(11)
    rows = [torch.tensor([1, 5, 9, 40]), torch.tensor([0, 2, 63])]
    sums = [torch.randn(r.numel(), 8, generator=g) * 2.0 for r in rows]
    for s, r, x in zip(shards, rows, sums):
        me_rows.add_sparse_grad(s, r.to(DEV), x.to(DEV))
    norm = rt.clip(1.0)
    ref_sums = [x.clone() for x in sums]
    ref_norm = oracle.clip(ref_sums, 1.0)
    assert norm == pytest.approx(ref_norm, rel=1e-6) and norm > 1.0
    coef = oracle.clip_coef(norm, 1.0)  # the coefficient of the GPU's own norm
    for s, x in zip(shards, sums):
        assert np.array_equal(s.sparse_grad[1].cpu().numpy().view(np.int32), (x * coef).numpy().view(np.int32))
    scaled = [s.sparse_grad[1].cpu().clone() for s in shards]
    rt.step(5e-3)
    for k, s in enumerate(shards):
        p_ref, m_ref, v_ref = _oracle_step(init[k], rows[k], scaled[k], 1, k)
        st = rt.optimizer.state[s]
        _assert_bf16_close(s.detach().cpu(), p_ref)
        _assert_bf16_close(st["exp_avg"].cpu(), m_ref)
        assert torch.allclose(st["exp_avg_sq"].cpu(), v_ref, rtol=1e-6, atol=0)
        assert s.sparse_grad is None


def test_row_tables_clip_dense_bf16_in_place_then_step():
    """Dense bf16 table gradients: p.grad.mul_(coef.to(bf16)) in place, bit-equal to the
    oracle's given the same norm; then the lazy step over every row (all-zero rows skipped)."""
    eng, shards, rt = _clip_engram(torch.bfloat16, sparse=False)
    init = [s.detach().cpu().clone() for s in shards]
    g = torch.Generator().manual_seed(12)
    grads = []
    for s in shards:
        x = torch.zeros(s.shape)
        x[torch.randperm(s.shape[0], generator=g)[:10]] = torch.randn(10, 8, generator=g) * 3.0
        grads.append(x.bfloat16())
        s.grad = grads[-1].to(DEV)
    norm = rt.clip(0.5)
    ref = [x.clone() for x in grads]
    ref_norm = oracle.clip(ref, 0.5)
    assert norm == pytest.approx(ref_norm, rel=1e-6) and norm > 0.5
    coef = oracle.clip_coef(norm, 0.5).to(torch.bfloat16)
    for s, x in zip(shards, grads):
        want = (x * coef)  # bf16 * bf16: fp32 product rounded to bf16
        assert torch.equal(s.grad.cpu().view(torch.int16), want.view(torch.int16))
    scaled = [s.grad.cpu().float() for s in shards]
    rt.step(5e-3)
    for k, s in enumerate(shards):
        p_ref, m_ref, v_ref = _oracle_step(init[k], torch.arange(s.shape[0]), scaled[k], 1, k)
        _assert_bf16_close(s.detach().cpu(), p_ref)


def test_row_tables_clip_then_zero_grad_leaves_nothing():
    """A clip without a step, then zero_grad: the next step sees only its own gradients."""
    eng, shards, rt = _clip_engram(torch.bfloat16, sparse=True)
    init = [s.detach().cpu().clone() for s in shards]
    me_rows.add_sparse_grad(shards[0], torch.tensor([3], device=DEV), torch.full((1, 8), 50.0, device=DEV))
    rt.clip(1e-3)
    rt.zero_grad()
    assert all(s.sparse_grad is None for s in shards)
    x = torch.full((1, 8), 1e-3)
    me_rows.add_sparse_grad(shards[1], torch.tensor([7], device=DEV), x.to(DEV))
    rt.step(5e-3)
    assert torch.equal(shards[0].detach().cpu(), init[0])  # untouched
    p_ref, _, _ = _oracle_step(init[1], torch.tensor([7]), x, 1, 1)
    _assert_bf16_close(shards[1].detach().cpu(), p_ref)


# ------------------------------------------------------------ the sparse-update workload
def test_sparse_update_workload():
    """The Gemma prefill batch's 196,608 (table, row) lookups with fp32 gradients N(0, 1e-3):
    dedup bit-exact, then one row-wise Adam step (lr 5e-3, betas 0.9/0.999, eps 1e-8) on the
    bf16 tables with stochastic rounding, against the oracle drawing the same noise."""
    eng = synthetic.build_engram("gemma", DEV, seed=0)
    ids, pos, _ = synthetic.prefill_inputs(seed=0, device=DEV)
    idx = torch.stack(eng.hash_ids(ids, pos)).reshape(len(eng.tables), -1)
    offs = [0]
    for r in eng.table_rows:
        offs.append(offs[-1] + r)
    keys = (idx + torch.tensor(offs[:-1], device=DEV)[:, None]).t().reshape(-1)
    grads = synthetic.lookup_grads(keys.numel(), eng.engram_dim, seed=0, device=DEV)
    uniq, inv, gsum = me_rows.dedup_rows(keys, offs[-1], grads)
    u, i, acc = oracle.dedup(keys.cpu().numpy(), grads.cpu().numpy())
    assert np.array_equal(uniq.cpu().numpy(), u) and np.array_equal(inv.cpu().numpy(), i)
    assert np.array_equal(gsum.cpu().numpy().view(np.int32), acc.view(np.int32))

    bounds = np.searchsorted(u, np.array(offs))
    tables = [t.weight for t in eng.tables]
    before = [t.detach()[torch.from_numpy(u[bounds[k]:bounds[k + 1]] - offs[k]).to(DEV)].cpu()
              for k, t in enumerate(tables)]
    opt = LazyAdamW([{"params": tables, "lazy": True, "rowwise": True}], lr=5e-3, seed=2024)
    for k, t in enumerate(tables):
        t.sparse_grad = (uniq[bounds[k]:bounds[k + 1]] - offs[k], gsum[bounds[k]:bounds[k + 1]])
    opt.step()
    for k, t in enumerate(tables):
        rows = torch.from_numpy(u[bounds[k]:bounds[k + 1]] - offs[k])
        p_ref = before[k].clone()
        m_ref = torch.zeros_like(p_ref)
        v_ref = torch.zeros(rows.numel())

        def noise(r, which, rows=rows, k=k):
            return torch.from_numpy(oracle.sr_noise(2024, 1, k, rows[r].numpy(), 64, which))

        oracle.sparse_adam_step(p_ref, m_ref, v_ref, torch.arange(rows.numel()),
                                torch.from_numpy(acc[bounds[k]:bounds[k + 1]]), 1, 5e-3,
                                stochastic_rounding=True, noise=noise)
        got = t.detach()[rows.to(DEV)].cpu()
        _assert_bf16_close(got, p_ref)
        _assert_bf16_close(opt.state[t]["exp_avg"][rows.to(DEV)].cpu(), m_ref)
        assert torch.allclose(opt.state[t]["exp_avg_sq"][rows.to(DEV)].cpu(), v_ref, rtol=1e-6, atol=0)
    del eng, opt
    torch.cuda.empty_cache()


def test_bf16_second_moment_freeze_vs_stochastic_rounding():
    # test_optim.py:92-110 through LazyAdamW on the GPU
    torch.manual_seed(0)
    init = torch.randn(16, 8).bfloat16()
    out = {}
    for name, kw in (("plain", dict(stochastic_rounding=False)), ("sr", {}), ("rowwise", dict(rowwise=True))):
        p = torch.nn.Parameter(init.clone().to(DEV))
        opt = LazyAdamW([p], lr=0.0, seed=3, **kw)
        for _ in range(1500):
            p.grad = torch.ones_like(p)
            opt.step()
        out[name] = float(opt.state[p]["exp_avg_sq"].float().mean()) / (1 - 0.999 ** 1500)
    assert out["plain"] < 0.5 and abs(out["sr"] - 1) < 0.02 and abs(out["rowwise"] - 1) < 1e-4


@pytest.mark.parametrize("case", ["random", "empty_tables", "zero_count", "boundaries"])
def test_dedup_table_bounds(case):
    # the one-launch bounds against numpy's searchsorted over the unique keys (rows.py:123-129):
    # every unique key's local row and each table's first index, with empty tables, a count
    # below the array length and keys right at the table boundaries
    g = torch.Generator().manual_seed(len(case))
    sizes = [97, 0, 5, 1 << 20, 3, 0, 1000] if case == "empty_tables" else [131, 257, 97, 4099]
    offs = [0]
    for r in sizes:
        offs.append(offs[-1] + r)
    if case == "boundaries":
        keys = torch.tensor(sorted(set(offs[:-1]) | {o - 1 for o in offs[1:]}), dtype=torch.int64)
    else:
        keys = torch.unique(torch.randint(0, offs[-1], (600,), generator=g))
    n = keys.numel() + 7  # slots past the count, as the dedup output has
    uniq = torch.full((n,), -5, dtype=torch.int64)
    uniq[:keys.numel()] = keys
    cnt = 0 if case == "zero_count" else keys.numel()
    local, info = ops.dedup_table_bounds(uniq.to(DEV), torch.tensor([cnt], device=DEV), offs)
    valid = uniq[:cnt].numpy()
    want_bounds = np.searchsorted(valid, np.array(offs), side="left")
    assert info.cpu().tolist() == [cnt] + want_bounds.tolist()
    tbl = np.searchsorted(np.array(offs[:-1]), valid, side="right") - 1
    assert np.array_equal(local.cpu().numpy()[:cnt], valid - np.array(offs)[tbl])


def test_training_step_fast_paths_equal_the_general_ones():
    # the clip and the optimizer address a backward's per-table sparse gradients through the
    # buffers they are slices of (SparseBatch); with that link removed they take the general
    # per-table paths. Two identical engrams, three training steps each (norms, tables, both
    # moments, step counters): bit for bit. The third step of the general run also reloads the
    # optimizer state, so the shared step-counter buffer is re-adopted from loaded tensors.
    def run(general):
        torch.manual_seed(3)  # the dense tables' init draws from the global generator
        eng = MicroEngram(model_dim=64, table_size=211, engram_dim=8, num_heads=2, orders=(2, 3, 4),
                          vocab_size=1000, gate="scalar_sqrt", seed=3)
        synthetic.fill_dense(eng, seed=3, std=0.2)
        eng = eng.to(DEV)
        eng.shard_rows(0, 1, device=DEV, dtype=torch.bfloat16)
        rt = me_rows.RowTables([("e.", eng)], lr=5e-3, lazy=True, rowwise=True, sparse_grads=True, seed=11)
        gen = torch.Generator().manual_seed(4)
        norms = []
        for k in range(3):
            ids = torch.randint(0, 40, (2, 60), generator=gen).to(DEV)
            h = torch.randn(2, 60, 64, generator=gen).to(DEV).requires_grad_(True)
            eng(h, ids).backward(torch.randn(2, 60, 64, generator=gen).to(DEV))
            if general:
                for p in eng.row_shards:
                    p.__dict__.pop("_sparse_batch", None)
                if k == 2:
                    rt.optimizer.load_state_dict(rt.optimizer.state_dict())
            norms.append(rt.clip(0.05))
            rt.step(5e-3)
        st = rt.optimizer.state
        return norms, [(p.detach().clone(), st[p]["exp_avg"].clone(), st[p]["exp_avg_sq"].clone(),
                        float(st[p]["step"])) for p in eng.row_shards]

    fast_norms, fast = run(False)
    gen_norms, general = run(True)
    assert fast_norms == gen_norms
    for (p1, m1, v1, s1), (p2, m2, v2, s2) in zip(fast, general):
        assert torch.equal(p1, p2) and torch.equal(m1, m2) and torch.equal(v1, v2) and s1 == s2 == 3.0


@pytest.mark.parametrize("D,rowwise,lazy", [(1536, False, False), (1536, True, True), (64, True, True),
                                            (64, False, False), (12, False, True), (3, True, False)])
def test_sparse_adam_reads_bf16_gradients_as_their_fp32_values(D, rowwise, lazy):
    # bf16 gradient rows (the dense weights' autograd gradients) go to the kernel as they are:
    # the update equals the one from their fp32 copies bit for bit, on the wide (1536 columns),
    # vector (64, 12) and generic (3) kernels
    g = torch.Generator().manual_seed(D)
    R, n = 200, 90
    init = (torch.randn(R, D, generator=g) * 0.02).bfloat16().to(DEV)
    rows = torch.randperm(R, generator=g)[:n].sort().values.to(DEV)
    grads = (torch.randn(n, D, generator=g) * 1e-3).bfloat16().to(DEV)
    grads[::5] = 0
    outs = []
    for gr in (grads, grads.float()):
        p, m = init.clone(), (init * 0.1).clone()
        v = torch.full((R,), 1e-6, device=DEV) if rowwise else (init.float() ** 2).bfloat16()
        for step in (1, 2):
            ops.sparse_adam([p], [m], [v], [rows], [gr], [step], [5], lr=5e-3, betas=(0.9, 0.999),
                            eps=1e-8, weight_decay=0.01, rowwise=rowwise, lazy=lazy,
                            stochastic_rounding=True, seed=77)
        outs.append((p, m, v))
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
