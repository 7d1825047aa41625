"""Pins the oracle's training half (dedup, Philox, stochastic rounding, the sparse LazyAdamW
step) against known answers, brute force and torch.optim.AdamW (test_optim.py:38-139 cases)."""
import os

import numpy as np
import pytest
import torch

import oracle


# ---------------------------------------------------------------------------------- Philox
@pytest.mark.parametrize("ctr,key,want", [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_known_answers(ctr, key, want):
    # Random123 known-answer vectors for philox4x32_10
    got = oracle.philox4x32_10(np.array([ctr], np.uint32), np.array([key], np.uint32))[0]
    assert tuple(int(x) for x in got) == want


def test_sr_noise_layout():
    # element (row, col) takes half (col & 1) of word (col >> 1) & 3 of the call for col >> 3
    seed, step, table = 12345, 7, 3
    rows = np.array([0, 5, 2**33 + 1])
    n = oracle.sr_noise(seed, step, table, rows, 16, 1)
    for r_i, row in enumerate(rows):
        for col in range(16):
            ctr = np.array([[row & 0xffffffff, row >> 32, step, (table << 16) | (1 << 14) | (col >> 3)]], np.uint32)
            key = np.array([[seed & 0xffffffff, seed >> 32]], np.uint32)
            w = oracle.philox4x32_10(ctr, key)[0][(col >> 1) & 3]
            assert n[r_i, col] == (int(w) >> (16 * (col & 1))) & 0xffff


# ----------------------------------------------------------------------- stochastic rounding
def test_stochastic_bf16_exhaustive_counts():
    # over all 2^16 noise values, x rounds up exactly (low 16 bits of x) times: P(up) = dropped part
    for x in (1.00149, -1.00149, 0.03, -3.0e-3, 1.0, 123.456, 2.0 ** -120):
        xs = torch.full((65536,), x, dtype=torch.float32)
        noise = torch.arange(65536, dtype=torch.int32)
        out = oracle.stochastic_bf16(xs, noise).float()
        bits = int(torch.tensor([x], dtype=torch.float32).view(torch.int32)) & 0xFFFF
        trunc = (torch.tensor([x], dtype=torch.float32).view(torch.int32) & -65536).view(torch.float32)
        ups = int((out.abs() > trunc.abs()).sum())
        assert ups == bits
        assert set(out.unique().tolist()) <= {float(trunc), float(out.max() if x > 0 else out.min())}


def test_stochastic_bf16_unbiased_and_special_values():
    # test_optim.py:112-120: the mean of many roundings is the value; inf kept
    rng = np.random.Generator(np.random.PCG64(0))
    for x in (1.00149, -1.00149):
        xs = torch.full((100_000,), x)
        noise = torch.from_numpy(rng.integers(0, 65536, 100_000).astype(np.int32))
        assert abs(float(oracle.stochastic_bf16(xs, noise).float().mean()) - x) < 2e-5
    inf = oracle.stochastic_bf16(torch.tensor([float("inf"), -float("inf")]), torch.tensor([65535, 65535]))
    assert torch.isinf(inf.float()).all()
    assert torch.isnan(oracle.stochastic_bf16(torch.tensor([float("nan")]), torch.tensor([7])).float()).all()


# ------------------------------------------------------------------------------------ dedup
def _dedup_brute(keys, grads):
    uniq = sorted(set(int(k) for k in keys))
    pos = {k: i for i, k in enumerate(uniq)}
    acc = np.zeros((len(uniq),) + grads.shape[1:], np.float32)
    inv = np.empty(len(keys), np.int64)
    for i, k in enumerate(keys):  # index order, fp32 adds from +0.0
        inv[i] = pos[int(k)]
        acc[pos[int(k)]] = (acc[pos[int(k)]] + grads[i]).astype(np.float32)
    return np.array(uniq, np.int64), inv, acc


@pytest.mark.parametrize("seed", range(4))
def test_dedup_equals_bruteforce(seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    keys = rng.integers(0, 30, size=200) * rng.integers(1, 1000)
    grads = (rng.standard_normal((200, 5)) * 10 ** rng.uniform(-4, 2, size=(200, 1))).astype(np.float32)
    u, inv, acc = oracle.dedup(keys, grads)
    bu, binv, bacc = _dedup_brute(keys, grads)
    assert np.array_equal(u, bu) and np.array_equal(inv, binv)
    assert np.array_equal(acc.view(np.int32), bacc.view(np.int32))  # bit-exact
    assert np.array_equal(u[inv], keys)


def test_dedup_matches_torch_unique_index_add():
    # the reference's own library routines (rows.py:81, 117-118) on the CPU
    rng = np.random.Generator(np.random.PCG64(11))
    keys = torch.from_numpy(rng.integers(0, 500, size=3000))
    grads = torch.from_numpy(rng.standard_normal((3000, 8)).astype(np.float32))
    uniq, inv = torch.unique(keys, return_inverse=True)
    acc = torch.zeros(uniq.numel(), 8).index_add_(0, inv, grads)
    u, i, a = oracle.dedup(keys.numpy(), grads.numpy())
    assert np.array_equal(u, uniq.numpy()) and np.array_equal(i, inv.numpy())
    assert np.array_equal(a.view(np.int32), acc.numpy().view(np.int32))


@pytest.mark.parametrize("seed", range(3))
def test_dedup_torch_equals_bruteforce(seed):
    # the sparse-update baseline's torch-op dedup: the brute force's unique keys, inverse and
    # fp32 sums bit for bit
    rng = np.random.Generator(np.random.PCG64(40 + seed))
    keys = rng.integers(0, 40, size=300) * rng.integers(1, 5000)
    grads = (rng.standard_normal((300, 6)) * 10 ** rng.uniform(-4, 2, size=(300, 1))).astype(np.float32)
    u, inv, acc = oracle.dedup_torch(keys, grads)
    bu, binv, bacc = _dedup_brute(keys, grads)
    assert np.array_equal(u.numpy(), bu) and np.array_equal(inv.numpy(), binv)
    assert np.array_equal(acc.numpy().view(np.int32), bacc.view(np.int32))


def test_dedup_golden_fixture():
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "dedup_small.npz"))
    u, inv, acc = oracle.dedup(f["keys"], f["grads"])
    assert np.array_equal(u, f["uniq"]) and np.array_equal(inv, f["inv"])
    assert np.array_equal(acc.view(np.int32), f["acc"].view(np.int32))


# ------------------------------------------------------------------------ sparse LazyAdamW
def _run_oracle(init, grads, rowwise, wd=0.0, lr=1e-2, dtype=torch.float32, sr=False, seed=0):
    p = init.clone().to(dtype)
    m = torch.zeros_like(p)
    v = torch.zeros(p.shape[0]) if rowwise else torch.zeros_like(p)
    for step, g in enumerate(grads, start=1):
        rows = torch.arange(p.shape[0])

        def noise(r, which, step=step):
            return torch.from_numpy(oracle.sr_noise(seed, step, 0, r.numpy(), p.shape[1], which))

        oracle.sparse_adam_step(p, m, v, rows, g.clone(), step, lr, (0.9, 0.999), 1e-8, wd,
                                stochastic_rounding=sr, noise=noise)
    return p.float(), m, v


def test_sparse_step_equals_adamw_when_rows_uniform():
    # test_optim.py:74-80: with |g| equal across each row, the row mean of g^2 is every value's g^2
    torch.manual_seed(0)
    R, C = 16, 8
    init = torch.randn(R, C)
    row_scale = torch.rand(R, 1) + 0.5
    grads = [row_scale * torch.sign(torch.randn(R, C)) * (i + 1) for i in range(5)]
    for wd in (0.0, 0.1):
        p = torch.nn.Parameter(init.clone())
        opt = torch.optim.AdamW([p], lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd, foreach=False)
        for g in grads:
            p.grad = g.clone()
            opt.step()
        got, _, _ = _run_oracle(init, grads, rowwise=True, wd=wd)
        assert torch.allclose(got, p.detach(), atol=1e-6)


def test_sparse_step_per_value_equals_adamw():
    # per-value second moment, every row touched every step: plain AdamW (test_optim.py:38-42)
    torch.manual_seed(1)
    init = torch.randn(10, 6)
    grads = [torch.randn(10, 6) for _ in range(4)]
    p = torch.nn.Parameter(init.clone())
    opt = torch.optim.AdamW([p], lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, foreach=False)
    for g in grads:
        p.grad = g.clone()
        opt.step()
    got, _, _ = _run_oracle(init, grads, rowwise=False)
    assert torch.allclose(got, p.detach(), atol=1e-6)


def test_sparse_step_lazy_invariants():
    # test_optim.py:56-65, 84-88: rows with an all-zero gradient keep weights and both moments
    torch.manual_seed(2)
    init = torch.randn(8, 4)
    p, m, v = init.clone(), torch.zeros(8, 4), torch.zeros(8)
    g = torch.randn(8, 4)
    g[5:] = 0
    oracle.sparse_adam_step(p, m, v, torch.arange(8), g, 1, 1e-2, stochastic_rounding=False)
    assert torch.equal(p[5:], init[5:]) and torch.equal(v[5:], torch.zeros(3))
    assert torch.equal(m[5:], torch.zeros(3, 4)) and not torch.equal(p[:5], init[:5])


def test_sparse_step_fp32_ignores_rounding_flag():
    # test_optim.py:137-139: fp32 tables are bit-identical with and without stochastic rounding
    torch.manual_seed(3)
    init = torch.randn(6, 4)
    grads = [torch.randn(6, 4) for _ in range(3)]
    a, _, _ = _run_oracle(init, grads, rowwise=True, sr=True)
    b, _, _ = _run_oracle(init, grads, rowwise=True, sr=False)
    assert torch.equal(a, b)


def test_bf16_second_moment_freeze_vs_stochastic_rounding():
    # test_optim.py:92-110: gradient 1 for 1500 steps, so the bias-corrected v is exactly 1. A
    # per-value bf16 second moment freezes with plain rounding; with stochastic rounding (weights,
    # first AND second moment written back through it) it tracks 1; the fp32 row-wise one is exact.
    R, C, steps = 4, 64, 1500
    rng = np.random.Generator(np.random.PCG64(4))
    init = torch.randn(R, C).bfloat16()
    results = {}
    for name, rowwise, sr in (("plain", False, False), ("sr", False, True), ("rowwise", True, True)):
        p = init.clone()
        m = torch.zeros_like(p)
        v = torch.zeros(R) if rowwise else torch.zeros_like(p)
        for step in range(1, steps + 1):
            noise = lambda r, which: torch.from_numpy(rng.integers(0, 65536, (r.numel(), C)).astype(np.int32))
            oracle.sparse_adam_step(p, m, v, torch.arange(R), torch.ones(R, C), step, 0.0,
                                    stochastic_rounding=sr, noise=noise)
        results[name] = float(v.float().mean()) / (1 - 0.999 ** steps)
    assert results["plain"] < 0.5
    assert abs(results["sr"] - 1) < 0.02
    assert abs(results["rowwise"] - 1) < 1e-4


# ------------------------------------------------------------------------------------- clip
def test_clip_norm_of_known_gradients():
    """rows.py:214-223: the norm over every gradient, dense and sparse: 3-4-12 gives 13."""
    a = torch.tensor([[3.0, 0.0]])
    b = torch.tensor([[4.0], [12.0]])
    assert oracle.clip([a, b], 0.0) == 13.0
    assert torch.equal(a, torch.tensor([[3.0, 0.0]]))  # max_norm 0: no scaling


def test_clip_scales_to_max_norm():
    """coef < 1 scales the gradients so that their norm becomes max_norm (within fp32)."""
    g = torch.Generator().manual_seed(0)
    grads = [torch.randn(50, 8, generator=g) * 3, torch.randn(7, 8, generator=g)]
    norm = oracle.clip(grads, 2.5)
    assert norm > 2.5
    after = float(torch.cat([x.reshape(-1) for x in grads]).double().pow(2).sum().sqrt())
    assert after == pytest.approx(2.5, rel=1e-6)


def test_clip_below_max_norm_is_identity():
    """coef = min(max_norm / (norm + 1e-6), 1) = 1 exactly: the gradients stay bit-equal."""
    g = torch.Generator().manual_seed(1)
    grads = [torch.randn(20, 4, generator=g) * 1e-3, (torch.randn(5, 4, generator=g) * 1e-3).bfloat16()]
    before = [x.clone() for x in grads]
    oracle.clip(grads, 10.0)
    for x, y in zip(grads, before):
        assert torch.equal(x, y)


def test_clip_bf16_uses_rounded_coef():
    """A bf16 gradient is scaled by the coefficient rounded to bf16 (p.grad.mul_(coef.to(bf16))):
    with norm 3 and max_norm 1 the coefficient 1/3 rounds to 0.333984375 in bf16, so 3.0
    becomes round_bf16(3 x 0.333984375) = 1.0 (1.001953125 is nearer 1.0 than 1.0078125), while fp32
    sums are scaled by the fp32 coefficient."""
    dense = torch.tensor([3.0], dtype=torch.bfloat16)
    sparse = torch.tensor([[0.0]])
    oracle.clip([dense, sparse], 1.0)
    assert float(torch.tensor(1 / 3).bfloat16()) == 0.333984375
    assert float(dense) == 1.0
    f32 = torch.tensor([3.0])
    oracle.clip([f32], 1.0)
    assert float(f32) == pytest.approx(1.0, rel=1e-6) and float(f32) != 1.001953125


def test_clip_coef_matches_clip():
    c = oracle.clip_coef(torch.tensor(200.0).sqrt(), 1.0)
    x = torch.tensor([10.0, 10.0])  # norm^2 = 200
    oracle.clip([x], 1.0)
    assert torch.equal(x, torch.full((2,), 10.0) * c)
