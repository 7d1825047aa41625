"""The closed-form gate backward of the oracle, pinned against torch autograd of the oracle's
own inject (micro_engram/module.py:239-261) and against finite differences, on the CPU."""
import pytest
import torch

import oracle


def _inputs(seed, n=37, d=48, M=24, dtype=torch.float64, keep=False, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(n, d, generator=g, dtype=dtype) * 3
    mem = torch.randn(n, M, generator=g, dtype=dtype) * 0.5
    wk = torch.randn(d, M, generator=g, dtype=dtype) * 0.3 * scale
    wv = torch.randn(d, M, generator=g, dtype=dtype) * 0.3
    dq = torch.randn(d, generator=g, dtype=dtype) * 0.1
    dk = torch.randn(d, generator=g, dtype=dtype) * 0.1
    kp = (torch.rand(n, generator=g) > 0.3) if keep else None
    go = torch.randn(n, d, generator=g, dtype=dtype)
    return hidden, mem, wk, wv, dq, dk, kp, go


@pytest.mark.parametrize("gate", ["scalar_sqrt", "scalar"])
@pytest.mark.parametrize("keep", [False, True])
def test_closed_form_matches_autograd(gate, keep):
    hidden, mem, wk, wv, dq, dk, kp, go = _inputs(1 if gate == "scalar" else 2, keep=keep)
    leaves = [t.clone().requires_grad_(True) for t in (hidden, mem, wk, wv, dq, dk)]
    h, m, a_k, a_v, a_q, a_kd = leaves
    out = oracle.inject(h, m, a_k, a_v, gate, a_q, a_kd, keep=kp)
    out.backward(go)
    dx, dK, dV, gq, gk = oracle.inject_backward(go, hidden, mem, wk, wv, gate, dq, dk, keep=kp)
    tol = dict(rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(h.grad, dx, **tol)
    torch.testing.assert_close(m.grad, dK @ wk + dV @ wv, **tol)
    torch.testing.assert_close(a_k.grad, dK.T @ mem, **tol)
    torch.testing.assert_close(a_v.grad, dV.T @ mem, **tol)
    if gate == "scalar_sqrt":
        torch.testing.assert_close(a_q.grad, gq, **tol)
        torch.testing.assert_close(a_kd.grad, gk, **tol)


def test_closed_form_matches_finite_differences():
    # the formula against the derivative itself, not against another implementation of it
    hidden, mem, wk, wv, dq, dk, _, go = _inputs(5, n=6, d=16, M=8)
    dx, dK, dV, gq, gk = oracle.inject_backward(go, hidden, mem, wk, wv, "scalar_sqrt", dq, dk)
    loss = lambda h, q: (oracle.inject(h, mem, wk, wv, "scalar_sqrt", q, dk) * go).sum()
    eps = 1e-6
    for (i, j) in [(0, 0), (2, 5), (5, 15)]:
        hp, hm = hidden.clone(), hidden.clone()
        hp[i, j] += eps
        hm[i, j] -= eps
        fd = (loss(hp, dq) - loss(hm, dq)) / (2 * eps)
        assert abs(float(fd) - float(dx[i, j])) < 1e-6 * max(1.0, abs(float(fd)))
    for j in (0, 7):
        qp, qm = dq.clone(), dq.clone()
        qp[j] += eps
        qm[j] -= eps
        fd = (loss(hidden, qp) - loss(hidden, qm)) / (2 * eps)
        assert abs(float(fd) - float(gq[j])) < 1e-6 * max(1.0, abs(float(fd)))


def test_zero_value_weight_step0():
    # module.py:80 zero-inits W_V: the output is hidden, and only W_V gets a gradient
    # (test_gate.py:29-35): dK = 0 and d hidden = g exactly
    hidden, mem, wk, _, dq, dk, _, go = _inputs(7)
    wv = torch.zeros_like(wk)
    dx, dK, dV, gq, gk = oracle.inject_backward(go, hidden, mem, wk, wv, "scalar_sqrt", dq, dk)
    assert torch.equal(dx, go) and not dK.any() and dV.abs().sum() > 0
    assert not gq.any() and not gk.any()


def test_backward_at_given_stats_equals_recomputed():
    # evaluated at the forward statistics it would compute itself (float64 sums, alpha), the
    # closed form is the same; the term magnitudes bound what the products are made of
    g = torch.Generator().manual_seed(21)
    n, d, m = 23, 40, 12
    hidden = torch.randn(n, d, generator=g, dtype=torch.float64)
    mem = torch.randn(n, m, generator=g, dtype=torch.float64)
    wk = torch.randn(d, m, generator=g, dtype=torch.float64) * 0.3
    wv = torch.randn(d, m, generator=g, dtype=torch.float64) * 0.3
    dq = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    dk = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    go = torch.randn(n, d, generator=g, dtype=torch.float64)
    K = mem @ wk.T
    w = (1 + dq) * (1 + dk)
    sx2, sk2, sck = (hidden ** 2).sum(-1), (K ** 2).sum(-1), (hidden * w * K).sum(-1)
    eps = float(torch.finfo(torch.float32).eps)
    s0 = sck / torch.sqrt(sx2 / d + eps) / torch.sqrt(sk2 / d + eps) / d ** 0.5
    alpha = torch.sigmoid(s0.sign() * s0.abs().clamp_min(1e-6).sqrt())
    stats = torch.stack([sx2, sk2, sck, alpha], dim=1)
    plain = oracle.inject_backward(go, hidden, mem, wk, wv, "scalar_sqrt", dq, dk)
    given = oracle.inject_backward(go, hidden, mem, wk, wv, "scalar_sqrt", dq, dk, stats=stats,
                                   with_terms=True)
    for a, b in zip(plain, given[:5]):
        assert torch.allclose(a, b, rtol=1e-12, atol=1e-14)
    t_dx, t_dk, t_p = given[5]
    assert bool(((given[0] - go).abs() <= t_dx * (1 + 1e-12)).all())
    assert bool((given[1].abs() <= t_dk * (1 + 1e-12)).all())
    assert bool((given[3].abs() <= (1 + dk).abs() * t_p * (1 + 1e-12)).all())


def test_given_stats_bound_catches_a_dropped_term():
    # the GPU test's per-element bound (stored-value rounding + 2^-6 x the term magnitudes) has
    # teeth: a bf16 rounding of the right d hidden stays inside it, d hidden without its
    # r_h^2 sck / d term does not
    g = torch.Generator().manual_seed(5)
    n, d, m = 64, 48, 16
    hidden = torch.randn(n, d, generator=g, dtype=torch.float64) * 2
    mem = torch.randn(n, m, generator=g, dtype=torch.float64)
    wk = torch.randn(d, m, generator=g, dtype=torch.float64) * 0.3
    wv = torch.randn(d, m, generator=g, dtype=torch.float64) * 0.3
    dq = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    dk = torch.randn(d, generator=g, dtype=torch.float64) * 0.1
    go = torch.randn(n, d, generator=g, dtype=torch.float64)
    dx, dK, _, _, _, (t_dx, _, _) = oracle.inject_backward(go, hidden, mem, wk, wv, "scalar_sqrt",
                                                           dq, dk, with_terms=True)
    ulp = lambda x: torch.pow(2.0, torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126))) - 7)
    bound = ulp(dx) + 2.0 ** -6 * t_dx
    assert bool(((dx.to(torch.bfloat16).double() - dx).abs() <= bound).all())
    K = mem @ wk.T
    w = (1 + dq) * (1 + dk)
    eps = float(torch.finfo(torch.float32).eps)
    rh = 1 / torch.sqrt((hidden ** 2).mean(-1) + eps)
    sck = (hidden * w * K).sum(-1)
    c2_term = hidden * (rh * rh * sck / d)[:, None]
    # d hidden without its c2 part: dx - g = a (w K - c2 x), so add a c2 x back (a recovered by
    # least squares from dx - g)
    a = ((dx - go) * (w * K - c2_term)).sum(-1) / ((w * K - c2_term) ** 2).sum(-1)
    wrong = dx + a[:, None] * c2_term
    assert bool(((wrong - dx).abs() > bound).any())
