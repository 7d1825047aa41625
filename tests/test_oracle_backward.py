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
