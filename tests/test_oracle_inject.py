"""Pins of oracle.inject (micro_engram/module.py:228-261) against facts the mathematics fixes,
independent of the oracle's own formula:

  * value weight 0 -> out == hidden bit for bit (the reference's step-0 no-op,
    test_gate.py:24-27);
  * keep=False tokens unchanged, keep=True tokens equal to the unmasked result
    (test_gate.py:122-130);
  * hidden = 0 -> the score is 0 -> alpha = 1/2 exactly for both gates, so out = V / 2, with V
    chosen exactly representable;
  * hidden = c * 1 and K = c' * 1 (unit scales) -> s0 = sqrt(d) c c' r_h r_k with
    r = 1 / sqrt(x^2 + eps), eps = fp32 eps (visible at c^2 ~ eps); alpha = sigmoid(s0) for
    "scalar", sigmoid(sign(s0) sqrt|s0|) for "scalar_sqrt";
  * q scale 2 (delta 1) doubles s0; k scale 1/2 halves it;
  * |s0| < 1e-6 -> |s| = sqrt(fp32(1e-6)) (the clamp), sign kept; s0 = 0 -> s = 0;
  * bf16 storage: K and V rounded to bf16 by the Linear, the injected term rounded to bf16
    before the add.

The expected values are computed here in float64 from those closed forms (math module), not
from the oracle's code path.
"""
import math

import numpy as np
import pytest
import torch

import oracle

EPS32 = float(np.finfo(np.float32).eps)  # 2^-23: F.rms_norm's eps for fp32 input


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def _one_hot_mem(n, M, col=0, dtype=torch.float32):
    """Memory vectors that select column `col` of the weights: W @ e = W[:, col] exactly."""
    mem = torch.zeros(n, M, dtype=dtype)
    mem[:, col] = 1
    return mem


def _weights_with_column(d, M, col_values, col=0, dtype=torch.float32, seed=0):
    """[d, M] weight whose column `col` is col_values and the rest random (never selected)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(d, M, generator=g).to(dtype)
    w[:, col] = torch.as_tensor(col_values, dtype=torch.float64).to(dtype)
    return w


@pytest.mark.parametrize("gate", ["scalar", "scalar_sqrt"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_value_zero_is_exact_noop(gate, dtype):
    g = torch.Generator().manual_seed(1)
    N, d, M = 7, 48, 40
    hidden = torch.randn(N, d, generator=g).to(dtype)
    mem = torch.randn(N, M, generator=g).to(dtype)
    wk = torch.randn(d, M, generator=g).to(dtype)
    wv = torch.zeros(d, M, dtype=dtype)
    dq, dk = torch.randn(d, generator=g) * 0.1, torch.randn(d, generator=g) * 0.1
    out = oracle.inject(hidden, mem, wk, wv, gate, dq, dk)
    assert out.dtype == dtype
    assert torch.equal(out.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       hidden.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))


@pytest.mark.parametrize("gate", ["scalar", "scalar_sqrt"])
def test_keep_mask(gate):
    g = torch.Generator().manual_seed(2)
    N, d, M = 9, 32, 24
    hidden = torch.randn(N, d, generator=g)
    mem = torch.randn(N, M, generator=g)
    wk, wv = torch.randn(d, M, generator=g), torch.randn(d, M, generator=g)
    dq, dk = torch.randn(d, generator=g) * 0.1, torch.randn(d, generator=g) * 0.1
    keep = torch.tensor([True, False, True, True, False, False, True, False, True])
    full = oracle.inject(hidden, mem, wk, wv, gate, dq, dk)
    masked = oracle.inject(hidden, mem, wk, wv, gate, dq, dk, keep=keep)
    assert torch.equal(masked[~keep], hidden[~keep])
    assert torch.equal(masked[keep], full[keep])
    assert not torch.equal(full[~keep], hidden[~keep])  # the mask did something


@pytest.mark.parametrize("gate", ["scalar", "scalar_sqrt"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_zero_hidden_gives_half_gate(gate, dtype):
    """h = 0 -> s = 0 -> alpha = 1/2 exactly; sign(0) = 0 keeps the scalar_sqrt score at 0
    although the clamp lifts |s0| to 1e-6. V = W_V[:, 0] holds multiples of 1/4 below 2^7, so
    V / 2 is exact in bf16 and fp32: out == V / 2 bit for bit."""
    N, d, M = 5, 16, 12
    hidden = torch.zeros(N, d, dtype=dtype)
    mem = _one_hot_mem(N, M, dtype=dtype)
    vcol = (np.arange(d) - 7) * 0.75
    wv = _weights_with_column(d, M, vcol, dtype=dtype, seed=3)
    wk = _weights_with_column(d, M, np.linspace(-2, 3, d), dtype=dtype, seed=4)
    dq = torch.full((d,), 0.3)
    dk = torch.full((d,), -0.2)
    out, alpha = oracle.inject(hidden, mem, wk, wv, gate, dq, dk, return_alpha=True)
    assert torch.equal(alpha, torch.full((N,), 0.5))
    want = torch.as_tensor(vcol / 2, dtype=torch.float64).to(dtype).expand(N, d)
    assert torch.equal(out, want)


def _const_case(c, cp, d, dq=0.0, dk=0.0, M=6, dtype=torch.float32):
    hidden = torch.full((1, d), c, dtype=torch.float64).to(dtype)
    mem = _one_hot_mem(1, M, col=2, dtype=dtype)
    wk = _weights_with_column(d, M, [cp] * d, col=2, dtype=dtype, seed=5)
    wv = _weights_with_column(d, M, [1.0] * d, col=2, dtype=dtype, seed=6)
    return hidden, mem, wk, wv, torch.full((d,), dq), torch.full((d,), dk)


def _closed_s0(c, cp, d, qs=1.0, ks=1.0):
    """s0 = sum_j (c r_h qs)(c' r_k ks) / sqrt(d) = sqrt(d) c c' r_h r_k qs ks."""
    rh = 1.0 / math.sqrt(c * c + EPS32)
    rk = 1.0 / math.sqrt(cp * cp + EPS32)
    return math.sqrt(d) * c * cp * rh * rk * qs * ks


def _signed_sqrt(s0):
    return math.copysign(math.sqrt(max(abs(s0), 1e-6)), s0) if s0 != 0 else 0.0


@pytest.mark.parametrize("c,cp,d", [(1.5, 0.25, 64), (-2.0, 0.75, 100), (0.5, -3.0, 5376),
                                     (2.0 ** -12, 1.0, 4), (3.0, 2.0 ** -12, 9)])
def test_constant_vectors_closed_form(c, cp, d):
    """Constant hidden and key: the gate is a closed form of (c, c', d). At c = 2^-12,
    c^2 = 2^-24 is a third of eps + c^2, so rms_norm's eps must be fp32's eps exactly; a
    wrong eps, a missing or squared sqrt(d), or a dropped norm moves alpha far past the
    tolerance."""
    hidden, mem, wk, wv, dq, dk = _const_case(c, cp, d)
    s0 = _closed_s0(c, cp, d)
    _, a_scalar = oracle.inject(hidden, mem, wk, wv, "scalar", return_alpha=True)
    _, a_sqrt = oracle.inject(hidden, mem, wk, wv, "scalar_sqrt", dq, dk, return_alpha=True)
    assert float(a_scalar) == pytest.approx(sigmoid(s0), rel=2e-6, abs=1e-7)
    assert float(a_sqrt) == pytest.approx(sigmoid(_signed_sqrt(s0)), rel=2e-6, abs=1e-7)


def test_eps_is_visible():
    """The case c = 2^-12 (d = 4, so the gate is far from saturation) distinguishes fp32 eps
    from eps = 0, 1e-6 and 1e-5."""
    c, cp, d = 2.0 ** -12, 1.0, 4
    hidden, mem, wk, wv, dq, dk = _const_case(c, cp, d)
    _, a = oracle.inject(hidden, mem, wk, wv, "scalar", return_alpha=True)
    right = sigmoid(_closed_s0(c, cp, d))
    for wrong_eps in (0.0, 1e-6, 1e-5):
        rh = 1.0 / math.sqrt(c * c + wrong_eps)
        rk = 1.0 / math.sqrt(cp * cp + wrong_eps)
        wrong = sigmoid(math.sqrt(d) * c * cp * rh * rk)
        assert abs(wrong - right) > 1e-3
    assert float(a) == pytest.approx(right, rel=2e-6)


@pytest.mark.parametrize("c,cp", [(1.0, 0.01), (-0.7, 0.003)])
def test_scales_multiply_the_score(c, cp):
    """scalar_sqrt: q scale 1 + 1 = 2 doubles s0, k scale 1 - 0.5 halves it."""
    d = 64
    for dq, dk, factor in ((1.0, 0.0, 2.0), (0.0, -0.5, 0.5), (1.0, -0.5, 1.0), (0.5, 1.0, 3.0)):
        hidden, mem, wk, wv, q, k = _const_case(c, cp, d, dq=dq, dk=dk)
        _, a = oracle.inject(hidden, mem, wk, wv, "scalar_sqrt", q, k, return_alpha=True)
        s0 = _closed_s0(c, cp, d, 1 + dq, 1 + dk)
        assert s0 == pytest.approx(factor * _closed_s0(c, cp, d))
        assert float(a) == pytest.approx(sigmoid(_signed_sqrt(s0)), rel=2e-6)


def test_tiny_score_is_clamped():
    """|s0| < 1e-6: scalar_sqrt uses sign(s0) sqrt(1e-6) = +-1e-3; the scalar gate uses s0."""
    d, M = 4, 3
    x = torch.tensor([[1.0, 1.0, 1.0, 1.0]])
    for t in (1e-7, -1e-7, 3e-8):
        kcol = [1.0, -1.0, 1.0, -1.0 + t]
        mem = _one_hot_mem(1, M)
        wk = _weights_with_column(d, M, kcol, seed=7)
        wv = _weights_with_column(d, M, [1.0] * d, seed=8)
        zeros = torch.zeros(d)
        _, a = oracle.inject(x, mem, wk, wv, "scalar_sqrt", zeros, zeros, return_alpha=True)
        k32 = np.asarray(kcol, dtype=np.float32).astype(np.float64)
        s0 = (1.0 / math.sqrt(1.0 + EPS32)) / math.sqrt((k32 ** 2).mean() + EPS32) * k32.sum() / 2.0
        assert 0 < abs(s0) < 1e-6
        clamp = float(np.sqrt(np.float32(1e-6)))
        assert float(a) == pytest.approx(sigmoid(math.copysign(clamp, s0)), rel=1e-6)
        _, a_lin = oracle.inject(x, mem, wk, wv, "scalar", return_alpha=True)
        assert float(a_lin) == pytest.approx(sigmoid(s0), rel=1e-6)
    # s0 exactly 0 (K orthogonal to hidden): sign(0) = 0 -> alpha = 1/2 exactly
    wk = _weights_with_column(d, M, [1.0, -1.0, 1.0, -1.0], seed=9)
    zeros = torch.zeros(d)
    _, a0 = oracle.inject(x, _one_hot_mem(1, M), wk, wv, "scalar_sqrt", zeros, zeros, return_alpha=True)
    assert float(a0) == 0.5


def test_negative_score_gives_gate_below_half():
    hidden, mem, wk, wv, dq, dk = _const_case(1.0, -1.0, 16)
    _, a = oracle.inject(hidden, mem, wk, wv, "scalar_sqrt", dq, dk, return_alpha=True)
    s0 = _closed_s0(1.0, -1.0, 16)
    assert s0 < 0 and float(a) < 0.5
    assert float(a) == pytest.approx(sigmoid(-math.sqrt(-s0)), rel=2e-6)


def test_bf16_roundings():
    """bf16 engram and hidden: V is the bf16 Linear output, alpha * V is rounded to bf16 and then
    added to hidden in bf16. With alpha = 1/2 and V = 1 + 2^-7 (exact in bf16), alpha * V =
    1/2 + 2^-8 is exact; added to hidden = 1 it gives 1.5 + 2^-8, a tie between 1.5 and
    1.5 + 2^-7 that rounds to even, 1.5 -- where an fp32 add would keep 1.50390625."""
    N, d, M = 2, 8, 4
    hidden = torch.zeros(N, d, dtype=torch.bfloat16)
    mem = _one_hot_mem(N, M, dtype=torch.bfloat16)
    v = 1.0 + 2.0 ** -7  # exactly representable in bf16 (7 mantissa bits)
    wv = _weights_with_column(d, M, [v] * d, dtype=torch.bfloat16, seed=10)
    wk = _weights_with_column(d, M, [0.5] * d, dtype=torch.bfloat16, seed=11)
    out, alpha = oracle.inject(hidden, mem, wk, wv, "scalar", return_alpha=True)
    assert torch.equal(alpha, torch.full((N,), 0.5))
    assert torch.equal(out.float(), torch.full((N, d), v / 2))  # v/2 is exact too
    one = torch.ones(N, d, dtype=torch.bfloat16)
    wk0 = _weights_with_column(d, M, [0.0] * d, dtype=torch.bfloat16, seed=12)  # K = 0 -> s = 0
    out1, a1 = oracle.inject(one, mem, wk0, wv, "scalar", return_alpha=True)
    assert torch.equal(a1, torch.full((N,), 0.5))
    assert torch.equal(out1.float(), torch.full((N, d), 1.5))


def test_bf16_key_is_rounded():
    """K is the bf16 Linear output: with two memory entries of 1, K_0 = 1 + 2^-8 (a tie in bf16,
    rounded to even: 1.0) and K_1 = 1. Against hidden (1, -1) the rounded key gives s0 = 0 and
    alpha = 1/2 exactly; an unrounded key would give s0 = r_h r_k 2^-8 / sqrt(2) > 0."""
    d, M = 2, 3
    hidden = torch.tensor([[1.0, -1.0]], dtype=torch.bfloat16)
    mem = torch.tensor([[1.0, 1.0, 0.0]], dtype=torch.bfloat16)
    wk = torch.tensor([[1.0, 2.0 ** -8, 5.0], [0.5, 0.5, -3.0]], dtype=torch.bfloat16)
    wv = torch.ones(d, M, dtype=torch.bfloat16)
    assert float(wk[0, 1]) == 2.0 ** -8  # the term itself is exact in bf16
    for gate in ("scalar", "scalar_sqrt"):
        _, a = oracle.inject(hidden, mem, wk, wv, gate, torch.zeros(d), torch.zeros(d),
                             return_alpha=True)
        assert float(a) == 0.5, gate


def test_add_runs_in_hidden_dtype():
    """fp32 engram, bf16 hidden: alpha V = 2^-8 + 2^-16 is rounded to bf16 first (a tie ->
    2^-8) and then added to hidden = 1 in bf16 (1 + 2^-8, a tie -> 1.0). Adding in fp32 and
    rounding once would give 1 + 2^-7."""
    d, M = 4, 2
    hidden = torch.ones(1, d, dtype=torch.bfloat16)
    mem = torch.tensor([[1.0, 0.0]])
    wk = torch.zeros(d, M)  # K = 0 -> s = 0 -> alpha = 1/2
    wv = torch.zeros(d, M)
    wv[:, 0] = 2.0 ** -7 + 2.0 ** -15
    out, a = oracle.inject(hidden, mem, wk, wv, "scalar", return_alpha=True)
    assert float(a) == 0.5
    assert out.dtype == torch.bfloat16
    assert torch.equal(out.float(), torch.ones(1, d))
