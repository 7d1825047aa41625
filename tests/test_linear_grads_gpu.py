"""me_linear_grads (the key / value Linear layers' gradients, autograd's nn.Linear backward for
micro_engram/module.py:245, 254) against references of the same products:

  grad_mem = gK W_K + gV W_V,  grad_W_K = gK^T mem,  grad_W_V = gV^T mem     (bf16 in and out)

Bound per element: the output is one bf16 rounding of an fp32 sum, so
  |got - ref| <= 2^-8 |ref| + 2^-18 (|A| |B|)
with (|A| |B|) the same product of the operands' magnitudes: half a bf16 ulp plus far more than
the fp32 summation error of either side. A dropped product, a transposed or shifted operand or
a misplaced k-row is off by the order of |ref| itself. Small shapes take a float64 CPU
reference; the Gemma-scale one (8192 tokens, model dim 5376, memory width 1536) a torch fp32
GEMM on the GPU.
"""
import pytest
import torch

from micro_engram_fork_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(n, d, M, seed):
    g = torch.Generator().manual_seed(seed)
    gk = torch.randn(n, d, generator=g) * torch.logspace(-2, 1, n).unsqueeze(1)
    gv = torch.randn(n, d, generator=g)
    mem = torch.randn(n, M, generator=g) * 0.5
    wk = torch.randn(d, M, generator=g) * 0.05
    wv = torch.randn(d, M, generator=g) * 0.05
    return [t.bfloat16() for t in (gk, gv, mem, wk, wv)]


def _refs(gk, gv, mem, wk, wv, dtype, dev):
    c = [t.to(dev).to(dtype) for t in (gk, gv, mem, wk, wv)]
    gk, gv, mem, wk, wv = c
    a = [t.abs() for t in c]
    return ((gk @ wk + gv @ wv, a[0] @ a[3] + a[1] @ a[4]),
            (gk.t() @ mem, a[0].t() @ a[2]),
            (gv.t() @ mem, a[1].t() @ a[2]))


def _check(got, ref, mag, name):
    got = got.to(ref.device).to(ref.dtype)
    err = (got - ref).abs()
    bad = err > 2.0 ** -8 * ref.abs() + 2.0 ** -18 * mag
    assert not bool(bad.any()), (name, int(bad.sum()), float(err.max()))


@pytest.mark.parametrize("n,d,M", [(300, 64, 48), (1000, 128, 200), (517, 320, 1536), (64, 64, 8),
                                   (1, 64, 16), (2049, 192, 392)])
def test_linear_grads_small_shapes_float64(n, d, M):
    # partial tiles on every side: ragged token counts (the grad_W reduction's last slab), model
    # dims that are not whole 256-row tiles, memory widths that are not whole 192 / 256 columns
    ops_in = _operands(n, d, M, seed=n + d + M)
    gk, gv, mem, wk, wv = (t.to(DEV) for t in ops_in)
    d_mem, d_wk, d_wv = ops.linear_grads(gk, gv, mem, wk, wv, True, True, True)
    assert d_mem.shape == (n, M) and d_wk.shape == (d, M) and d_wv.shape == (d, M)
    refs = _refs(*ops_in, torch.float64, "cpu")
    for got, (ref, mag), name in zip((d_mem, d_wk, d_wv), refs, ("mem", "w_key", "w_value")):
        _check(got, ref, mag, name)


def test_linear_grads_gemma_scale_fp32_reference():
    n, d, M = 8192, 5376, 1536
    ops_in = _operands(n, d, M, seed=5)
    gk, gv, mem, wk, wv = (t.to(DEV) for t in ops_in)
    d_mem, d_wk, d_wv = ops.linear_grads(gk, gv, mem, wk, wv, True, True, True)
    refs = _refs(gk, gv, mem, wk, wv, torch.float32, DEV)
    for got, (ref, mag), name in zip((d_mem, d_wk, d_wv), refs, ("mem", "w_key", "w_value")):
        _check(got, ref, mag, name)
    # two calls agree bit for bit (no atomics: every output element is one workgroup's sum)
    again = ops.linear_grads(gk, gv, mem, wk, wv, True, True, True)
    assert all(torch.equal(a, b) for a, b in zip(again, (d_mem, d_wk, d_wv)))


def test_linear_grads_subsets_and_unaligned_operands():
    n, d, M = 700, 128, 96
    gk, gv, mem, wk, wv = (t.to(DEV) for t in _operands(n, d, M, seed=9))
    full = ops.linear_grads(gk, gv, mem, wk, wv, True, True, True)

    def shifted(t):  # the same values one element past a 16-byte boundary
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=DEV)
        view = buf[1:].view(t.shape)
        view.copy_(t)
        return view

    only_v = ops.linear_grads(shifted(gk), shifted(gv), shifted(mem), shifted(wk), shifted(wv),
                              False, False, True)
    assert only_v[0].numel() == 0 and only_v[1].numel() == 0
    assert torch.equal(only_v[2], full[2])
    only_mem = ops.linear_grads(gk, gv, mem, wk, wv, True, False, False)
    assert torch.equal(only_mem[0], full[0]) and only_mem[2].numel() == 0


def test_linear_grads_empty_batch_zero_weight_grads():
    d, M = 64, 32
    z = torch.zeros(0, d, dtype=torch.bfloat16, device=DEV)
    m = torch.zeros(0, M, dtype=torch.bfloat16, device=DEV)
    w = torch.randn(d, M, device=DEV).bfloat16()
    d_mem, d_wk, d_wv = ops.linear_grads(z, z, m, w, w, True, True, True)
    assert d_mem.shape == (0, M)
    assert d_wk.shape == (d, M) and not d_wk.any() and not d_wv.any()


def test_linear_grads_rejects_other_dtypes_and_shapes():
    x = torch.zeros(4, 64, device=DEV)
    with pytest.raises(ValueError):
        ops.linear_grads(x, x, torch.zeros(4, 8, device=DEV), torch.zeros(64, 8, device=DEV),
                         torch.zeros(64, 8, device=DEV), True, True, True)
    b = x.bfloat16()
    with pytest.raises(ValueError):
        ops.linear_grads(b, b, torch.zeros(4, 8, device=DEV).bfloat16(),
                         torch.zeros(32, 8, device=DEV).bfloat16(), torch.zeros(32, 8, device=DEV).bfloat16(),
                         True, True, True)
