"""me_gate_residual_noalloc through the C-ABI: the same results as me_gate_residual (the same
kernels, bit for bit) with its scratch in the library's static device array -- two calls in a
row, the second on fewer tokens, so the second reads scratch the first left behind -- and a call
beyond the array's capacity refused before anything is launched."""
import ctypes

import pytest
import torch

from micro_engram_fork_amd import _lib, ops
from micro_engram_fork_amd._lib import ME_BF16, ME_F32, ME_GATE_SCALAR, ME_GATE_SCALAR_SQRT

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(n, d, m, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    hidden = torch.randn(n, d, generator=g, device=DEV).to(dtype)
    mem = (torch.randn(n, m, generator=g, device=DEV) * 0.5).to(dtype)
    wk = (torch.randn(d, m, generator=g, device=DEV) * 0.05).to(dtype)
    wv = (torch.randn(d, m, generator=g, device=DEV) * 0.05).to(dtype)
    dq = torch.randn(d, generator=g, device=DEV) * 0.1
    dk = torch.randn(d, generator=g, device=DEV) * 0.1
    keep = (torch.rand(n, generator=g, device=DEV) > 0.2).to(torch.uint8)
    return hidden, mem, wk, wv, dq, dk, keep


def _args(case, mode, out, alpha, stats):
    hidden, mem, wk, wv, dq, dk, keep = case
    n, d = hidden.shape
    code = ME_BF16 if hidden.dtype == torch.bfloat16 else ME_F32
    return (hidden.data_ptr(), code, n, d, mem.data_ptr(), mem.shape[1], wk.data_ptr(), wv.data_ptr(),
            code, dq.data_ptr(), dk.data_ptr(), ME_F32, mode, keep.data_ptr(), out.data_ptr(),
            alpha.data_ptr(), stats.data_ptr())


def _outputs(case):
    hidden = case[0]
    n = hidden.shape[0]
    return (torch.empty_like(hidden), torch.empty(n, device=DEV), torch.empty(n, 4, device=DEV))


def _with_workspace(case, mode):
    out, alpha, stats = _outputs(case)
    n, d = case[0].shape
    ws = torch.empty(ops.gate_workspace_bytes(n, d), dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.call("me_gate_residual", *_args(case, mode, out, alpha, stats), ws.data_ptr(), ws.numel(), stream)
    return out, alpha, stats


def _without(case, mode):
    out, alpha, stats = _outputs(case)
    stream = torch.cuda.current_stream().cuda_stream
    _lib.call("me_gate_residual_noalloc", *_args(case, mode, out, alpha, stats), stream)
    return out, alpha, stats


def _same_bits(a, b):
    return torch.equal(a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32),
                       b.view(torch.int16 if b.dtype == torch.bfloat16 else torch.int32))


@pytest.mark.parametrize("dtype,mode", [(torch.bfloat16, ME_GATE_SCALAR_SQRT), (torch.float32, ME_GATE_SCALAR)])
def test_noalloc_equals_workspace_entry_point(dtype, mode):
    # the second call is smaller and runs on the scratch the first one filled
    for n, seed in ((3000, 1), (700, 2)):
        case = _case(n, 1024, 512, dtype, seed)
        got = _without(case, mode)
        want = _with_workspace(case, mode)
        torch.cuda.synchronize()
        for g, w in zip(got, want):
            assert _same_bits(g, w), f"n={n}"
        assert not torch.equal(got[0], case[0])  # the gate did add something


def test_noalloc_gemma_decode_shape():
    # the serving decode shape: 256 tokens of model dim 5376, memory 1536 bf16
    case = _case(256, 5376, 1536, torch.bfloat16, 3)
    got = _without(case, ME_GATE_SCALAR_SQRT)
    want = _with_workspace(case, ME_GATE_SCALAR_SQRT)
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert _same_bits(g, w)


def test_noalloc_refuses_more_than_its_scratch():
    # 14,365 tokens at model dim 5376 need more than the 4 MiB array: an error, nothing launched.
    # The operands are real device tensors of that shape, so a regressed size check could only
    # give a wrong result, never an access outside an allocation.
    n, d, m = 14_365, 5376, 1536
    need = ops.gate_workspace_bytes(n, d)
    assert need > 4 << 20 >= ops.gate_workspace_bytes(n - 1, d)
    hidden = torch.zeros(n, d, dtype=torch.bfloat16, device=DEV)
    mem = torch.zeros(n, m, dtype=torch.bfloat16, device=DEV)
    wk = torch.zeros(d, m, dtype=torch.bfloat16, device=DEV)
    wv = torch.zeros(d, m, dtype=torch.bfloat16, device=DEV)
    dq = torch.zeros(d, device=DEV)
    dk = torch.zeros(d, device=DEV)
    out = torch.full_like(hidden, 1.5)
    stream = torch.cuda.current_stream().cuda_stream
    with pytest.raises(_lib.EngramLibError, match="static scratch"):
        _lib.call("me_gate_residual_noalloc", hidden.data_ptr(), ME_BF16, n, d, mem.data_ptr(), m,
                  wk.data_ptr(), wv.data_ptr(), ME_BF16, dq.data_ptr(), dk.data_ptr(), ME_F32,
                  ME_GATE_SCALAR_SQRT, None, out.data_ptr(), None, None, stream)
    torch.cuda.synchronize()
    assert bool((out == 1.5).all())  # nothing was written
