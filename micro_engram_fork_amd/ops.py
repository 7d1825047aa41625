"""torch custom ops over the C-ABI of libmicro_engram_amd.so.

Each op takes device tensors, allocates its outputs with torch (the library never allocates),
and enqueues the HIP kernels on the current stream. Ops are registered with
torch.library.custom_op plus a fake implementation, so torch.compile and CUDA-graph capture see
shape-only functions with no host synchronisation (the reference's own custom-op idiom,
micro_engram/train/vendor/op_registry.py:40-67). CPU tensors raise: there is no CPU path.
"""
import ctypes
import functools
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import ME_BF16, ME_F32, ME_I32, ME_I64, ME_U8, call, i32_array, i64_array, ptr_array

_DTYPES = {torch.int32: ME_I32, torch.int64: ME_I64, torch.float32: ME_F32,
           torch.bfloat16: ME_BF16, torch.bool: ME_U8, torch.uint8: ME_U8}


def dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"[micro_engram] unsupported dtype {t.dtype}") from None


def require_gpu(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        d = t.device
        if d == dev:
            continue
        if d.type != "cuda":
            raise RuntimeError(
                f"[micro_engram] the engram path runs only on the GPU (HIP kernels); got a tensor on "
                f"{d}. Move the engram and its inputs to a GPU.")
        if dev is not None:
            raise RuntimeError(f"[micro_engram] tensors on different devices: {dev} and {d}")
        dev = d
    return dev


def stream_of(device):
    """Raw handle of the current stream on `device` (a cuda torch.device): one C call, where
    torch.cuda.current_stream resolves the device and builds a Stream object each time."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


_PLAIN_TENSORS = (torch.Tensor, torch.nn.Parameter)


def _plain(value):
    """True for a plain eager tensor (or parameter), a list/tuple of them, or a non-tensor."""
    if isinstance(value, torch.Tensor):
        return type(value) in _PLAIN_TENSORS
    if isinstance(value, (list, tuple)):
        return all(_plain(v) for v in value)
    return True


def _direct_call(args, kwargs):
    """Whether a call may skip the op's dispatch: nothing is tracing (dynamo), no dispatch mode
    is active (make_fx, FlopCounterMode, debug or recording modes see only the dispatcher) and
    every tensor argument is a plain tensor (fake tensors and other subclasses need the op)."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack():  # this order: dynamo
        return False                                                           # folds the first
    for a in (*args, *kwargs.values()) if kwargs else args:
        tp = type(a)
        if tp in _PLAIN_TENSORS or a is None:
            continue
        if tp is list or tp is tuple:
            for v in a:
                if isinstance(v, torch.Tensor) and type(v) not in _PLAIN_TENSORS:
                    return False
        elif isinstance(a, torch.Tensor):
            return False
    return True


def _custom_op(name):
    """Registers the decorated function as the custom op micro_engram_amd::<name> (what
    torch.compile traces and what a captured graph replays; its fake is added with
    .register_fake) and returns a function that calls the implementation itself for plain eager
    tensors when nothing traces or intercepts the call: the op's dispatch costs ~20 us of host
    time per call, and an eager training step is bound by the rate at which the host issues its
    launches. Everything else (tracing, dispatch modes, fake tensors or other tensor subclasses)
    goes through the op."""
    def wrap(fn):
        op = torch.library.custom_op(f"micro_engram_amd::{name}", mutates_args=())(fn)

        @functools.wraps(fn)
        def dispatch(*args, **kwargs):
            if _direct_call(args, kwargs):
                return fn(*args, **kwargs)
            return op(*args, **kwargs)

        dispatch.op = op
        dispatch.register_fake = op.register_fake
        return dispatch
    return wrap


def _p(t):
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------------------------ hashing
def _pos_arg(position_ids, batch, seq_len):
    """(tensor, batch stride) for position_ids broadcast like .expand_as(ids) in module.py:195."""
    if position_ids is None:
        return None, 0
    pos = position_ids
    if pos.dim() == 1:
        pos = pos.unsqueeze(0)
    if pos.dim() != 2 or pos.shape[-1] != seq_len or pos.shape[0] not in (1, batch):
        raise ValueError(f"[micro_engram] position_ids of shape {tuple(position_ids.shape)} do not "
                         f"broadcast to the ids' [{batch}, {seq_len}]")
    if pos.dtype not in (torch.int32, torch.int64):
        pos = pos.long()
    pos = pos.contiguous()
    return pos, (0 if pos.shape[0] == 1 else seq_len)


def _ids2d(input_ids):
    if input_ids.dim() != 2:
        raise ValueError(f"[micro_engram] input_ids must be [batch, seq], got {tuple(input_ids.shape)}")
    ids = input_ids if input_ids.dtype in (torch.int32, torch.int64) else input_ids.long()
    return ids.contiguous()


def _canon_ptr(canon, identity):
    """The canon map's address, or NULL for the identity map (the kernels then skip the read)."""
    return None if identity else canon.data_ptr()


def _table_args(table_orders, table_rows):
    return _table_args_of(tuple(table_orders), tuple(table_rows))


@functools.lru_cache(maxsize=64)
def _table_args_of(table_orders, table_rows):
    # ctypes arrays the kernels only read: one per distinct table layout
    return len(table_orders), i32_array(list(table_orders)), i64_array(list(table_rows))


@_custom_op("hash_ids")
def hash_ids(input_ids: torch.Tensor, position_ids: Optional[torch.Tensor], canon: torch.Tensor,
             mults: torch.Tensor, table_orders: List[int], table_rows: List[int],
             pad_id: int, identity_canon: bool = False) -> torch.Tensor:
    """Row ids int64 [n_tables, B, T] (micro_engram/module.py:183-205). identity_canon: the
    caller guarantees canon[i] == i, so the kernel skips the canon read."""
    dev = require_gpu(input_ids, position_ids, canon, mults)
    ids = _ids2d(input_ids)
    B, T = ids.shape
    pos, pstride = _pos_arg(position_ids, B, T)
    nt, orders, rows = _table_args(table_orders, table_rows)
    out = torch.empty((nt, B, T), dtype=torch.int64, device=dev)
    call("me_hash_ngrams", ids.data_ptr(), dtype_code(ids), B, T, _p(pos),
         dtype_code(pos) if pos is not None else 0, pstride, _canon_ptr(canon, identity_canon),
         canon.numel(), mults.data_ptr(), mults.shape[1], nt, orders, rows, pad_id, out.data_ptr(),
         stream_of(dev))
    return out


@hash_ids.register_fake
def _(input_ids, position_ids, canon, mults, table_orders, table_rows, pad_id, identity_canon=False):
    return input_ids.new_empty((len(table_orders), *input_ids.shape), dtype=torch.int64)


def _prev_ids(ids):
    if ids.dim() != 2:
        raise ValueError(f"[micro_engram] ids must be [n, max_order], got {tuple(ids.shape)}")
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.long()
    if ids.stride(1) != 1:
        ids = ids.contiguous()
    return ids


@_custom_op("hash_prev")
def hash_prev(ids: torch.Tensor, canon: torch.Tensor, mults: torch.Tensor,
              table_orders: List[int], table_rows: List[int], pad_id: int,
              identity_canon: bool = False) -> torch.Tensor:
    """Row ids int64 [n_tables, N] from [N, W] predecessor ids (micro_engram/module.py:207-226)."""
    dev = require_gpu(ids, canon, mults)
    ids = _prev_ids(ids)
    N, W = ids.shape
    nt, orders, rows = _table_args(table_orders, table_rows)
    out = torch.empty((nt, N), dtype=torch.int64, device=dev)
    call("me_hash_prev", ids.data_ptr(), dtype_code(ids), N, W, ids.stride(0) if N else W,
         _canon_ptr(canon, identity_canon), canon.numel(), mults.data_ptr(), mults.shape[1], nt,
         orders, rows, pad_id, out.data_ptr(), stream_of(dev))
    return out


@hash_prev.register_fake
def _(ids, canon, mults, table_orders, table_rows, pad_id, identity_canon=False):
    return ids.new_empty((len(table_orders), ids.shape[0]), dtype=torch.int64)


# ------------------------------------------------------------------------------------- gather
_TABLES_ARGS = {}


def _tables_arg(tables: Sequence[torch.Tensor]):
    """(pointer array, row counts, row width) of the tables, checked: kept per (address, shape,
    strides, dtype) of every table, which fix all three (the arrays are only read)."""
    key = tuple((t.data_ptr(), t.shape, t.stride(), t.dtype) for t in tables)
    hit = _TABLES_ARGS.get(key)
    if hit is None:
        if len(_TABLES_ARGS) >= 256:
            _TABLES_ARGS.clear()
        hit = _TABLES_ARGS[key] = _tables_arg_checked(tables)
    return hit


def _tables_arg_checked(tables):
    t0 = tables[0]
    dim = t0.shape[1]
    for t in tables:
        if t.dim() != 2 or t.shape[1] != dim or t.dtype != t0.dtype:
            raise ValueError("[micro_engram] tables must be 2-D with one row width and dtype")
        if not t.is_contiguous():
            raise ValueError("[micro_engram] tables must be contiguous")
    return ptr_array([t.data_ptr() for t in tables]), i64_array([t.shape[0] for t in tables]), dim


@_custom_op("gather")
def gather(idx: torch.Tensor, tables: List[torch.Tensor]) -> torch.Tensor:
    """mem [N, n_tables * D] from row ids int64 [n_tables, N] (module.py:146-154, 233; rows
    outside a table read as zeros, micro_engram_vllm/tp.py:20-39)."""
    dev = require_gpu(idx, *tables)
    if idx.dim() != 2 or idx.shape[0] != len(tables) or idx.dtype != torch.int64:
        raise ValueError("[micro_engram] idx must be int64 [n_tables, N]")
    if idx.stride(1) != 1:
        idx = idx.contiguous()
    ptrs, rows, dim = _tables_arg(tables)
    N = idx.shape[1]
    mem = torch.empty((N, len(tables) * dim), dtype=tables[0].dtype, device=dev)
    call("me_gather", idx.data_ptr(), idx.stride(0) if len(tables) > 1 else N, N, len(tables),
         ptrs, rows, dim, dtype_code(tables[0]), mem.data_ptr(), stream_of(dev))
    return mem


@gather.register_fake
def _(idx, tables):
    return tables[0].new_empty((idx.shape[1], len(tables) * tables[0].shape[1]))


@_custom_op("hash_gather")
def hash_gather(input_ids: torch.Tensor, position_ids: Optional[torch.Tensor], canon: torch.Tensor,
                mults: torch.Tensor, table_orders: List[int], table_rows: List[int], pad_id: int,
                tables: List[torch.Tensor], with_idx: bool,
                identity_canon: bool = False) -> List[torch.Tensor]:
    """[mem [B*T, n_tables*D]] or [mem, idx [n_tables, B, T]]: hash_ids + lookup + cat in one
    kernel (module.py:263-265)."""
    dev = require_gpu(input_ids, position_ids, canon, mults, *tables)
    ids = _ids2d(input_ids)
    B, T = ids.shape
    pos, pstride = _pos_arg(position_ids, B, T)
    nt, orders, rows = _table_args(table_orders, table_rows)
    ptrs, _rows, dim = _tables_arg(tables)
    mem = torch.empty((B * T, nt * dim), dtype=tables[0].dtype, device=dev)
    idx = torch.empty((nt, B, T), dtype=torch.int64, device=dev) if with_idx else None
    call("me_hash_gather", ids.data_ptr(), dtype_code(ids), B, T, _p(pos),
         dtype_code(pos) if pos is not None else 0, pstride, _canon_ptr(canon, identity_canon),
         canon.numel(), mults.data_ptr(), mults.shape[1], nt, orders, rows, pad_id, ptrs, dim,
         dtype_code(tables[0]), mem.data_ptr(), _p(idx), stream_of(dev))
    return [mem, idx] if with_idx else [mem]


@hash_gather.register_fake
def _(input_ids, position_ids, canon, mults, table_orders, table_rows, pad_id, tables, with_idx,
      identity_canon=False):
    n = input_ids.shape[0] * input_ids.shape[1]
    mem = tables[0].new_empty((n, len(tables) * tables[0].shape[1]))
    if with_idx:
        return [mem, input_ids.new_empty((len(tables), *input_ids.shape), dtype=torch.int64)]
    return [mem]


@_custom_op("hash_prev_gather")
def hash_prev_gather(ids: torch.Tensor, canon: torch.Tensor, mults: torch.Tensor,
                     table_orders: List[int], table_rows: List[int], pad_id: int,
                     tables: List[torch.Tensor], with_idx: bool,
                     identity_canon: bool = False) -> List[torch.Tensor]:
    """[mem [N, n_tables*D]] or [mem, idx [n_tables, N]]: hash_prev + lookup in one kernel."""
    dev = require_gpu(ids, canon, mults, *tables)
    ids = _prev_ids(ids)
    N, W = ids.shape
    nt, orders, rows = _table_args(table_orders, table_rows)
    ptrs, _rows, dim = _tables_arg(tables)
    mem = torch.empty((N, nt * dim), dtype=tables[0].dtype, device=dev)
    idx = torch.empty((nt, N), dtype=torch.int64, device=dev) if with_idx else None
    call("me_hash_prev_gather", ids.data_ptr(), dtype_code(ids), N, W, ids.stride(0) if N else W,
         _canon_ptr(canon, identity_canon), canon.numel(), mults.data_ptr(), mults.shape[1], nt,
         orders, rows, pad_id, ptrs, dim, dtype_code(tables[0]), mem.data_ptr(), _p(idx),
         stream_of(dev))
    return [mem, idx] if with_idx else [mem]


@hash_prev_gather.register_fake
def _(ids, canon, mults, table_orders, table_rows, pad_id, tables, with_idx, identity_canon=False):
    mem = tables[0].new_empty((ids.shape[0], len(tables) * tables[0].shape[1]))
    if with_idx:
        return [mem, ids.new_empty((len(tables), ids.shape[0]), dtype=torch.int64)]
    return [mem]


# ----------------------------------------------------------------------------- gate + residual
def gate_workspace_bytes(n, d):
    size = ctypes.c_size_t(0)
    call("me_gate_workspace_size", n, d, ctypes.byref(size))
    return size.value


def _aligned(t):
    return t.data_ptr() % 16 == 0


def _gate_operands(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep):
    """Checked, contiguous, 16-byte aligned operands of the gate kernels."""
    d = hidden.shape[-1]
    x = hidden.reshape(-1, d)
    N = x.shape[0]
    if mem.dim() != 2 or mem.shape[0] != N:
        raise ValueError(f"[micro_engram] mem {tuple(mem.shape)} does not match {N} tokens")
    M = mem.shape[1]
    for w in (w_key, w_value):
        if tuple(w.shape) != (d, M) or w.dtype != mem.dtype:
            raise ValueError(f"[micro_engram] weight {tuple(w.shape)}/{w.dtype} does not match "
                             f"[{d}, {M}]/{mem.dtype}")
    x, mem = x.contiguous(), mem.contiguous()
    w_key, w_value = w_key.contiguous(), w_value.contiguous()
    if not all(_aligned(t) for t in (x, mem, w_key, w_value)):
        x, mem, w_key, w_value = (t.clone() if not _aligned(t) else t for t in (x, mem, w_key, w_value))
    scale_code = 0
    if gate_mode == _lib.ME_GATE_SCALAR_SQRT:
        if q_scale_delta is None or k_scale_delta is None:
            raise ValueError("[micro_engram] the scalar_sqrt gate needs q_scale and k_scale")
        q_scale_delta, k_scale_delta = q_scale_delta.contiguous(), k_scale_delta.contiguous()
        if q_scale_delta.dtype != k_scale_delta.dtype:
            k_scale_delta = k_scale_delta.to(q_scale_delta.dtype)
        if not (_aligned(q_scale_delta) and _aligned(k_scale_delta)):
            q_scale_delta, k_scale_delta = q_scale_delta.clone(), k_scale_delta.clone()
        scale_code = dtype_code(q_scale_delta)
    keep_u8 = None
    if keep is not None:
        keep_u8 = keep.reshape(-1).to(torch.uint8).contiguous()
        if keep_u8.numel() != N:
            raise ValueError(f"[micro_engram] keep has {keep_u8.numel()} entries for {N} tokens")
    return x, mem, w_key, w_value, q_scale_delta, k_scale_delta, scale_code, keep_u8, N, d, M


@_custom_op("gate_residual")
def gate_residual(hidden: torch.Tensor, mem: torch.Tensor, w_key: torch.Tensor,
                  w_value: torch.Tensor, q_scale_delta: Optional[torch.Tensor],
                  k_scale_delta: Optional[torch.Tensor], gate_mode: int,
                  keep: Optional[torch.Tensor], with_alpha: bool,
                  with_stats: bool = False) -> List[torch.Tensor]:
    """[out], plus alpha [N] fp32 when with_alpha, plus row stats [N, 4] fp32 (what the backward
    needs) when with_stats: hidden + gated W_V mem, the scalar gates of MicroEngram.inject
    (micro_engram/module.py:239-261). hidden [..., d]; mem [N, M] with N the number of hidden
    rows; weights [d, M] (nn.Linear layout) in mem's dtype."""
    dev = require_gpu(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, keep)
    x, mem, w_key, w_value, q_scale_delta, k_scale_delta, scale_code, keep_u8, N, d, M = \
        _gate_operands(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep)
    out = torch.empty_like(x)
    alpha = torch.empty(N, dtype=torch.float32, device=dev) if with_alpha else None
    stats = torch.empty((N, 4), dtype=torch.float32, device=dev) if with_stats else None
    ws = torch.empty(max(gate_workspace_bytes(N, d), 16), dtype=torch.uint8, device=dev)
    call("me_gate_residual", x.data_ptr(), dtype_code(x), N, d, mem.data_ptr(), M,
         w_key.data_ptr(), w_value.data_ptr(), dtype_code(mem), _p(q_scale_delta),
         _p(k_scale_delta), scale_code, gate_mode, _p(keep_u8), out.data_ptr(), _p(alpha),
         _p(stats), ws.data_ptr(), ws.numel(), stream_of(dev))
    res = [out.reshape(hidden.shape)]
    if with_alpha:
        res.append(alpha)
    if with_stats:
        res.append(stats)
    return res


@gate_residual.register_fake
def _(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep, with_alpha,
      with_stats=False):
    n = hidden.numel() // hidden.shape[-1]
    res = [torch.empty_like(hidden)]
    if with_alpha:
        res.append(hidden.new_empty((n,), dtype=torch.float32))
    if with_stats:
        res.append(hidden.new_empty((n, 4), dtype=torch.float32))
    return res


@_custom_op("kv_proj")
def kv_proj(mem: torch.Tensor, w_key: torch.Tensor, w_value: torch.Tensor) -> torch.Tensor:
    """[K | V] [N, 2d] in mem's dtype: the key and value nn.Linear outputs of
    MicroEngram.inject (module.py:245, 254) for few tokens, in one hand-written MFMA kernel
    (me_kv_proj). mem [N, M]; w_key, w_value [d, M] (nn.Linear layout)."""
    dev = require_gpu(mem, w_key, w_value)
    if mem.dim() != 2 or w_key.dim() != 2 or w_key.shape != w_value.shape or w_key.shape[1] != mem.shape[1]:
        raise ValueError(f"[micro_engram] kv_proj: mem {tuple(mem.shape)} and weights {tuple(w_key.shape)}/"
                         f"{tuple(w_value.shape)} do not fit")
    if not (mem.dtype == w_key.dtype == w_value.dtype):
        raise ValueError("[micro_engram] kv_proj: mem and the weights must share one dtype")
    mem, w_key, w_value = (t.contiguous() for t in (mem, w_key, w_value))
    mem, w_key, w_value = (t if _aligned(t) else t.clone() for t in (mem, w_key, w_value))
    N, M = mem.shape
    d = w_key.shape[0]
    kv = torch.empty((N, 2 * d), dtype=mem.dtype, device=dev)
    call("me_kv_proj", mem.data_ptr(), N, M, w_key.data_ptr(), w_value.data_ptr(), d, dtype_code(mem),
         kv.data_ptr(), stream_of(dev))
    return kv


@kv_proj.register_fake
def _(mem, w_key, w_value):
    return mem.new_empty((mem.shape[0], 2 * w_key.shape[0]))


def fits_mfma(model_dim, mem_dim, dtype):
    """Whether the MFMA gate kernels (me_gate_residual, me_gate_backward, me_kv_proj) take this
    shape: model dim a multiple of 8 and memory rows a multiple of 16 bytes. Other shapes run
    the row kernels (me_gate_rows, me_gate_rows_backward) after library GEMMs."""
    esize = 2 if dtype == torch.bfloat16 else 4
    return model_dim % 8 == 0 and (mem_dim * esize) % 16 == 0


def _kv_rows(k, v, d):
    """K and V rows for the row kernels: one stride for both (contiguous [N, d] tensors)."""
    k, v = k.reshape(-1, d).contiguous(), v.reshape(-1, d).contiguous()
    if k.dtype != v.dtype:
        raise ValueError("[micro_engram] K and V rows must share one dtype")
    return k, v


@_custom_op("gate_rows")
def gate_rows(hidden: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              q_scale_delta: Optional[torch.Tensor], k_scale_delta: Optional[torch.Tensor],
              gate_mode: int, keep: Optional[torch.Tensor], with_alpha: bool,
              with_stats: bool = False) -> List[torch.Tensor]:
    """The gate and residual add (module.py:239-261) from the key / value Linear outputs K, V
    [N, d] computed elsewhere: me_gate_rows, any model dim. [out] (+ alpha, + row stats)."""
    dev = require_gpu(hidden, k, v, q_scale_delta, k_scale_delta, keep)
    d = hidden.shape[-1]
    x = hidden.reshape(-1, d).contiguous()
    N = x.shape[0]
    k, v = _kv_rows(k, v, d)
    if k.shape[0] != N:
        raise ValueError(f"[micro_engram] K/V rows {tuple(k.shape)} do not match {N} tokens")
    q_scale_delta, k_scale_delta, scale_code = _scales(q_scale_delta, k_scale_delta, gate_mode)
    keep_u8 = _keep_u8(keep, N)
    out = torch.empty_like(x)
    alpha = torch.empty(N, dtype=torch.float32, device=dev) if with_alpha else None
    stats = torch.empty((N, 4), dtype=torch.float32, device=dev) if with_stats else None
    call("me_gate_rows", x.data_ptr(), dtype_code(x), N, d, k.data_ptr(), v.data_ptr(), d,
         dtype_code(k), _p(q_scale_delta), _p(k_scale_delta), scale_code, gate_mode, _p(keep_u8),
         out.data_ptr(), _p(alpha), _p(stats), stream_of(dev))
    res = [out.reshape(hidden.shape)]
    if with_alpha:
        res.append(alpha)
    if with_stats:
        res.append(stats)
    return res


@gate_rows.register_fake
def _(hidden, k, v, q_scale_delta, k_scale_delta, gate_mode, keep, with_alpha, with_stats=False):
    n = hidden.numel() // hidden.shape[-1]
    res = [torch.empty_like(hidden)]
    if with_alpha:
        res.append(hidden.new_empty((n,), dtype=torch.float32))
    if with_stats:
        res.append(hidden.new_empty((n, 4), dtype=torch.float32))
    return res


@_custom_op("gate_rows_backward")
def gate_rows_backward(grad_out: torch.Tensor, hidden: torch.Tensor, k: torch.Tensor,
                       v: torch.Tensor, q_scale_delta: Optional[torch.Tensor],
                       k_scale_delta: Optional[torch.Tensor], gate_mode: int,
                       keep: Optional[torch.Tensor], stats: torch.Tensor) -> List[torch.Tensor]:
    """Gradients of gate_rows from the same K, V rows (me_gate_rows_backward, any model dim):
    [grad_hidden, grad of K [N, d], grad of V [N, d], grad_q_scale_delta, grad_k_scale_delta
    ([d] fp32; empty for the scalar gate)]."""
    dev = require_gpu(grad_out, hidden, k, v, q_scale_delta, k_scale_delta, keep, stats)
    d = hidden.shape[-1]
    x = hidden.reshape(-1, d).contiguous()
    N = x.shape[0]
    k, v = _kv_rows(k, v, d)
    g = grad_out.reshape(-1, d).to(x.dtype).contiguous()
    stats = stats.contiguous()
    if tuple(stats.shape) != (N, 4) or stats.dtype != torch.float32:
        raise ValueError(f"[micro_engram] stats must be fp32 [{N}, 4], got {tuple(stats.shape)}")
    q_scale_delta, k_scale_delta, scale_code = _scales(q_scale_delta, k_scale_delta, gate_mode)
    keep_u8 = _keep_u8(keep, N)
    grad_hidden = torch.empty_like(x)
    grad_k = torch.empty((N, d), dtype=k.dtype, device=dev)
    grad_v = torch.empty((N, d), dtype=k.dtype, device=dev)
    sqrt = gate_mode == _lib.ME_GATE_SCALAR_SQRT
    grad_q = torch.empty(d if sqrt else 0, dtype=torch.float32, device=dev)
    grad_kd = torch.empty(d if sqrt else 0, dtype=torch.float32, device=dev)
    size = ctypes.c_size_t(0)
    call("me_gate_rows_backward_workspace_size", N, d, ctypes.byref(size))
    ws = torch.empty(max(size.value, 16), dtype=torch.uint8, device=dev)
    call("me_gate_rows_backward", x.data_ptr(), dtype_code(x), N, d, k.data_ptr(), v.data_ptr(), d,
         dtype_code(k), _p(q_scale_delta), _p(k_scale_delta), scale_code, gate_mode, _p(keep_u8),
         g.data_ptr(), stats.data_ptr(), grad_hidden.data_ptr(), grad_k.data_ptr(),
         grad_v.data_ptr(), grad_q.data_ptr() if sqrt else None, grad_kd.data_ptr() if sqrt else None,
         ws.data_ptr(), ws.numel(), stream_of(dev))
    return [grad_hidden.reshape(hidden.shape), grad_k, grad_v, grad_q, grad_kd]


@gate_rows_backward.register_fake
def _(grad_out, hidden, k, v, q_scale_delta, k_scale_delta, gate_mode, keep, stats):
    n, d = hidden.numel() // hidden.shape[-1], hidden.shape[-1]
    nd = d if gate_mode == _lib.ME_GATE_SCALAR_SQRT else 0
    return [torch.empty_like(hidden), k.new_empty((n, d)), k.new_empty((n, d)),
            hidden.new_empty((nd,), dtype=torch.float32), hidden.new_empty((nd,), dtype=torch.float32)]


def _scales(q_scale_delta, k_scale_delta, gate_mode):
    """(q delta, k delta, dtype code) for the row kernels; (None, None, 0) for the scalar gate."""
    if gate_mode != _lib.ME_GATE_SCALAR_SQRT:
        return None, None, 0
    if q_scale_delta is None or k_scale_delta is None:
        raise ValueError("[micro_engram] the scalar_sqrt gate needs q_scale and k_scale")
    q, k = q_scale_delta.contiguous(), k_scale_delta.contiguous()
    if q.dtype != k.dtype:
        k = k.to(q.dtype)
    return q, k, dtype_code(q)


def _keep_u8(keep, n):
    if keep is None:
        return None
    keep_u8 = keep.reshape(-1).to(torch.uint8).contiguous()
    if keep_u8.numel() != n:
        raise ValueError(f"[micro_engram] keep has {keep_u8.numel()} entries for {n} tokens")
    return keep_u8


@_custom_op("gate_residual_rows")
def gate_residual_rows(hidden: torch.Tensor, mem: torch.Tensor, w_key: torch.Tensor,
                       w_value: torch.Tensor, q_scale_delta: Optional[torch.Tensor],
                       k_scale_delta: Optional[torch.Tensor], gate_mode: int,
                       keep: Optional[torch.Tensor], with_alpha: bool,
                       with_stats: bool = False) -> List[torch.Tensor]:
    """gate_residual for few tokens: [K | V] from me_kv_proj (K and V rounded to mem's dtype, as
    the two nn.Linear calls of module.py:245, 254 give them), then the gate and the residual add
    in me_gate_rows."""
    dev = require_gpu(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, keep)
    x, mem, w_key, w_value, q_scale_delta, k_scale_delta, scale_code, keep_u8, N, d, M = \
        _gate_operands(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep)
    kv = torch.empty((N, 2 * d), dtype=mem.dtype, device=dev)
    if N:
        call("me_kv_proj", mem.data_ptr(), N, M, w_key.data_ptr(), w_value.data_ptr(), d,
             dtype_code(mem), kv.data_ptr(), stream_of(dev))
    out = torch.empty_like(x)
    alpha = torch.empty(N, dtype=torch.float32, device=dev) if with_alpha else None
    stats = torch.empty((N, 4), dtype=torch.float32, device=dev) if with_stats else None
    call("me_gate_rows", x.data_ptr(), dtype_code(x), N, d, kv.data_ptr(),
         kv.data_ptr() + d * kv.element_size(), 2 * d, dtype_code(kv), _p(q_scale_delta),
         _p(k_scale_delta), scale_code, gate_mode, _p(keep_u8), out.data_ptr(), _p(alpha),
         _p(stats), stream_of(dev))
    res = [out.reshape(hidden.shape)]
    if with_alpha:
        res.append(alpha)
    if with_stats:
        res.append(stats)
    return res


@gate_residual_rows.register_fake
def _(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep, with_alpha,
      with_stats=False):
    n = hidden.numel() // hidden.shape[-1]
    res = [torch.empty_like(hidden)]
    if with_alpha:
        res.append(hidden.new_empty((n,), dtype=torch.float32))
    if with_stats:
        res.append(hidden.new_empty((n, 4), dtype=torch.float32))
    return res


def gate_backward_workspace_bytes(n, d):
    size = ctypes.c_size_t(0)
    call("me_gate_backward_workspace_size", n, d, ctypes.byref(size))
    return size.value


@_custom_op("gate_backward")
def gate_backward(grad_out: torch.Tensor, hidden: torch.Tensor, mem: torch.Tensor,
                  w_key: torch.Tensor, w_value: torch.Tensor,
                  q_scale_delta: Optional[torch.Tensor], k_scale_delta: Optional[torch.Tensor],
                  gate_mode: int, keep: Optional[torch.Tensor],
                  stats: torch.Tensor) -> List[torch.Tensor]:
    """Gradients of gate_residual from the gradient of its output: [grad_hidden (like hidden),
    grad_key [N, d] and grad_value [N, d] (gradients of the key / value Linear outputs, in
    mem's dtype), grad_q_scale_delta, grad_k_scale_delta ([d] fp32; empty for the scalar
    gate)] -- what autograd gives through module.py:239-261."""
    dev = require_gpu(grad_out, hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, keep,
                      stats)
    x, mem, w_key, w_value, q_scale_delta, k_scale_delta, scale_code, keep_u8, N, d, M = \
        _gate_operands(hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep)
    g = grad_out.reshape(-1, d).to(x.dtype).contiguous()
    if not _aligned(g):
        g = g.clone()
    stats = stats.contiguous()
    if tuple(stats.shape) != (N, 4) or stats.dtype != torch.float32:
        raise ValueError(f"[micro_engram] stats must be fp32 [{N}, 4], got {tuple(stats.shape)}")
    grad_hidden = torch.empty_like(x)
    grad_key = torch.empty((N, d), dtype=mem.dtype, device=dev)
    grad_value = torch.empty((N, d), dtype=mem.dtype, device=dev)
    sqrt = gate_mode == _lib.ME_GATE_SCALAR_SQRT
    grad_q = torch.empty(d if sqrt else 0, dtype=torch.float32, device=dev)
    grad_k = torch.empty(d if sqrt else 0, dtype=torch.float32, device=dev)
    ws = torch.empty(max(gate_backward_workspace_bytes(N, d), 16), dtype=torch.uint8, device=dev)
    call("me_gate_backward", x.data_ptr(), dtype_code(x), N, d, mem.data_ptr(), M,
         w_key.data_ptr(), w_value.data_ptr(), dtype_code(mem), _p(q_scale_delta),
         _p(k_scale_delta), scale_code, gate_mode, _p(keep_u8), g.data_ptr(), stats.data_ptr(),
         grad_hidden.data_ptr(), grad_key.data_ptr(), grad_value.data_ptr(),
         grad_q.data_ptr() if sqrt else None, grad_k.data_ptr() if sqrt else None, ws.data_ptr(),
         ws.numel(), stream_of(dev))
    return [grad_hidden.reshape(hidden.shape), grad_key, grad_value, grad_q, grad_k]


@gate_backward.register_fake
def _(grad_out, hidden, mem, w_key, w_value, q_scale_delta, k_scale_delta, gate_mode, keep, stats):
    n, d = hidden.numel() // hidden.shape[-1], hidden.shape[-1]
    nd = d if gate_mode == _lib.ME_GATE_SCALAR_SQRT else 0
    return [torch.empty_like(hidden), mem.new_empty((n, d)), mem.new_empty((n, d)),
            hidden.new_empty((nd,), dtype=torch.float32), hidden.new_empty((nd,), dtype=torch.float32)]


def fits_linear_grads(n, model_dim, mem_dim, dtype):
    """Whether me_linear_grads takes the key / value Linear layers' gradients: bf16 operands,
    model dim a multiple of 64, memory width a multiple of 8, every operand under 2 GiB. Other
    shapes and fp32 engrams take the library GEMMs."""
    lim = 1 << 31
    return (dtype == torch.bfloat16 and model_dim % 64 == 0 and mem_dim % 8 == 0 and
            n * model_dim * 2 < lim and n * mem_dim * 2 < lim and model_dim * mem_dim * 2 < lim)


@_custom_op("linear_grads")
def linear_grads(grad_key: torch.Tensor, grad_value: torch.Tensor, mem: torch.Tensor,
                 w_key: torch.Tensor, w_value: torch.Tensor, need_mem: bool, need_w_key: bool,
                 need_w_value: bool) -> List[torch.Tensor]:
    """[grad_mem [N, M], grad_w_key [d, M], grad_w_value [d, M]] (an empty tensor for each one
    not needed): the gradients autograd gives the two nn.Linear calls of the reference's
    forward (micro_engram/module.py:245, 254) from the gradients of their outputs,
    grad_mem = gK W_K + gV W_V and grad_W = g^T mem, on the hand-written MFMA kernel. bf16."""
    dev = require_gpu(grad_key, grad_value, mem, w_key, w_value)
    n, d = grad_key.shape
    M = mem.shape[-1]
    if grad_value.shape != (n, d) or mem.numel() != n * M or w_key.shape != (d, M) or w_value.shape != (d, M):
        raise ValueError(f"[micro_engram] linear_grads: shapes {tuple(grad_key.shape)}, "
                         f"{tuple(grad_value.shape)}, {tuple(mem.shape)}, {tuple(w_key.shape)}, "
                         f"{tuple(w_value.shape)} do not match")
    if any(t.dtype != torch.bfloat16 for t in (grad_key, grad_value, mem, w_key, w_value)):
        raise ValueError("[micro_engram] linear_grads takes bf16 operands")

    def ready(t):
        t = t.contiguous()
        return t if _aligned(t) else t.clone()

    gk, gv, m, wk, wv = (ready(t) for t in (grad_key, grad_value, mem.reshape(n, M), w_key, w_value))
    bf = dict(dtype=torch.bfloat16, device=dev)
    d_mem = torch.empty((n, M) if need_mem else (0,), **bf)
    d_wk = torch.empty((d, M) if need_w_key else (0,), **bf)
    d_wv = torch.empty((d, M) if need_w_value else (0,), **bf)
    call("me_linear_grads", gk.data_ptr(), gv.data_ptr(), n, d, m.data_ptr(), M, wk.data_ptr(),
         wv.data_ptr(), d_mem.data_ptr() if need_mem else None,
         d_wk.data_ptr() if need_w_key else None, d_wv.data_ptr() if need_w_value else None,
         stream_of(dev))
    return [d_mem, d_wk, d_wv]


@linear_grads.register_fake
def _(grad_key, grad_value, mem, w_key, w_value, need_mem, need_w_key, need_w_value):
    n, d = grad_key.shape
    M = mem.shape[-1]
    return [grad_key.new_empty((n, M) if need_mem else (0,)),
            grad_key.new_empty((d, M) if need_w_key else (0,)),
            grad_key.new_empty((d, M) if need_w_value else (0,))]


def library_loaded():
    """Loads the HIP library (raises if it is missing) and returns its path."""
    _lib.load()
    return _lib.lib_path()


# ------------------------------------------------------------------------- training side
@functools.lru_cache(maxsize=64)
def dedup_workspace_bytes(n):
    size = ctypes.c_size_t(0)
    call("me_dedup_workspace_size", n, ctypes.byref(size))
    return size.value


@_custom_op("dedup")
def dedup(keys: torch.Tensor, key_bound: int, grads: Optional[torch.Tensor]) -> List[torch.Tensor]:
    """[uniq [n], inv [n], count [1]] or [uniq, inv, count, gsum [n, D]]: torch.unique(keys,
    return_inverse=True) with the fp32 index_add_ sums of `grads` (micro_engram/rows.py:81,
    117-118, 144-146). Only uniq[:count] and gsum[:count] are meaningful."""
    dev = require_gpu(keys, grads)
    keys = keys.reshape(-1).long().contiguous()
    n = keys.numel()
    uniq = torch.empty(n, dtype=torch.int64, device=dev)
    inv = torch.empty(n, dtype=torch.int64, device=dev)
    count = torch.empty(1, dtype=torch.int64, device=dev)
    gsum, gptr, gcode, dim = None, None, 0, 0
    if grads is not None:
        grads = grads.reshape(n, grads.shape[-1] if grads.dim() >= 2 else 1)
        if grads.dtype not in (torch.float32, torch.bfloat16):
            grads = grads.float()
        grads = grads.contiguous()
        dim = grads.shape[1]
        gsum = torch.empty((n, dim), dtype=torch.float32, device=dev)
        gptr, gcode = grads.data_ptr(), dtype_code(grads)
    ws = torch.empty(max(dedup_workspace_bytes(n), 16), dtype=torch.uint8, device=dev)
    call("me_dedup", _p(keys), n, key_bound, gptr, gcode, dim, _p(uniq), _p(inv), _p(gsum),
         count.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(dev))
    return [uniq, inv, count] if gsum is None else [uniq, inv, count, gsum]


@dedup.register_fake
def _(keys, key_bound, grads):
    n = keys.numel()
    outs = [keys.new_empty(n, dtype=torch.int64), keys.new_empty(n, dtype=torch.int64),
            keys.new_empty(1, dtype=torch.int64)]
    if grads is not None:
        outs.append(grads.new_empty((n, grads.shape[-1] if grads.dim() >= 2 else 1), dtype=torch.float32))
    return outs


@functools.lru_cache(maxsize=64)
def dedup_plan_bytes(n):
    size = ctypes.c_size_t(0)
    call("me_dedup_plan_size", n, ctypes.byref(size))
    return size.value


def dedup_keys(keys, key_bound):
    """[uniq [n], inv [n], count [1], plan (uint8)]: the key half of dedup -- torch.unique(keys,
    return_inverse=True) (micro_engram/rows.py:81) and the segment plan dedup_sums reads. Depends
    only on the keys, so it can run before the gradients exist."""
    dev = require_gpu(keys)
    keys = keys.reshape(-1).long().contiguous()
    n = keys.numel()
    ints = torch.empty(2 * n + 1, dtype=torch.int64, device=dev)  # three outputs, one allocation
    uniq, inv, count = ints[:n], ints[n:2 * n], ints[2 * n:]
    plan = torch.empty(max(dedup_plan_bytes(n), 16), dtype=torch.uint8, device=dev)
    ws = torch.empty(max(dedup_workspace_bytes(n), 16), dtype=torch.uint8, device=dev)
    call("me_dedup_keys", _p(keys), n, key_bound, _p(uniq), _p(inv), count.data_ptr(), plan.data_ptr(),
         plan.numel(), ws.data_ptr(), ws.numel(), stream_of(dev))
    return [uniq, inv, count, plan]


def dedup_table_bounds(uniq, count, offsets):
    """(local rows [n] int64, info [n_tables + 2] int64) of an ascending unique-key array over
    concatenated tables with the given host offsets (n_tables + 1, from 0): each unique key's row
    in its own table, and info = [count, first index of each table, ..., count] -- the
    searchsorted bounds of rows.py:123-129, in one launch."""
    dev = require_gpu(uniq, count)
    n = uniq.numel()
    out = torch.empty(n + len(offsets) + 1, dtype=torch.int64, device=dev)
    local, info = out[:n], out[n:]
    call("me_dedup_table_bounds", _p(uniq) if n else None, n, count.data_ptr(), i64_array(list(offsets)),
         len(offsets) - 1, _p(local) if n else None, info.data_ptr(), stream_of(dev))
    return local, info


def dedup_tables(idx2d, table_rows, inverse=True):
    """[uniq, local rows, inv, count, plan, info] of the token-major lookups of per-table row ids
    idx2d [n_tables, n] (key offset_k + idx2d[k, t] at position t * n_tables + k): what
    dedup_keys of those keys and dedup_table_bounds of its unique keys give (torch.unique of
    micro_engram/rows.py:81 and the table slices of rows.py:123-129), in two launches. count is
    info[:1]; info = [count, first unique index of each table, count]. inverse=False leaves inv
    unwritten (the segment sums do not read it) and saves its scattered writes."""
    dev = require_gpu(idx2d)
    if idx2d.dtype != torch.int64 or idx2d.stride(1) != 1:
        idx2d = idx2d.long().contiguous()
    nt, n = idx2d.shape
    N = n * nt
    rows = i64_array([int(r) for r in table_rows])
    ints = torch.empty(3 * N + nt + 2, dtype=torch.int64, device=dev)  # four outputs, one allocation
    uniq, local, inv, info = ints[:N], ints[N:2 * N], ints[2 * N:3 * N], ints[3 * N:]
    plan = torch.empty(max(dedup_plan_bytes(N), 16), dtype=torch.uint8, device=dev)
    size = ctypes.c_size_t(0)
    call("me_dedup_tables_workspace_size", n, nt, rows, ctypes.byref(size))
    ws = torch.empty(max(size.value, 16), dtype=torch.uint8, device=dev)
    call("me_dedup_tables", idx2d.data_ptr() if N else None, idx2d.stride(0) if n else 0, n, nt, rows,
         _p(uniq) if N else None, _p(local) if N else None, _p(inv) if N and inverse else None, info.data_ptr(),
         plan.data_ptr(), plan.numel(), ws.data_ptr(), ws.numel(), stream_of(dev))
    return [uniq, local, inv, info[:1], plan, info]


def dedup_sums(plan, count, grads):
    """fp32 [n, D]: row u = the index_add_ sum of the gradient rows of unique key u (rows.py:117-118),
    from the plan and count of dedup_keys on the same n keys; rows past the count are unset."""
    dev = require_gpu(plan, count, grads)
    n = grads.shape[0]
    grads = grads.reshape(n, grads.shape[-1] if grads.dim() >= 2 else 1)
    if grads.dtype not in (torch.float32, torch.bfloat16):
        grads = grads.float()
    grads = grads.contiguous()
    gsum = torch.empty((n, grads.shape[1]), dtype=torch.float32, device=dev)
    call("me_dedup_sums", plan.data_ptr(), plan.numel(), n, count.data_ptr(), grads.data_ptr(),
         dtype_code(grads), grads.shape[1], gsum.data_ptr(), stream_of(dev))
    return gsum


def sumsq(x, out=None, accumulate=False):
    """Sum of squares of an fp32 tensor into a device scalar (the squared gradient norm of
    RowTables.clip, micro_engram/rows.py:214-223)."""
    dev = require_gpu(x, out)
    x = x.reshape(-1).float().contiguous()
    if out is None:
        out = torch.zeros(1, dtype=torch.float32, device=dev)
    ws = torch.empty(1024, dtype=torch.uint8, device=dev)
    call("me_sumsq", _p(x), x.numel(), out.data_ptr(), int(accumulate), ws.data_ptr(), ws.numel(),
         stream_of(dev))
    return out


def clip_scale(x, sumsq, max_norm):
    """x *= min(max_norm / (sqrt(sumsq) + 1e-6), 1) in place, the scaling of RowTables.clip
    (micro_engram/rows.py:221-231); x fp32 or bf16 and contiguous, sumsq a device fp32 scalar.
    bf16 values are scaled by the coefficient rounded to bf16, as p.grad.mul_(coef.to(bf16))."""
    dev = require_gpu(x, sumsq)
    if not x.is_contiguous():
        raise ValueError("[micro_engram] clip_scale needs a contiguous tensor (it scales in place)")
    if x.data_ptr() % 16:
        raise ValueError("[micro_engram] clip_scale needs a 16-byte aligned tensor")
    if sumsq.dtype != torch.float32:
        raise ValueError("[micro_engram] clip_scale: sumsq must be fp32")
    call("me_clip_scale", x.data_ptr(), dtype_code(x), x.numel(), sumsq.data_ptr(), float(max_norm),
         stream_of(dev))
    return x


def sparse_adam(params, exp_avgs, exp_avg_sqs, rows, grads, steps, stream_ids, *, lr, betas, eps,
                weight_decay, rowwise, lazy, stochastic_rounding, seed):
    """One LazyAdamW step on the given rows of each table (micro_engram/optim.py:65-133), all
    tables in one launch. params/exp_avgs [rows_k, D]; exp_avg_sqs [rows_k] fp32 (row-wise) or
    like params; rows int64 [n_k] unique; grads fp32 [n_k, D]; steps: step counts after the
    increment. grads fp32, or all bf16. Updates the tensors in place."""
    dev = require_gpu(*params, *exp_avgs, *exp_avg_sqs, *rows, *grads)
    n = len(params)
    if not (len(exp_avgs) == len(exp_avg_sqs) == len(rows) == len(grads) == len(steps) == n):
        raise ValueError("[micro_engram] sparse_adam: per-table lists differ in length")
    if n == 0:
        return
    dim = params[0].shape[1]
    pdt = params[0].dtype
    f32, i64 = torch.float32, torch.int64
    gdt = grads[0].dtype if grads[0].dtype in (f32, torch.bfloat16) else f32
    # one pass: check every table's tensors (the kernel trusts these shapes) and collect the
    # pointers; rows and grads that are not contiguous are copied (kept alive in `held`)
    held, pp, mp, vp, rp, gp, counts = [], [], [], [], [], [], []
    for p, m, v, r, g in zip(params, exp_avgs, exp_avg_sqs, rows, grads):
        shape = p.shape
        if len(shape) != 2 or shape[1] != dim or p.dtype != pdt or not p.is_contiguous():
            raise ValueError("[micro_engram] sparse_adam: tables must be contiguous [rows, D] of one dtype")
        if m.shape != shape or m.dtype != pdt or not m.is_contiguous():
            raise ValueError("[micro_engram] sparse_adam: exp_avg must match its table")
        if (v.shape != ((shape[0],) if rowwise else shape) or not v.is_contiguous()
                or (rowwise and v.dtype != f32)):
            raise ValueError("[micro_engram] sparse_adam: exp_avg_sq has the wrong shape or dtype")
        k = r.numel()
        if r.dtype != i64 or g.dtype != gdt or g.shape != (k, dim):
            raise ValueError("[micro_engram] sparse_adam: rows must be int64 [n], grads fp32 (or all "
                             "bf16) [n, D]")
        if not r.is_contiguous():
            r = r.contiguous()
            held.append(r)
        if not g.is_contiguous():
            g = g.contiguous()
            held.append(g)
        pp.append(p.data_ptr())
        mp.append(m.data_ptr())
        vp.append(v.data_ptr())
        rp.append(r.data_ptr())
        gp.append(g.data_ptr())
        counts.append(k)
    sq_code = dtype_code(exp_avg_sqs[0]) if not rowwise else ME_F32
    sparse_adam_launch(dev, ptr_array(pp), ptr_array(mp), ptr_array(vp), n, dim, dtype_code(params[0]),
                       sq_code, ptr_array(rp), ptr_array(gp), i64_array(counts), steps, stream_ids,
                       lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, rowwise=rowwise, lazy=lazy,
                       stochastic_rounding=stochastic_rounding, seed=seed, grad_dtype=dtype_code(grads[0]))


def sparse_adam_launch(dev, param_ptrs, exp_avg_ptrs, exp_avg_sq_ptrs, n, dim, dtype, sq_dtype,
                       row_ptrs, grad_ptrs, counts, steps, stream_ids, *, lr, betas, eps, weight_decay,
                       rowwise, lazy, stochastic_rounding, seed, grad_dtype=ME_F32):
    """The launch of sparse_adam from pointer arrays (ctypes) that a caller has already checked
    against the tensors' shapes: n tables of [rows, dim] elements of `dtype`, their moments, and
    for each its `counts[k]` unique int64 rows and [counts[k], dim] gradient rows of grad_dtype
    (ME_F32 or ME_BF16); steps and stream_ids as lists or ready ctypes arrays. For callers that
    keep the arrays of tensors which stay put between steps (the optimizer)."""
    if not isinstance(steps, ctypes.Array):
        steps = i64_array([int(s) for s in steps])
    if not isinstance(stream_ids, ctypes.Array):
        stream_ids = i32_array([int(s) for s in stream_ids])
    call("me_sparse_adam", n, param_ptrs, exp_avg_ptrs, exp_avg_sq_ptrs, row_ptrs, grad_ptrs, grad_dtype, counts,
         steps, stream_ids, dim, dtype,
         int(bool(rowwise)), sq_dtype, int(bool(lazy)), float(lr), float(betas[0]), float(betas[1]),
         float(eps), float(weight_decay), int(bool(stochastic_rounding)), int(seed) & ((1 << 64) - 1),
         stream_of(dev))


def stochastic_bf16(x, seed, step=0, stream_id=0):
    """bf16 tensor like x: fp32 -> bf16 with stochastic rounding (micro_engram/optim.py:33-44);
    element i uses the noise of (row i // 4096, column i % 4096) of `stream_id` at `step`."""
    dev = require_gpu(x)
    xf = x.float().contiguous()
    out = torch.empty(xf.shape, dtype=torch.bfloat16, device=dev)
    call("me_stochastic_bf16", xf.data_ptr(), xf.numel(), out.data_ptr(),
         int(seed) & ((1 << 64) - 1), int(step) & 0xFFFFFFFF, int(stream_id), stream_of(dev))
    return out
