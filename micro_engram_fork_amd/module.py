"""MicroEngram for MI355X: the reference's module surface over the HIP kernels.

Drop-in for micro_engram.module.MicroEngram (micro_engram/module.py:26-283): the same
constructor, attributes (order_sizes, orders, _table_orders, table_rows, table_size), modules
(tables, key, value, q_scale, k_scale / down, up), buffers (mults, canon), state-dict names and
scale-as-delta conventions, and the same methods (hash_ids, hash_prev, lookup, inject, forward,
norm_scales, shard_rows, all_parameters, pop_gate_stats). The compute of hash_ids / hash_prev /
lookup / inject / forward runs in libmicro_engram_amd.so; tensors on the CPU raise instead of
taking any other path.

Differences from the reference, all deliberate:
  * forward() fuses hashing and the row gather into one kernel (the reference's hash_ids +
    lookup + cat), then one gate/residual op.
  * lookup() returns views into one concatenated [N, n_tables * D] buffer instead of separate
    tensors per table (same values).
  * Where a gradient is needed (grad mode on and hidden or a parameter requiring it), the
    forward keeps the memory vectors and per-token gate sums, and the backward runs the HIP
    gate backward (the projections recomputed on MFMA) plus four plain GEMMs for the weight and
    memory gradients; the table gradients go through the dedup kernel (rows.py). Without
    gradients, hashing and the gather run fused and nothing is kept.
  * The "ple" gate keeps its parameters (so checkpoints load) but has no HIP kernel.
"""

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from ._lib import ME_GATE_SCALAR, ME_GATE_SCALAR_SQRT, ME_MAX_ORDER, ME_MAX_TABLES

_PRIME = 2_147_483_647  # 2^31 - 1: the hash modulus (module.py:5)


def resolve_order_sizes(table_size, orders=(2, 3), table_sizes=None):
    """{order: rows per table}, sorted by order (module.py:8-23): every order in `orders` gets
    `table_size`; `table_sizes` overrides or adds orders (keys may be strings); 0/None drops."""
    sizes = {int(order): table_size for order in orders}
    for order, rows in (table_sizes or {}).items():
        sizes[int(order)] = rows
    resolved = {order: int(rows) for order, rows in sorted(sizes.items()) if rows}
    if not resolved:
        raise ValueError("micro_engram: every n-gram order has size 0/None: nothing left to hash")
    if min(resolved) < 1 or min(resolved.values()) < 1:
        raise ValueError(f"micro_engram: bad orders/sizes {resolved}")
    return resolved


def _row_range(n_rows, rank, world):
    """(first row, count) of `rank`'s share (micro_engram/rows.py:39-44)."""
    per = -(-n_rows // world)
    start = min(rank * per, n_rows)
    return start, max(0, min(per, n_rows - start))


class _RowIds(list):
    """The per-table row ids hash_ids / hash_prev return (a list of n_tables tensors, as the
    reference's), which are the rows of one [n_tables, N] tensor: it remembers that tensor, so
    the lookup can take it as it is while the list and the tensor are unchanged (the same
    element objects, no in-place write since: the views share the tensor's version counter).
    From hash_prev without gradients it also carries the rows read with the ids."""

    __slots__ = ("stacked", "views", "version", "rows")

    def __init__(self, stacked, rows=None):
        views = stacked.unbind(0)
        super().__init__(views)
        self.views = views
        self.stacked = stacked.reshape(len(views), -1)
        self.version = _version_of(stacked)
        self.rows = rows  # (memory vectors, their version, the tables' key) read with the ids

    def rows_for(self, tables):
        """The memory vectors read together with these ids, while the ids, the vectors and the
        tables (address, shape and version counter of each) are all as they were then."""
        rows = self.rows
        if (rows is None or not self.unchanged() or _version_of(rows[0]) != rows[1]
                or rows[2] != _tables_key(tables)):
            return None
        return rows[0]

    def unchanged(self):
        return (len(self) == len(self.views) and _version_of(self.stacked) == self.version
                and all(a is b for a, b in zip(self, self.views)))


def _version_of(t):
    """A tensor's version counter; None for an inference tensor, which keeps none."""
    return None if t.is_inference() else t._version


def _tables_key(tables):
    return tuple((t.data_ptr(), t.shape, _version_of(t)) for t in tables)


class _GateResidual(torch.autograd.Function):
    """hidden + the gated projection of the memory vectors (module.py:239-261) with its
    gradients: the HIP backward gives the gradients of hidden, of the key / value Linear
    outputs and of the scale deltas; the Linear layers' own gradients (dW = dY^T mem,
    dmem = dY_K W_K + dY_V W_V) come from _linear_grads."""

    @staticmethod
    def forward(ctx, hidden, mem, w_key, w_value, q_delta, k_delta, gate_mode, keep):
        out, alpha, stats = ops.gate_residual(
            hidden, mem, w_key.detach(), w_value.detach(),
            None if q_delta is None else q_delta.detach(),
            None if k_delta is None else k_delta.detach(), gate_mode, keep, True, True)
        ctx.save_for_backward(hidden, mem, w_key, w_value, q_delta, k_delta, keep, stats)
        ctx.gate_mode = gate_mode
        ctx.mark_non_differentiable(alpha)
        return out, alpha

    @staticmethod
    def backward(ctx, grad_out, _grad_alpha):
        hidden, mem, w_key, w_value, q_delta, k_delta, keep, stats = ctx.saved_tensors
        need = ctx.needs_input_grad
        wk, wv = w_key.detach(), w_value.detach()
        g_hidden, g_key, g_value, g_q, g_k = ops.gate_backward(
            grad_out.contiguous(), hidden.detach(), mem.detach(), wk, wv,
            None if q_delta is None else q_delta.detach(),
            None if k_delta is None else k_delta.detach(), ctx.gate_mode, keep, stats)
        d_mem, d_wk, d_wv = _linear_grads(g_key, g_value, mem.detach(), wk, wv, need[1:4])
        d_q = g_q.to(q_delta.dtype) if need[4] else None
        d_k = g_k.to(k_delta.dtype) if need[5] else None
        return g_hidden if need[0] else None, d_mem, d_wk, d_wv, d_q, d_k, None, None


def _linear_grads(g_key, g_value, mem, wk, wv, need):
    """Gradients of the key / value Linear layers from those of their outputs (autograd's
    nn.Linear backward for module.py:245, 254): d_mem = dK W_K + dV W_V and dW = dY^T mem, each
    None where `need` (mem, w_key, w_value) says so. bf16 shapes the hand-written MFMA kernel
    takes run on it (me_linear_grads); others on the library GEMMs."""
    if not any(need):
        return None, None, None
    n, M = g_key.shape[0], mem.shape[-1]
    m = mem.reshape(n, M)
    if ops.fits_linear_grads(n, g_key.shape[1], M, m.dtype) and wk.dtype == wv.dtype == g_key.dtype == m.dtype:
        d_mem, d_wk, d_wv = ops.linear_grads(g_key, g_value, m, wk, wv, *need)
        return (d_mem.reshape(mem.shape) if need[0] else None, d_wk if need[1] else None,
                d_wv if need[2] else None)
    d_mem = torch.addmm(g_key @ wk, g_value, wv).reshape(mem.shape) if need[0] else None
    d_wk = g_key.t() @ m if need[1] else None
    d_wv = g_value.t() @ m if need[2] else None
    return d_mem, d_wk, d_wv


class _GateResidualRows(torch.autograd.Function):
    """The same as _GateResidual for shapes the MFMA kernels do not take (model dim not a
    multiple of 8, memory rows not a multiple of 16 bytes): the key / value projections are the
    library GEMM of nn.Linear (module.py:245, 254), the gate, residual add and their backward the
    HIP row kernels (me_gate_rows, me_gate_rows_backward); K and V are kept for the backward."""

    @staticmethod
    def forward(ctx, hidden, mem, w_key, w_value, q_delta, k_delta, gate_mode, keep):
        m = mem.reshape(-1, mem.shape[-1])
        k = torch.nn.functional.linear(m, w_key.detach())
        v = torch.nn.functional.linear(m, w_value.detach())
        q = None if q_delta is None else q_delta.detach()
        kd = None if k_delta is None else k_delta.detach()
        out, alpha, stats = ops.gate_rows(hidden, k, v, q, kd, gate_mode, keep, True, True)
        ctx.save_for_backward(hidden, mem, w_key, w_value, q_delta, k_delta, keep, stats, k, v)
        ctx.gate_mode = gate_mode
        ctx.mark_non_differentiable(alpha)
        return out, alpha

    @staticmethod
    def backward(ctx, grad_out, _grad_alpha):
        hidden, mem, w_key, w_value, q_delta, k_delta, keep, stats, k, v = ctx.saved_tensors
        need = ctx.needs_input_grad
        wk, wv = w_key.detach(), w_value.detach()
        g_hidden, g_key, g_value, g_q, g_k = ops.gate_rows_backward(
            grad_out.contiguous(), hidden.detach(), k, v,
            None if q_delta is None else q_delta.detach(),
            None if k_delta is None else k_delta.detach(), ctx.gate_mode, keep, stats)
        d_mem, d_wk, d_wv = _linear_grads(g_key, g_value, mem.detach(), wk, wv, need[1:4])
        d_q = g_q.to(q_delta.dtype) if need[4] else None
        d_k = g_k.to(k_delta.dtype) if need[5] else None
        return g_hidden if need[0] else None, d_mem, d_wk, d_wv, d_q, d_k, None, None


class MicroEngram(nn.Module):
    """Hashed n-gram memory added to the residual stream (micro_engram/module.py:26-47).

    At position t the n-grams ending at t (orders in `orders`, `num_heads` hash functions
    each) index per-(order, head) tables; the concatenated rows e feed a key/value projection,
    and a scalar gate from rms(h) . rms(W_K e) decides how much of W_V e to add to h."""

    GATES = ("scalar", "ple", "scalar_sqrt")
    SCALAR_GATES = ("scalar", "scalar_sqrt")
    DELTA_SCALES = ("q_scale", "k_scale")

    row_shards = None     # per-table row shards (shard_rows), outside parameters()
    row_info = None       # (rank, world, first row per table, rows per rank per table)
    row_lookup_fn = None  # a server's own lookup for row-sharded tables

    def __init__(self, model_dim, table_size=65_536, engram_dim=128, num_heads=4, orders=(2, 3),
                 pad_id=0, seed=0, vocab_size=262_144, canon=None, gate="scalar",
                 build_tables=True, table_sizes=None):
        super().__init__()
        if gate not in self.GATES:
            raise ValueError(f"gate must be one of {self.GATES}, got {gate!r}")
        self.gate = gate
        self.order_sizes = resolve_order_sizes(table_size, orders, table_sizes)
        self.orders = tuple(self.order_sizes)
        self.engram_dim = engram_dim
        self.seed = seed
        self.pad_id = pad_id
        # table k: order-major, head-minor (module.py:65-66)
        self._table_orders = [order for order in self.orders for _ in range(num_heads)]
        self.table_rows = [self.order_sizes[order] for order in self._table_orders]
        self.table_size = self.table_rows[0] if len(set(self.table_rows)) == 1 else None
        n_tables = len(self._table_orders)
        if n_tables > ME_MAX_TABLES or max(self.orders) > ME_MAX_ORDER:
            raise ValueError(f"[micro_engram] {n_tables} tables / order {max(self.orders)}: the HIP "
                             f"kernels take at most {ME_MAX_TABLES} tables and order {ME_MAX_ORDER}")

        if build_tables:
            self.tables = nn.ModuleList(nn.Embedding(rows, engram_dim) for rows in self.table_rows)
            for table in self.tables:
                nn.init.normal_(table.weight, std=0.02)

        mem_dim = engram_dim * n_tables
        if gate in self.SCALAR_GATES:
            self.key = nn.Linear(mem_dim, model_dim, bias=False)
            self.value = nn.Linear(mem_dim, model_dim, bias=False)
            nn.init.zeros_(self.value.weight)  # an untrained engram adds exactly nothing
            if gate == "scalar_sqrt":
                # stored as scale - 1 (module.py:81-87): bf16 cannot move 1.0 by an Adam step
                self.q_scale = nn.Parameter(torch.zeros(model_dim))
                self.k_scale = nn.Parameter(torch.zeros(model_dim))
        else:
            self.down = nn.Linear(model_dim, mem_dim, bias=False)
            self.up = nn.Linear(mem_dim, model_dim, bias=False)
            nn.init.zeros_(self.up.weight)

        # Hash multipliers from torch's CPU generator, exactly as the reference draws them
        # (module.py:93-99): the seed alone decides every row address.
        gen = torch.Generator().manual_seed(seed)
        mults = torch.randint(1, _PRIME, (n_tables, max(self.orders)), generator=gen,
                              device="cpu") | 1
        self.register_buffer("mults", mults)

        if canon is None:
            canon = torch.arange(vocab_size)
        else:
            canon = torch.as_tensor(canon).long().clone()
            if canon.shape != (vocab_size,):
                raise ValueError(f"canon must have shape ({vocab_size},), got {tuple(canon.shape)}")
        self.register_buffer("canon", canon)

    # ------------------------------------------------------------------ row shards (world = 1)
    def shard_rows(self, rank, world, device=None, dtype=None, requires_grad=True, empty=False,
                   pin_memory=False):
        """Keep only `rank`'s rows of every table (module.py:115-138). On one GPU (world 1) this
        is every row; the HIP lookup serves it directly. More ranks need the row exchange of
        micro_engram/rows.py, which this package does not provide."""
        spans = [_row_range(rows, rank, world) for rows in self.table_rows]
        pers = [-(-rows // world) for rows in self.table_rows]
        if "tables" in self._modules:
            src = [t.weight.detach()[a:a + c] for t, (a, c) in zip(self.tables, spans)]
            dtype = dtype or src[0].dtype
            del self.tables
        elif empty:
            pin = pin_memory and torch.cuda.is_available()
            src = [torch.empty(c, self.engram_dim, device=device, dtype=dtype, pin_memory=pin)
                   for _, c in spans]
        else:
            gen = torch.Generator().manual_seed(self.seed * 1_000_003 + rank)
            src = [torch.randn(c, self.engram_dim, generator=gen) * 0.02 for _, c in spans]
        shards = [nn.Parameter(t if empty else t.to(device=device, dtype=dtype).clone(),
                               requires_grad=requires_grad) for t in src]
        self.__dict__["row_shards"] = shards
        self.__dict__["row_info"] = (rank, world, [a for a, _ in spans], pers)
        return shards

    def all_parameters(self):
        return list(self.parameters()) + list(self.row_shards or [])

    def _table_weights(self):
        """The full tables as [rows, D] tensors (module tables or world-1 row shards)."""
        if self.row_shards is not None:
            rank, world = self.row_info[0], self.row_info[1]
            if world != 1:
                raise NotImplementedError(
                    f"[micro_engram] row-sharded tables over {world} ranks need the multi-GPU row "
                    "exchange, which this single-GPU build does not provide")
            return [s.detach() for s in self.row_shards]
        return [t.weight.detach() for t in self.tables]

    # ---------------------------------------------------------------- scales stored as deltas
    def norm_scales(self):
        """(q scale, k scale) in fp32: 1 + delta, the delta made fp32 first (module.py:161-164)."""
        return 1 + self.q_scale.float(), 1 + self.k_scale.float()

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        for name in self.DELTA_SCALES:
            key = prefix + name
            if key in destination:  # files hold the scale itself, in fp32 (module.py:166-172)
                destination[key] = destination[key].detach().float() + 1

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        for name in self.DELTA_SCALES:
            key = prefix + name
            if key in state_dict:
                state_dict[key] = state_dict[key].float() - 1
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    # ------------------------------------------------------------------------------- hashing
    def _hash_consts(self, device):
        """(canon, mults, False): the kernels read the canon map on every call, as module.py:186 and 216
        index it. (The ops' identity flag skips that read for a caller that vouches for an
        identity map; measured on the Gemma-scale prefill it saves 0.1-0.35 us of a 12.4 us
        gather, too little to trust a buffer that writes through .data can change unseen.)"""
        canon = self.canon if self.canon.device == device else self.canon.to(device)
        mults = self.mults if self.mults.device == device else self.mults.to(device)
        return canon, mults, False

    def hash_ids(self, input_ids, position_ids=None):
        """Row ids of the n-grams ending at every position: list of n_tables LongTensors shaped
        like input_ids [B, T] (module.py:183-205)."""
        canon, mults, ident = self._hash_consts(input_ids.device)
        pos = position_ids.to(input_ids.device) if position_ids is not None else None
        idx = ops.hash_ids(input_ids, pos, canon, mults, self._table_orders, self.table_rows,
                           int(self.pad_id), ident)
        return list(idx.unbind(0)) if torch.compiler.is_compiling() else _RowIds(idx)

    def hash_prev(self, ids):
        """Row ids from [N, W] ids of each token and its predecessors, -1 where missing: list of
        n_tables LongTensors [N] (module.py:207-226).

        Without gradients (serving) the rows are read in the same launch (me_hash_prev_gather:
        one kernel where hashing and gathering apart take two) and travel with the returned list,
        so that the next inject on it reads no rows again -- while the list, the tables and (for
        tensors made outside inference mode) the ids and rows are unchanged: version counters
        see in-place writes through the tensors, the optimizers' updates included, not writes
        through .data; ids made under inference_mode keep no counter, so an in-place write to
        them before the inject is not seen. lookup hands the rows out and drops them."""
        canon, mults, ident = self._hash_consts(ids.device)
        if not torch.compiler.is_compiling() and self._reads_rows_with_ids():
            tables = self._table_weights()
            key = _tables_key(tables)
            if all(k[2] is not None for k in key):
                mem, idx = ops.hash_prev_gather(ids, canon, mults, self._table_orders, self.table_rows,
                                                int(self.pad_id), tables, True, ident)
                return _RowIds(idx, (mem, _version_of(mem), key))
        idx = ops.hash_prev(ids, canon, mults, self._table_orders, self.table_rows,
                            int(self.pad_id), ident)
        return list(idx.unbind(0)) if torch.compiler.is_compiling() else _RowIds(idx)

    def _reads_rows_with_ids(self):
        """Whether hash_prev reads the rows with the ids: no gradients, the module's own lookup,
        tables of this module (not a row server's)."""
        return (not torch.is_grad_enabled() and not self._lookup_replaced()
                and not (self.row_lookup_fn is not None and self.row_shards is not None)
                and (self.row_shards is not None or "tables" in self._modules))

    # -------------------------------------------------------------------------------- lookup
    @staticmethod
    def _stacked_idx(idx):
        """[n_tables, N] int64 view of the per-table ids: no copy when they are the rows of one
        buffer (what hash_ids / hash_prev return), else a stacked copy. Under torch.compile the
        stack is what gets traced (storage addresses are not traceable); the compiler sees the
        unbind of one buffer followed by its stack."""
        if torch.compiler.is_compiling():
            return torch.stack([i.reshape(-1).long() for i in idx])
        if isinstance(idx, _RowIds) and idx.unchanged():
            return idx.stacked
        first = idx[0]
        n = first.numel()
        storage = first.untyped_storage().data_ptr()
        if all(i.dtype == torch.int64 and i.is_contiguous() and i.numel() == n
               and i.untyped_storage().data_ptr() == storage for i in idx):
            if len(idx) == 1:
                return first.reshape(1, n)
            step = idx[1].data_ptr() - first.data_ptr()
            if step % 8 == 0 and step // 8 >= n and all(
                    i.data_ptr() - first.data_ptr() == k * step for k, i in enumerate(idx)):
                return first.reshape(-1).as_strided((len(idx), n), (step // 8, 1))
        return torch.stack([i.reshape(-1).long() for i in idx])

    def _served_memory(self, idx):
        """The memory vectors [N, n_tables * D] through the installed row_lookup_fn: straight
        from its concatenated buffer when it offers one (this package's tp_lookup), else the
        concatenation of its per-table rows (module.py:149-150, 233)."""
        fn = self.row_lookup_fn
        memory = getattr(fn, "memory", None)
        if memory is not None:
            return memory(self, idx)
        return torch.cat(fn(self, idx), dim=-1).reshape(idx[0].numel(), -1)

    def _mem(self, idx, hand_out=False):
        if self.row_lookup_fn is not None and self.row_shards is not None:
            return self._served_memory(idx)
        tables = self._table_weights()
        if isinstance(idx, _RowIds) and idx.rows is not None:
            mem = idx.rows_for(tables)
            if hand_out:  # views of the rows leave the module: no later read may trust them
                idx.rows = None
            if mem is not None:  # read together with the ids by hash_prev
                return mem
        return ops.gather(self._stacked_idx(idx), tables)

    def _mem_grad(self, idx):
        """The memory vectors [N, n_tables * D] with the tables' gradients attached: the row
        lookup of rows.py (dense table gradients, or sparse ones for row shards so marked)."""
        if self.row_shards is not None:
            if self.row_lookup_fn is not None:
                return self._served_memory(idx)
            rank, world = self.row_info[0], self.row_info[1]
            if world != 1:
                raise NotImplementedError(
                    f"[micro_engram] row-sharded tables over {world} ranks need the multi-GPU row "
                    "exchange, which this single-GPU build does not provide")
            weights = list(self.row_shards)
        else:
            weights = [t.weight for t in self.tables]
        from .rows import _RowLookup, _table_offsets

        return _RowLookup.apply(self._stacked_idx(idx), _table_offsets(self), *weights)

    def lookup(self, idx):
        """The table rows for the hashed ids: list of n_tables tensors [*idx shape, D]
        (module.py:146-154). Row-sharded tables go through the server's lookup or the
        differentiable row lookup (sparse row gradients, micro_engram/rows.py:150-161). Plain
        tables carry their gradients when grad mode is on and a table requires one, as
        nn.Embedding does (the row lookup: dense table gradients through the dedup kernels)."""
        if self.row_shards is not None:
            if self.row_lookup_fn is not None:
                return self.row_lookup_fn(self, idx)
            from .rows import row_lookup

            return row_lookup(self, idx)
        shape = tuple(idx[0].shape)
        if torch.is_grad_enabled() and any(t.weight.requires_grad for t in self.tables):
            mem = self._mem_grad(idx)
        else:
            mem = self._mem(idx, hand_out=True)
        D = self.engram_dim
        return [mem[:, k * D:(k + 1) * D].reshape(*shape, D) for k in range(len(idx))]

    def _lookup_replaced(self):
        """True when `lookup` is not this class's own: set on the instance (as the reference's
        tests do, test_zero_order.py:84-88) or overridden by a subclass. inject and forward then
        read the rows through it, as module.py:233 does."""
        return "lookup" in self.__dict__ or type(self).lookup is not MicroEngram.lookup

    # -------------------------------------------------------------------------------- inject
    def _needs_grad(self, hidden):
        return torch.is_grad_enabled() and (hidden.requires_grad or any(
            p.requires_grad for p in self.all_parameters()))

    def _gate(self, hidden, mem, keep):
        if self.gate not in self.SCALAR_GATES:
            raise NotImplementedError("[micro_engram] the 'ple' gate has no HIP kernel")
        reader = self.key.weight
        if mem.dtype != reader.dtype:
            mem = mem.to(reader.dtype)  # rows stored in another dtype (module.py:234-238)
        sqrt = self.gate == "scalar_sqrt"
        mode = ME_GATE_SCALAR_SQRT if sqrt else ME_GATE_SCALAR
        fits = ops.fits_mfma(hidden.shape[-1], mem.shape[-1], mem.dtype)
        if self._needs_grad(hidden) or mem.requires_grad:
            fn = _GateResidual if fits else _GateResidualRows
            out, alpha = fn.apply(hidden, mem, self.key.weight, self.value.weight,
                                  self.q_scale if sqrt else None, self.k_scale if sqrt else None,
                                  mode, keep)
            if self.training:
                self._record_gate(alpha)
            return out
        q = self.q_scale.detach() if sqrt else None
        k = self.k_scale.detach() if sqrt else None
        if not fits:  # any width: library GEMMs for K and V, then the row kernel
            m = mem.reshape(-1, mem.shape[-1])
            outs = ops.gate_rows(hidden, F.linear(m, self.key.weight.detach()),
                                 F.linear(m, self.value.weight.detach()), q, k, mode, keep,
                                 self.training)
            if self.training:
                self._record_gate(outs[1])
            return outs[0]
        n_tok = hidden.numel() // hidden.shape[-1]
        if mem.dtype == torch.bfloat16:
            limit = self.few_tokens_max
        else:  # also bounded by the fp32 K|V rows the few-token path writes ([N, 2d])
            limit = min(self.few_tokens_max_fp32, self.few_tokens_kv_bytes // (8 * hidden.shape[-1]))
        if n_tok <= limit:
            outs = ops.gate_residual_rows(hidden, mem, self.key.weight.detach(), self.value.weight.detach(),
                                          q, k, mode, keep, self.training)
        else:
            outs = ops.gate_residual(hidden, mem, self.key.weight.detach(), self.value.weight.detach(),
                                     q, k, mode, keep, self.training)
        if self.training:
            self._record_gate(outs[1])
        return outs[0]

    # Token counts up to which the gate without gradients runs the key and value projections
    # in the few-token kernel (me_kv_proj) and the gate in the row kernel (me_gate_rows) instead
    # of the fused kernel, whose 256-token tiles come in whole rounds of the CUs and leave many
    # of them idle below the last round. Measured on MI355X (model dim 5376, memory dim 1536,
    # bf16): 256 tokens 33 us against 73, 1024 tokens 61 against 74, 1536 tokens 88 against 76.
    # fp32 engrams: the fused kernel's fp32 tiles are 256 x 256 on 32x32x2 MFMAs, so a 2048-token
    # batch (model dim 1024) gives it 32 tiles per pass (538 us) and the few-token path (72 us for
    # the projection) stays ahead far longer. That range was measured at model dim 1024 only, so
    # for fp32 the token count is also capped by the bytes of the [N, 2d] fp32 K|V rows the
    # few-token path writes: 128 MiB, i.e. 16384 tokens at model dim 1024, 3120 at 5376.
    few_tokens_max = 1024
    few_tokens_max_fp32 = 16384
    few_tokens_kv_bytes = 128 << 20

    def inject(self, hidden, idx, keep=None):
        """hidden + gated memory of the rows `idx` (module.py:228-261); keep: optional [N] bool,
        False leaves that token unchanged. Returns a new tensor."""
        if self._lookup_replaced():
            rows = self.lookup(idx)
            mem = torch.cat(rows, dim=-1)
            return self._gate(hidden, mem.reshape(-1, mem.shape[-1]), keep)
        if not self._needs_grad(hidden):
            return self._gate(hidden, self._mem(idx), keep)
        from .rows import key_plans_after

        with key_plans_after():  # the row dedup's key plan is issued behind the gate
            return self._gate(hidden, self._mem_grad(idx), keep)

    def forward(self, hidden, input_ids, position_ids=None):
        """inject(hidden, hash_ids(input_ids, position_ids)) (module.py:263-265); without
        gradients the hashing and the gather run as one fused kernel (unless `lookup` has been
        replaced, which then reads the rows)."""
        if (self._needs_grad(hidden) or self._lookup_replaced()
                or (self.row_lookup_fn is not None and self.row_shards is not None)):
            return self.inject(hidden, self.hash_ids(input_ids.to(hidden.device), position_ids))
        return self._gate(hidden, self.hashed_memory(input_ids, position_ids, hidden.device), None)

    def hashed_memory(self, input_ids, position_ids=None, device=None):
        """The concatenated memory vectors [B*T, n_tables * D] of every position: hash_ids +
        lookup + cat (module.py:183-205, 146-154, 233) as one fused kernel."""
        device = device or input_ids.device
        input_ids = input_ids.to(device)
        canon, mults, ident = self._hash_consts(device)
        pos = position_ids.to(device) if position_ids is not None else None
        return ops.hash_gather(input_ids, pos, canon, mults, self._table_orders, self.table_rows,
                               int(self.pad_id), self._table_weights(), False, ident)[0]

    def gate_residual(self, hidden, mem, keep=None):
        """hidden + the gated projection of the memory vectors `mem` (module.py:239-261)."""
        return self._gate(hidden, mem, keep)

    # ------------------------------------------------------------------------- gate statistics
    # gate tensors kept before they are folded into the running sums
    _GATE_KEEP = 32

    def _record_gate(self, alpha):
        """Records the step's gates for (sum of alpha, count, count of alpha > 0.99)
        (module.py:268-274): the tensor is kept and reduced on the device when pop_gate_stats
        reads the sums or every _GATE_KEEP records, so a training forward -- whose host issue
        time bounds it -- pays no launches for it; no host sync either way."""
        pending = self.__dict__.setdefault("_gate_pending", [])
        a = alpha.detach()
        if pending and pending[0].device != a.device:
            self._fold_gate_stats()
        pending.append(a)
        if len(pending) >= self._GATE_KEEP:
            self._fold_gate_stats()

    def _fold_gate_stats(self):
        pending = self.__dict__.get("_gate_pending")
        if not pending:
            return
        a = torch.cat([t.reshape(-1).float() for t in pending])
        pending.clear()
        stats = getattr(self, "_gate_stats", None)
        if stats is None or stats.device != a.device:
            stats = torch.zeros(3, device=a.device)
        self._gate_stats = stats + torch.stack([a.sum(), a.new_full((), float(a.numel())),
                                                (a > 0.99).float().sum()])

    def pop_gate_stats(self):
        """(mean gate, fraction of tokens with gate > 0.99) since the last call, or None."""
        self._fold_gate_stats()
        stats = getattr(self, "_gate_stats", None)
        self._gate_stats = None
        if stats is None or stats[1] == 0:
            return None
        s, n, sat = stats.tolist()
        return s / n, sat / n


def engram_from_spec(spec, model_dim, vocab_size, pad_default=0, canon=None, build_tables=True):
    """A MicroEngram from one engram spec dict (module.py:299-315); the seed decides every hash
    address, so it is taken from the spec."""
    return MicroEngram(
        model_dim=model_dim,
        table_size=spec["table_size"],
        table_sizes=spec.get("table_sizes"),
        engram_dim=spec["engram_dim"],
        num_heads=spec["num_heads"],
        orders=tuple(spec.get("orders") or (2, 3)),
        pad_id=spec["pad_id"] if spec.get("pad_id") is not None else pad_default,
        seed=spec.get("seed") or 0,
        vocab_size=vocab_size,
        canon=canon,
        gate=spec.get("gate") or "scalar",
        build_tables=build_tables,
    )


def check_loaded(engram, sd, where):
    """Load `sd` into `engram`, refusing multipliers that differ from the seed's
    (module.py:318-328)."""
    if "mults" in sd and not torch.equal(sd["mults"].to(engram.mults.device).long(), engram.mults.long()):
        raise ValueError(f"[micro_engram] {where}: the saved hash multipliers differ from the ones "
                         f"this engram's seed gives; the seed is wrong for these weights")
    result = engram.load_state_dict(sd, strict=False)
    problems = [k for k in result.missing_keys if k != "mults"] + list(result.unexpected_keys)
    if problems:
        raise ValueError(f"[micro_engram] {where} does not match the engram settings: {problems[:10]}")
    return result


SEED_STRIDE = 10007  # default seed of the engram at layer L is SEED_STRIDE * L (weights.py:157)


def default_seed(layer):
    return SEED_STRIDE * int(layer)


# ------------------------------------------------------------------- attaching to a model
def find_text_layers(model):
    """(name, ModuleList) of the text decoder's layers (module.py:286-296): among the
    ModuleLists whose name ends in "layers", the language model's if there is one, else the
    first that belongs to neither a vision nor an audio tower."""
    lists = [(name, mod) for name, mod in model.named_modules()
             if isinstance(mod, nn.ModuleList) and name.endswith("layers")]
    for name, mod in lists:
        if "language_model" in name:
            return name, mod
    for name, mod in lists:
        if "vision" not in name and "audio" not in name:
            return name, mod
    raise RuntimeError("[micro_engram] no text decoder layers found in the model; print(model) and "
                       "pass the layer list yourself")


# parameter classes of bitsandbytes whose dtype is a packed storage type, not the compute type
_PACKED_PARAMS = ("Params4bit", "Int8Params")


def layer_device_dtype(layer):
    """(device, compute dtype) an engram placed in `layer` should take (module.py:334-352): the
    first floating-point parameter that is not a packed quantized weight, else a submodule's
    `compute_dtype`, else bf16 on the first parameter's device."""
    params = list(layer.parameters())
    if not params:
        raise RuntimeError("[micro_engram] the decoder layer has no parameters")
    for p in params:
        if p.is_floating_point() and type(p).__name__ not in _PACKED_PARAMS:
            return p.device, p.dtype
    for mod in layer.modules():
        dtype = getattr(mod, "compute_dtype", None)
        if isinstance(dtype, torch.dtype) and dtype.is_floating_point:
            return params[0].device, dtype
    return params[0].device, torch.bfloat16


def attach_engram(model, engram, layer_idx, dtype=None, get_ids=None):
    """Place `engram` inside decoder layer `layer_idx` as its submodule `micro_engram` and add its
    memory to the layer's output with a forward hook (module.py:355-393), so sharding,
    offloading and checkpointing of that layer carry the engram with it.

    The engram moves to the layer's device, in `dtype` or the layer's compute dtype (integer
    buffers keep theirs). get_ids: a callable returning (input_ids, position_ids) for the
    current forward; without it a pre-hook on `model` takes them from its forward's arguments
    (keyword `input_ids` / `position_ids`, or the first positional argument). Returns the
    layer's name and the hook handles."""
    name, layers = find_text_layers(model)
    layer = layers[layer_idx]
    device, layer_dtype = layer_device_dtype(layer)
    engram.to(device=device, dtype=dtype or layer_dtype)
    layer.add_module("micro_engram", engram)
    seen = {}

    def remember_ids(_module, args, kwargs):
        ids = kwargs.get("input_ids")
        if ids is None and args:
            ids = args[0]
        seen["input_ids"] = ids
        seen["position_ids"] = kwargs.get("position_ids")

    def add_memory(_module, _args, output):
        if get_ids is not None:
            ids, pos = get_ids()
        else:
            ids, pos = seen.get("input_ids"), seen.get("position_ids")
        if ids is None:
            return output
        if isinstance(output, tuple):
            return (engram(output[0], ids, pos), *output[1:])
        return engram(output, ids, pos)

    handles = [layer.register_forward_hook(add_memory)]
    if get_ids is None:
        handles.append(model.register_forward_pre_hook(remember_ids, with_kwargs=True))
    return f"{name}.{layer_idx}", handles
