"""Row tables on one GPU: touched-row dedup, coalesced sparse gradients, clipping and the row
optimizer (the surface of micro_engram/rows.py at world size 1).

With one GPU every table is whole in HBM, so the reference's all_to_all row exchange
(rows.py:57-134) reduces to: gather the rows, and in the backward sum the gradient rows of
equal (table, row) keys -- torch.unique + index_add_ in the reference (rows.py:81, 117-118),
the radix-sort dedup kernel here (bit-exact: same unique keys, inverse and fp32 sums) -- and
keep them per table as p.sparse_grad = (unique rows, fp32 sums) (rows.py:137-147). More than one
rank needs that exchange, which this single-GPU build does not provide; it raises.
"""
import contextlib
import os
import threading

import torch

from . import ops
from .optim import LazyAdamW, SparseBatch

ROWS_DIR = "micro_engram_rows"              # complete engram (tables + the rest), DCP (rows.py:27)
ROWS_OPTIM_DIR = "micro_engram_rows_optim"  # the tables' optimizer state, DCP (rows.py:28)


def row_range(n_rows, rank, world):
    """(first row, row count) owned by `rank`: ceil(n / world) rows each (rows.py:39-44)."""
    per = -(-n_rows // world)
    start = min(rank * per, n_rows)
    return start, max(0, min(per, n_rows - start))


def dedup_rows(keys, key_bound, grads=None):
    """(unique keys ascending, inverse, fp32 sums of `grads` per unique key) -- torch.unique(
    return_inverse=True) + zeros().index_add_(0, inv, grads.float()) (rows.py:81, 117-118),
    bit-exact. Reads the unique count back to the host (the reference syncs here too,
    rows.py:92)."""
    outs = ops.dedup(keys, int(key_bound), grads)
    n = int(outs[2].item())
    uniq, inv = outs[0][:n], outs[1]
    return (uniq, inv, outs[3][:n]) if grads is not None else (uniq, inv, None)


def add_sparse_grad(p, rows, g):
    """Add gradient rows `g` [n, dim] for local rows `rows` to p.sparse_grad, kept coalesced:
    (unique rows, their fp32 sums), the previous entries first (rows.py:137-147)."""
    cur = getattr(p, "sparse_grad", None)
    if cur is not None:
        rows, g = torch.cat([cur[0], rows]), torch.cat([cur[1], g])
    u, _, acc = dedup_rows(rows.long(), p.shape[0], g.float())
    p.sparse_grad = (u, acc)


def _spans(tensors):
    """The tensors as few 1-D fp32 views: consecutive contiguous fp32 tensors that tile one
    buffer in order (the row lookup's backward leaves every table's sparse gradient as the next
    slice of one dedup output) merge into one view, so one reduction launch covers them."""
    spans = []
    for t in tensors:
        if t.dtype == torch.float32 and t.is_contiguous() and spans:
            last = spans[-1]
            if (last.dtype == torch.float32 and last.dim() == 1 and last.is_contiguous() and
                    last.untyped_storage().data_ptr() == t.untyped_storage().data_ptr() and
                    last.data_ptr() + last.numel() * 4 == t.data_ptr()):
                spans[-1] = last.as_strided((last.numel() + t.numel(),), (1,), last.storage_offset())
                continue
        spans.append(t.reshape(-1) if t.is_contiguous() else t)
    return spans


def _table_offsets(engram):
    offs = [0]
    for rows in engram.table_rows:
        offs.append(offs[-1] + rows)
    return offs


_OFFSETS_ON = {}


def _offsets_on(offsets, device):
    """The table offsets as an int64 tensor on `device`, made once per (offsets, device): a
    tensor built from a host list per backward is a host-to-device copy on every step."""
    key = (tuple(offsets), device)
    t = _OFFSETS_ON.get(key)
    if t is None:
        t = _OFFSETS_ON[key] = torch.tensor(offsets, dtype=torch.int64, device=device)
    return t


def _lookup_keys(idx2d, offs):
    """Token-major keys of the lookups: lookup i*nt + k is (token i, table k), whose gradient
    row is grad[i, k*D:(k+1)*D]; equal keys share a table, so within a key this is token order,
    the order of the reference's table-major flattening. One launch: the sum is written
    straight into the token-major buffer."""
    nt, n = idx2d.shape
    keys = torch.empty(n * nt, dtype=torch.int64, device=idx2d.device)
    torch.add(idx2d.t(), offs, out=keys.view(n, nt))
    return keys


class _KeyPlan:
    """The key half of a row lookup's dedup (unique keys, inverse, segment plan; torch.unique of
    rows.py:81) and the tables' bounds in it, made once: at the lookup, or when the launches
    issued after it are out (key_plans_after). The bounds go to pinned host memory by an
    asynchronous copy with an event behind it, so the backward's host read waits for the plan
    only, not for the gate's backward and the weight products queued before it."""

    def __init__(self, idx2d, offsets):
        self.idx2d, self.offsets, self.outs = idx2d, offsets, None

    def make(self):
        if self.outs is None:
            rows = [b - a for a, b in zip(self.offsets, self.offsets[1:])]
            uniq, self.local_all, inv, count, plan, info = ops.dedup_tables(self.idx2d, rows, inverse=False)
            self.outs = [uniq, inv, count, plan]  # inv unwritten: the segment sums read the plan
            self.host = _pinned_take(info.numel())
            self.host.copy_(info, non_blocking=True)
            self.ready = torch.cuda.Event()
            self.ready.record(torch.cuda.current_stream(info.device))  # the copy's stream
            self.idx2d = None
        return self.outs

    def bounds(self):
        """(local rows of the unique keys, [count, table bounds] as host ints)."""
        self.make()
        self.ready.synchronize()
        buf, self.host = self.host, None
        host = buf.tolist()
        _pinned_give(buf)  # its copy is done and read (a plan that is never read keeps its own)
        return self.local_all, host


_PINNED = {}


def _pinned_take(n):
    """A pinned int64 host buffer of n values from the pool (allocating pinned memory is a
    host-allocator call on every step otherwise)."""
    free = _PINNED.get(n)
    return free.pop() if free else torch.empty(n, dtype=torch.int64, pin_memory=True)


def _pinned_give(t):
    free = _PINNED.setdefault(t.numel(), [])
    if len(free) < 8:
        free.append(t)


_PLANS = threading.local()


@contextlib.contextmanager
def key_plans_after():
    """Row lookups inside the block leave their key plans to the block's end, so that the host
    issues them after the launches that follow the lookup (the gate): the training forward is
    bound by the host's issue rate, and the plan's host work then overlaps the gate on the GPU.
    On an exception the plans are left to the backward."""
    outer = getattr(_PLANS, "pending", None)
    _PLANS.pending = pending = []
    try:
        yield
    finally:
        _PLANS.pending = outer
    for plan in pending:
        plan.make()


class _RowLookup(torch.autograd.Function):
    """Per-table rows for hashed ids, world size 1. Backward: the gradient rows of every lookup
    are deduplicated over (table, row) and added to each shard's sparse gradient (shards marked
    _sparse_rows) or to a dense gradient (rows.py:71-134).

    The dedup's key half (unique keys, inverse and the segment plan; torch.unique of
    rows.py:81) depends only on the row ids, so when a table needs its gradient the forward
    makes it (after the gate's launches inside key_plans_after) and the backward runs only the
    segment sums (rows.py:117-118). (On a second stream beside the gate it ran slower: a gate
    tile holds a whole CU's LDS, so a dedup workgroup taking a CU between two rounds of gate
    tiles delays the next round.)"""

    @staticmethod
    def forward(ctx, idx2d, offsets, *shards):
        mem = ops.gather(idx2d, list(shards))  # no graph is recorded inside forward
        ctx.save_for_backward(idx2d)
        ctx.offsets = offsets
        ctx.shapes = [(s.shape, s.dtype) for s in shards]
        ctx.shards = shards if any(getattr(s, "_sparse_rows", False) for s in shards) else None
        ctx.plan = None
        if any(ctx.needs_input_grad[2:]) and idx2d.numel() > 0:
            ctx.plan = _KeyPlan(idx2d, offsets)
            pending = getattr(_PLANS, "pending", None)
            if pending is None:
                ctx.plan.make()
            else:
                pending.append(ctx.plan)
        return mem

    @staticmethod
    def backward(ctx, grad):
        (idx2d,) = ctx.saved_tensors
        nt, n = idx2d.shape
        D = ctx.shapes[0][0][1]
        offs_all = _offsets_on(ctx.offsets, idx2d.device)
        offs = offs_all[:-1]
        if ctx.plan is not None:  # the key half and the bounds ran in the forward
            uniq_all, inv, count, plan = ctx.plan.make()
            outs = [uniq_all, inv, count, ops.dedup_sums(plan, count, grad.reshape(n * nt, D))]
            local_all, host = ctx.plan.bounds()
            ctx.plan = None
        else:
            outs = ops.dedup(_lookup_keys(idx2d, offs), int(ctx.offsets[-1]), grad.reshape(n * nt, D))
            # one host read for the unique count and every table's bounds
            local_all, info = ops.dedup_table_bounds(outs[0], outs[2], ctx.offsets)
            host = info.tolist()
        cnt, bounds = host[0], host[1:]
        # each table's slice of the unique rows and sums (bounds[0] = 0, bounds[nt] = count)
        sizes = [bounds[k + 1] - bounds[k] for k in range(nt)]
        locals_ = local_all[:cnt].split(sizes)
        sums = outs[3][:cnt].split(sizes)
        batch = SparseBatch(local_all[:cnt], outs[3][:cnt], bounds)
        grads = []
        for k, (shape, dtype) in enumerate(ctx.shapes):
            if not ctx.needs_input_grad[2 + k]:
                grads.append(None)
                continue
            if ctx.shards is not None and getattr(ctx.shards[k], "_sparse_rows", False):
                shard = ctx.shards[k]
                if getattr(shard, "sparse_grad", None) is None:
                    # this table's part of the dedup is already coalesced: unique rows in
                    # ascending order and fp32 sums that start from +0.0, as index_add_'s do
                    # (what add_sparse_grad would return for it, without a second dedup)
                    shard.sparse_grad = batch.member(shard, k, locals_[k], sums[k])
                else:
                    add_sparse_grad(shard, locals_[k], sums[k])
                grads.append(None)
                continue
            g = torch.zeros(shape, dtype=torch.float32, device=grad.device)
            g[locals_[k]] = sums[k]  # unique rows: a plain scatter
            grads.append(g.to(dtype))
        return (None, None, *grads)


def row_lookup(engram, idx):
    """Per-table rows [*idx shape, dim] for the hashed ids `idx` (rows.py:150-161), world 1."""
    shards = engram.row_shards
    _rank, world, _starts, _pers = engram.row_info
    if world != 1:
        raise NotImplementedError("[micro_engram] row-sharded lookup over several ranks needs the "
                                  "multi-GPU row exchange, not part of this single-GPU build")
    idx2d = engram._stacked_idx(idx)
    mem = _RowLookup.apply(idx2d, _table_offsets(engram), *shards)
    D = engram.engram_dim
    shape = tuple(idx[0].shape)
    return [mem[:, k * D:(k + 1) * D].reshape(*shape, D) for k in range(len(shards))]


class RowTables:
    """The engrams' row tables on one GPU: optimizer, clipping (rows.py:179-247). entries:
    [(prefix, engram)] with row shards (MicroEngram.shard_rows(0, 1))."""

    def __init__(self, entries, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, lazy=False,
                 rowwise=False, stochastic_rounding=True, sparse_grads=False, seed=None):
        self.entries = entries
        self.world = 1
        train = [p for _, e in entries for p in e.row_shards if p.requires_grad]
        if sparse_grads and not lazy:
            raise ValueError("sparse row gradients need a lazy optimizer (lazy_adam / rowwise_adam): "
                             "plain AdamW updates every row every step")
        self.sparse = bool(sparse_grads)
        for p in train:
            p._sparse_rows = self.sparse
        self.optimizer = LazyAdamW([{"params": train, "lazy": lazy, "rowwise": rowwise}], lr=lr, betas=betas,
                                   eps=eps, weight_decay=weight_decay, stochastic_rounding=stochastic_rounding,
                                   seed=seed) if train else None
        self.last_grad_norm = None

    def params(self):
        return [p for _, e in self.entries for p in e.row_shards]

    def clip(self, max_norm):
        """Global norm of the table gradients, and the gradients scaled down in place to
        max_norm if it is larger (rows.py:208-233): dense p.grad and sparse_grad sums alike, by
        min(max_norm / (norm + 1e-6), 1), computed on the device from the norm (no host read
        before the scaling). Returns the norm (a host read, as in the reference)."""
        ps = [p for p in self.params() if p.requires_grad]
        if not ps:
            return None
        sq = torch.zeros(1, dtype=torch.float32, device=ps[0].device)
        batch, ks = SparseBatch.common(ps) if all(p.grad is None for p in ps) else (None, None)
        if (batch is not None and sorted(ks) == list(range(len(batch.bounds) - 1))
                and batch.sums.is_contiguous() and batch.sums.data_ptr() % 16 == 0):
            # every table's gradient is its slice of one backward's sums, which tile them
            span = batch.sums.reshape(-1)
            ops.sumsq(span, sq, accumulate=True)
            if max_norm and max_norm > 0:
                ops.clip_scale(span, sq, max_norm)
            if self.optimizer is not None:
                self.optimizer.prepare_step()  # host work of the next step, before the host read
            self.last_grad_norm = float(sq.sqrt().item())
            return self.last_grad_norm
        squares, scaled = [], []
        for p in ps:
            if p.grad is not None:
                squares.append(p.grad if p.grad.dtype == torch.float32 else p.grad.float())
                scaled.append(p.grad)
            sg = getattr(p, "sparse_grad", None)
            if sg is not None:
                squares.append(sg[1])
                scaled.append(sg[1])
        square_spans = _spans(squares)
        for span in square_spans:
            ops.sumsq(span, sq, accumulate=True)
        if max_norm and max_norm > 0:
            # the same tensors (fp32 gradients) make the same spans
            same = len(squares) == len(scaled) and all(a is b for a, b in zip(squares, scaled))
            for span in (square_spans if same else _spans(scaled)):
                if span.is_contiguous() and span.data_ptr() % 16 == 0:
                    ops.clip_scale(span, sq, max_norm)
                else:  # a view the kernel cannot scale in place: scale a copy, write it back
                    span.copy_(ops.clip_scale(span.contiguous().clone(), sq, max_norm))
        self.last_grad_norm = float(sq.sqrt().item())
        return self.last_grad_norm

    def step(self, lr):
        if self.optimizer is None:
            return
        for g in self.optimizer.param_groups:
            g["lr"] = lr
        self.optimizer.step()
        self.zero_grad()

    def zero_grad(self):
        if self.optimizer is not None:
            self.optimizer.zero_grad(set_to_none=True)
        for p in self.params():
            p.sparse_grad = None
            p.__dict__.pop("_sparse_batch", None)

    # --- checkpoints: DCP folders (rows.py:257-343 fixes their names and contents) ---------
    def _trainable_tables(self, include_frozen=False):
        """(name in the checkpoint, shard) of every table of the engrams that train rows."""
        for prefix, engram in self.entries:
            if include_frozen or any(p.requires_grad for p in engram.row_shards):
                for k, shard in enumerate(engram.row_shards):
                    yield f"{prefix}tables.{k}.weight", shard

    def save(self, folder, optim_folder=None):
        """Write the engrams that train rows, complete (their tables and every other tensor under
        full names, the scales as 1 + delta), to the DCP folder `folder`; and the tables'
        optimizer state -- <table name>.exp_avg, .exp_avg_sq and .step -- to `optim_folder`.
        With one GPU each shard is a whole table and is written as it is."""
        import torch.distributed.checkpoint as dcp

        tensors = {}
        for prefix, engram in self.entries:
            if any(p.requires_grad for p in engram.row_shards):
                tensors.update((prefix + k, v.detach()) for k, v in engram.state_dict().items())
        tensors.update((name, shard.detach()) for name, shard in self._trainable_tables())
        if tensors:
            dcp.save(tensors, checkpoint_id=folder, no_dist=True)
        if not optim_folder or self.optimizer is None:
            return
        state = {}
        for name, shard in self._trainable_tables():
            st = self.optimizer.state.get(shard)
            if st:
                state[name + ".exp_avg"] = st["exp_avg"]
                state[name + ".exp_avg_sq"] = st["exp_avg_sq"]
                state[name + ".step"] = st["step"].detach().clone().reshape(())
        if state:
            dcp.save(state, checkpoint_id=optim_folder, no_dist=True)

    def _locate_tables(self, folder, meta):
        """{name in the folder: shard to fill} for every table of every engram. A table is found
        under the engram's own layer, else under a name without a layer; its row count must be
        the engram's (a run cannot resume onto tables of another size)."""
        from .weights import EngramKey

        saved = {}
        for name in meta:
            key = EngramKey.parse(name)
            if key is not None and key.local.startswith("tables."):
                saved[(key.layer, key.local)] = name
        plan = {}
        for prefix, engram in self.entries:
            layer = EngramKey.parse(prefix + "x")
            layer = None if layer is None else layer.layer
            for k, shard in enumerate(engram.row_shards):
                local = f"tables.{k}.weight"
                name = saved.get((layer, local)) or saved.get((None, local))
                if name is None:
                    raise ValueError(f"[micro_engram] {folder} holds no {local} for the engram at "
                                     f"{prefix.rstrip('.')}")
                rows = meta[name].size[0]
                if rows != engram.table_rows[k]:
                    raise ValueError(
                        f"[micro_engram] {folder}: {local} was saved with {rows:,} rows; this engram's "
                        f"table {k} (order {engram._table_orders[k]}) has {engram.table_rows[k]:,}. "
                        "Resuming needs the same table sizes.")
                plan[name] = shard
        return plan

    def load(self, folder, optim_folder=None):
        """Fill the row shards in place from a DCP folder -- a micro_engram_rows folder, or the
        model checkpoint of a run that did not shard rows -- and, when `optim_folder` exists, the
        tables' optimizer state, converting the second moment if the other optimizer wrote it
        (per value <-> per row). Returns (tables loaded, whether optimizer state was loaded)."""
        import torch.distributed.checkpoint as dcp

        meta = dcp.FileSystemReader(folder).read_metadata().state_dict_metadata
        plan = self._locate_tables(folder, meta)
        dcp.load({name: shard.data for name, shard in plan.items()}, checkpoint_id=folder, no_dist=True)
        self.converted = 0
        if optim_folder and self.optimizer is not None and os.path.isdir(optim_folder):
            return len(plan), self._load_optimizer(optim_folder)
        return len(plan), False

    def _load_optimizer(self, optim_folder):
        import torch.distributed.checkpoint as dcp

        meta = dcp.FileSystemReader(optim_folder).read_metadata().state_dict_metadata
        group = self.optimizer.param_groups[0]
        targets, steps, foreign = {}, {}, {}
        for name, shard in self._trainable_tables():
            if name + ".exp_avg" not in meta:
                continue
            st = self.optimizer.state[shard]
            if not st:
                LazyAdamW.init_state(st, shard, group)
            targets[name + ".exp_avg"] = st["exp_avg"]
            saved_dims = len(meta[name + ".exp_avg_sq"].size)
            if saved_dims == st["exp_avg_sq"].dim():
                targets[name + ".exp_avg_sq"] = st["exp_avg_sq"]
            else:  # the other optimizer's layout: read it as saved, convert below
                shape = shard.shape if saved_dims == shard.dim() else shard.shape[:1]
                foreign[shard] = torch.zeros(shape, dtype=torch.float32, device=shard.device)
                targets[name + ".exp_avg_sq"] = foreign[shard]
            steps[shard] = targets[name + ".step"] = torch.zeros((), dtype=torch.float32)
        if not targets:
            return False
        dcp.load(targets, checkpoint_id=optim_folder, no_dist=True)
        for shard, step in steps.items():
            self.optimizer.state[shard]["step"] = step
        for shard, saved in foreign.items():
            self.optimizer.state[shard]["exp_avg_sq"].copy_(_convert_second_moment(saved, shard))
        self.converted = len(foreign)
        return True


def _convert_second_moment(saved, shard):
    """The second moment one optimizer saved, in the layout of the other (rows.py:330-339).
    Per value -> per row: the row mean, which is exactly what the row-wise optimizer keeps (the
    moment is linear in g^2 and the row-wise one averages g^2 over the row). Per row -> per
    value: every value of a row takes the row's moment."""
    if saved.dim() == shard.dim():
        return saved.flatten(1).mean(dim=1)
    return saved.reshape(-1, *([1] * (shard.dim() - 1))).expand_as(shard)
