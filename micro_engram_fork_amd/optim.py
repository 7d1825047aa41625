"""LazyAdamW for the engram tables on MI355X (micro_engram/optim.py:47-133 surface).

AdamW in which, for groups with lazy=True, a table row whose gradient is all zero keeps its
weights and both moments exactly (like torch.optim.SparseAdam); rowwise=True keeps one fp32
second moment per row (the running mean of the row's g^2). State names match
torch.optim.AdamW (step, exp_avg, exp_avg_sq). Row gradients arrive either as
p.sparse_grad = (unique rows, fp32 [n, D]) (the row-sharded training path,
micro_engram/rows.py:137-147) or as a dense p.grad.

The update runs as HIP launches of libmicro_engram_amd.so (me_sparse_adam), all tables of a
parameter group with the same layout in one launch. bf16 weights and moments are written back
with stochastic rounding whose noise comes from a counter-based generator (Philox4x32-10 keyed
by `seed`, the table's step and the element's position) instead of torch.randint: the same
rounding distribution, reproducible for a given seed.
"""
import torch

from . import ops


def stochastic_bf16(x, seed=None, step=0, stream_id=0):
    """fp32 -> bf16 with stochastic rounding (micro_engram/optim.py:33-44): the magnitude rounds
    up with probability equal to the dropped fraction, so on average nothing is lost; inf and
    NaN are kept. seed None draws one from torch's default generator."""
    if seed is None:
        seed = int(torch.randint(0, 2**62, (1,)).item())
    return ops.stochastic_bf16(x, seed, step, stream_id)


class SparseBatch:
    """The sparse gradients one row-lookup backward leaves on its tables: every table's
    (rows, sums) is a slice of the same two buffers (unique local rows, fp32 sums), at the
    bounds of that backward. Consumers that see a table's sparse_grad still be the exact tuple
    handed out here (nothing replaced it since) may address all tables from the two buffers at
    once -- the optimizer's pointer arrays and the clip's one reduction -- instead of touching
    each table's slices."""

    __slots__ = ("rows", "sums", "bounds", "handed", "__weakref__")

    def __init__(self, rows, sums, bounds):
        self.rows, self.sums, self.bounds = rows, sums, bounds
        self.handed = {}

    def member(self, shard, k, rows, sums):
        grad = (rows, sums)
        self.handed[k] = grad
        shard.__dict__["_sparse_batch"] = (self, k)
        return grad

    @staticmethod
    def common(params):
        """The batch every param's sparse_grad still comes from, with each param's table index,
        or (None, None)."""
        batch, ks = None, []
        for p in params:
            ref = p.__dict__.get("_sparse_batch")
            if ref is None:
                return None, None
            b, k = ref
            if (batch is not None and b is not batch) or b.handed.get(k) is not getattr(p, "sparse_grad", None):
                return None, None
            batch = b
            ks.append(k)
        return batch, ks


class LazyAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, lazy=False,
                 rowwise=False, stochastic_rounding=True, seed=None):
        """stochastic_rounding: bf16 weights and states are written back with stochastic rounding
        (fp32 ones are unaffected). seed: key of the rounding noise (drawn from torch's default
        generator when None)."""
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, lazy=lazy,
                                      rowwise=rowwise, stochastic_rounding=stochastic_rounding))
        self.seed = int(torch.randint(0, 2**62, (1,)).item()) if seed is None else int(seed)

    def load_state_dict(self, state_dict):
        """torch.optim's load, which casts every floating state tensor to its parameter's
        dtype; the row-wise second moment (one fp32 value per row of a table) is then put back
        from the saved fp32 values, since cast to a bf16 table's dtype it would lose what the
        row-wise update accumulates."""
        saved = state_dict["state"]
        ids = [i for g in state_dict["param_groups"] for i in g["params"]]
        super().load_state_dict(state_dict)
        params = [p for g in self.param_groups for p in g["params"]]
        for i, p in zip(ids, params):
            v = saved.get(i, {}).get("exp_avg_sq")
            if torch.is_tensor(v) and v.is_floating_point() and v.dim() == 1 and p.dim() >= 2:
                self.state[p]["exp_avg_sq"] = v.detach().to(dtype=torch.float32, device=p.device,
                                                             copy=True)
        self._plans = {}

    @staticmethod
    def init_state(state, p, group):
        """Fresh state: exp_avg like p; exp_avg_sq like p, or [rows] fp32 when row-wise
        (optim.py:55-63)."""
        state["step"] = torch.zeros((), dtype=torch.float32)
        state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
        if group.get("rowwise") and p.dim() >= 2:
            state["exp_avg_sq"] = torch.zeros(p.shape[0], dtype=torch.float32, device=p.device)
        else:
            state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)

    @staticmethod
    def _as_rows(t, n):
        if t.dim() == 2:  # tables: already [rows, D] (a view costs a few us of host time per table)
            return t
        return t.view(n, -1) if t.dim() > 2 else t.view(n, 1)

    def _launch_plan(self, gi, group, live):
        """The parts of group gi's launches that stay put between steps, for the live parameters:
        per (device, dtype, width, row-wise, lazy) batch the checked table / moment pointer arrays, the
        members' positions in `live`, their noise stream ids and the tensors the kernel writes.
        Kept while every parameter keeps its storage and shape and its state the same tensors
        (load_state_dict, a new .data or new parameters make a new plan)."""
        plans = self.__dict__.setdefault("_plans", {})
        key = (tuple(id(p) for p in live), bool(group["lazy"]))
        plan = plans.get(gi)
        if plan is not None and plan["key"] == key and all(
                p.data_ptr() == ptr and p.shape == shape and self.state[p]["exp_avg"] is m
                and self.state[p]["exp_avg_sq"] is v for p, ptr, shape, m, v in plan["members"]):
            return plan
        index = {id(p): i for i, p in enumerate(p for g in self.param_groups for p in g["params"])}
        members, batches = [], {}
        for i, p in enumerate(live):
            state = self.state[p]
            members.append((p, p.data_ptr(), p.shape, state["exp_avg"], state["exp_avg_sq"]))
            n = p.shape[0] if p.dim() >= 1 else 1
            rowwise = state["exp_avg_sq"].dim() == 1 and p.dim() >= 2
            # the reference's lazy branches need rows (p.dim() >= 2); others are plain AdamW
            lazy = bool(group["lazy"]) and p.dim() >= 2
            P = self._as_rows(p.data, n)
            M = self._as_rows(state["exp_avg"], n)
            V = state["exp_avg_sq"] if rowwise else self._as_rows(state["exp_avg_sq"], n)
            ops.require_gpu(P, M, V)
            if not (P.is_contiguous() and M.is_contiguous() and V.is_contiguous()):
                raise ValueError("[micro_engram] LazyAdamW: parameters and their state must be contiguous")
            if M.shape != P.shape or M.dtype != P.dtype or V.shape != ((n,) if rowwise else P.shape) or (
                    rowwise and V.dtype != torch.float32):
                raise ValueError("[micro_engram] LazyAdamW: optimizer state does not match its parameter")
            b = batches.setdefault((P.device, P.dtype, P.shape[1], rowwise, lazy, V.dtype),
                                   {"pos": [], "P": [], "M": [], "V": [], "stream_ids": [], "written": [],
                                    "arange": []})
            b["pos"].append(i)
            b["P"].append(P.data_ptr())
            b["M"].append(M.data_ptr())
            b["V"].append(V.data_ptr())
            b["stream_ids"].append(index[id(p)] % 65536)
            b["written"] += [p, state["exp_avg"], state["exp_avg_sq"]]
            b["arange"].append(None)  # all rows of a dense gradient, made on first use
        for (device, dtype, dim, rowwise, lazy, vdtype), b in batches.items():
            b.update(device=device, dim=dim, dtype=ops.dtype_code(torch.empty(0, dtype=dtype)), rowwise=rowwise, lazy=lazy,
                     sq_dtype=ops.ME_F32 if rowwise else ops.dtype_code(torch.empty(0, dtype=vdtype)),
                     P_arr=ops.ptr_array(b["P"]), M_arr=ops.ptr_array(b["M"]), V_arr=ops.ptr_array(b["V"]),
                     stream_arr=ops.i32_array(b["stream_ids"]))
        plan = plans[gi] = {"key": key, "members": members, "batches": list(batches.values())}
        return plan

    def _advance_steps(self, gi, group, live):
        """Adds 1 to the step counter of every live parameter and returns the new values. The
        counters are CPU tensors, as torch.optim.AdamW keeps them; those of a group are views
        into one buffer of the group (adopted on first sight, and again after anything put a
        tensor of its own in their place, e.g. load_state_dict), so the usual step -- every
        parameter live -- is one add and one host read."""
        bufs = self.__dict__.setdefault("_step_bufs", {})
        params = group["params"]
        entry = bufs.get(gi)
        if entry is None or entry[2] != tuple(id(p) for p in params):
            buf = torch.zeros(len(params), dtype=torch.float32)
            entry = bufs[gi] = (buf, [buf[i] for i in range(len(params))], tuple(id(p) for p in params))
        buf, views, _ = entry
        if len(live) == len(params) and all(a is b for a, b in zip(live, params)):
            states = [self.state[p] for p in params]
            for i, st in enumerate(states):
                if st["step"] is not views[i]:
                    step = st["step"]
                    if step.device.type != "cpu" or step.numel() != 1:
                        step = step.detach().reshape(()).cpu()
                    views[i].copy_(step.float())
                    st["step"] = views[i]
            buf.add_(1)
            return buf.tolist()
        counters = [self.state[p]["step"] for p in live]
        for c in counters:
            c.add_(1)
        return [float(c) for c in counters]

    @staticmethod
    def _batch_pointers(b, live, step_of):
        """The launch's row / gradient pointer arrays straight from a SparseBatch when every
        member's sparse gradient is still its slice of one row-lookup backward (the tables of a
        training step): (held tensors, row ptrs, grad ptrs, counts, steps), or None."""
        members = [live[i] for i in b["pos"]]
        batch, ks = SparseBatch.common(members)
        if batch is None:
            return None
        return LazyAdamW._batch_pointers_of(b, batch, ks, step_of)

    @staticmethod
    def _batch_pointers_of(b, batch, ks, step_of):
        rows, sums = batch.rows, batch.sums
        if (rows.dtype != torch.int64 or sums.dtype != torch.float32 or not rows.is_contiguous()
                or not sums.is_contiguous() or sums.dim() != 2 or sums.shape[1] != b["dim"]
                or rows.device != b["device"] or sums.device != b["device"]):
            return None
        bnd, dim = batch.bounds, b["dim"]
        rb, gb = rows.data_ptr(), sums.data_ptr()
        return ([rows, sums], [rb + bnd[k] * 8 for k in ks], [gb + bnd[k] * dim * 4 for k in ks],
                [bnd[k + 1] - bnd[k] for k in ks], [int(step_of[i]) for i in b["pos"]])

    def step(self, *args, **kwargs):
        """One step (closure: optional, as torch.optim's). torch.optim wraps an optimizer's step
        in a profiler range and its step hooks; that range is a dispatched op (~25 us of host
        time per step, paid with no profiler running, on a training step bound by its host's
        issue rate), so this optimizer runs the hooks itself, with the same order and return
        rules, and opens the range only while the autograd profiler is on."""
        if torch.autograd.profiler._is_profiler_enabled:
            with torch.autograd.profiler.record_function(f"Optimizer.step#{type(self).__name__}.step"):
                return self._hooked_step(args, kwargs)
        return self._hooked_step(args, kwargs)

    step.hooked = True  # torch.optim.Optimizer leaves a step marked so unwrapped

    def _hooked_step(self, args, kwargs):
        from torch.optim.optimizer import _global_optimizer_post_hooks, _global_optimizer_pre_hooks

        for pre_hook in (*_global_optimizer_pre_hooks.values(), *self._optimizer_step_pre_hooks.values()):
            result = pre_hook(self, args, kwargs)
            if result is not None:
                if isinstance(result, tuple) and len(result) == 2:
                    args, kwargs = result
                else:
                    raise RuntimeError(f"optimizer step pre-hooks must return None or a tuple of "
                                       f"(new_args, new_kwargs), but got {result}.")
        out = self._step(*args, **kwargs)
        self._optimizer_step_code()
        for post_hook in (*self._optimizer_step_post_hooks.values(), *_global_optimizer_post_hooks.values()):
            post_hook(self, args, kwargs)
        return out

    def zero_grad(self, set_to_none=True):
        """torch.optim's zero_grad; with set_to_none (the default) without its profiler range
        (opened only while the autograd profiler is on, as for step)."""
        if not set_to_none or torch.autograd.profiler._is_profiler_enabled:
            return super().zero_grad(set_to_none)
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    p.grad = None

    @torch.no_grad()
    def prepare_step(self):
        """Builds ahead of time the launch arguments of the next step for the batches whose
        members' sparse gradients are all slices of one row-lookup backward (SparseBatch), so
        that step() only checks that nothing changed -- the same batch, the same step counts --
        and launches. Meant for the time between the backward and a host sync (RowTables.clip
        calls it before it reads the norm): this host work then overlaps the GPU's backward
        instead of following the sync. Without a step() after it, it changes nothing."""
        prepared = {}
        for gi, group in enumerate(self.param_groups):
            if not group["lazy"]:
                continue
            live = [p for p in group["params"]
                    if p.grad is not None or getattr(p, "sparse_grad", None) is not None]
            if not live or any(not self.state[p] for p in live):
                continue
            nxt = [float(self.state[p]["step"]) + 1 for p in live]
            plan = self._launch_plan(gi, group, live)
            for bi, b in enumerate(plan["batches"]):
                batch, ks = SparseBatch.common([live[i] for i in b["pos"]])
                if batch is None:
                    continue
                fast = self._batch_pointers_of(b, batch, ks, nxt)
                if fast is None:
                    continue
                held, rp, gp, counts, steps = fast
                prepared[(gi, bi)] = (batch, ks, held, steps, ops.ptr_array(rp), ops.ptr_array(gp),
                                      ops.i64_array(counts), ops.i64_array(steps))
        self._prepared = prepared

    def _prepared_launch(self, gi, bi, b, live, step_of):
        """The arrays prepare_step built for batch bi of group gi, if they still hold."""
        prepared = self.__dict__.get("_prepared")
        pre = prepared.pop((gi, bi), None) if prepared else None
        if pre is None:
            return None
        batch, ks = SparseBatch.common([live[i] for i in b["pos"]])
        if batch is not pre[0] or ks != pre[1] or [int(step_of[i]) for i in b["pos"]] != pre[3]:
            return None
        return pre

    @torch.no_grad()
    def _step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for gi, group in enumerate(self.param_groups):
            live = [p for p in group["params"]
                    if p.grad is not None or getattr(p, "sparse_grad", None) is not None]
            if not live:
                continue
            for p in live:
                if not self.state[p]:
                    self.init_state(self.state[p], p, group)
            step_of = self._advance_steps(gi, group, live)
            plan = self._launch_plan(gi, group, live)
            for bi, b in enumerate(plan["batches"]):
                pre = self._prepared_launch(gi, bi, b, live, step_of) if group["lazy"] else None
                if pre is not None:  # arguments built by prepare_step while the GPU was busy
                    ops.sparse_adam_launch(b["device"], b["P_arr"], b["M_arr"], b["V_arr"], len(pre[3]),
                                           b["dim"], b["dtype"], b["sq_dtype"], pre[4], pre[5], pre[6], pre[7],
                                           b["stream_arr"], lr=group["lr"], betas=group["betas"],
                                           eps=group["eps"], weight_decay=group["weight_decay"],
                                           rowwise=b["rowwise"], lazy=b["lazy"],
                                           stochastic_rounding=group.get("stochastic_rounding", True),
                                           seed=self.seed)
                    torch.autograd.graph.increment_version(b["written"])
                    continue
                dim, held, rp, gp, counts, steps = b["dim"], [], [], [], [], []
                fast = self._batch_pointers(b, live, step_of) if group["lazy"] else None
                if fast is not None:
                    held, rp, gp, counts, steps = fast
                # gradients go to the kernel as they are when all are fp32 or all bf16 (it reads
                # either), else as fp32 copies
                grad_dtype = torch.float32
                if fast is None:
                    dts = {(p.sparse_grad[1] if getattr(p, "sparse_grad", None) is not None else p.grad).dtype
                           for p in (live[i] for i in b["pos"])}
                    if dts == {torch.bfloat16}:
                        grad_dtype = torch.bfloat16
                for j, i in enumerate(b["pos"] if fast is None else ()):
                    p = live[i]
                    sparse = getattr(p, "sparse_grad", None)
                    if sparse is not None:
                        if not group["lazy"]:
                            raise ValueError("sparse row gradients need lazy=True")
                        rows, g = sparse
                        rows = rows if rows.dtype == torch.int64 else rows.long()
                        g = g if g.dtype == grad_dtype else g.float()
                    else:
                        g = p.grad if p.grad.dtype == grad_dtype else p.grad.float()
                        rows = b["arange"][j]
                        n = p.shape[0] if p.dim() >= 1 else 1
                        if rows is None or rows.numel() != n or rows.device != p.device:
                            rows = b["arange"][j] = torch.arange(n, device=p.device)  # all-zero rows skip
                    k = rows.numel()
                    if g.dim() != 2 or g.shape[0] != k:
                        g = g.reshape(k, -1)
                    if g.shape[1] != dim or rows.dim() != 1:
                        raise ValueError("[micro_engram] LazyAdamW: gradient rows do not match the parameter")
                    if rows.device != p.device or g.device != p.device:
                        raise RuntimeError("[micro_engram] LazyAdamW: gradients must be on their parameter's GPU")
                    if not rows.is_contiguous():
                        rows = rows.contiguous()
                    if not g.is_contiguous():
                        g = g.contiguous()
                    held += [rows, g]
                    rp.append(rows.data_ptr())
                    gp.append(g.data_ptr())
                    counts.append(k)
                    steps.append(int(step_of[i]))
                ops.sparse_adam_launch(b["device"], b["P_arr"], b["M_arr"], b["V_arr"], len(rp), dim,
                                       b["dtype"], b["sq_dtype"], ops.ptr_array(rp), ops.ptr_array(gp),
                                       ops.i64_array(counts), steps, b["stream_arr"], lr=group["lr"],
                                       betas=group["betas"], eps=group["eps"],
                                       weight_decay=group["weight_decay"], rowwise=b["rowwise"], lazy=b["lazy"],
                                       stochastic_rounding=group.get("stochastic_rounding", True), seed=self.seed,
                                       grad_dtype=ops.ME_BF16 if grad_dtype == torch.bfloat16 else ops.ME_F32)
                # the kernel wrote through raw pointers: move the version counters as torch's
                # own in-place ops would (autograd's saved-tensor checks and caches keyed on
                # them then see the update) (p itself: p.data has a version counter of its own)
                torch.autograd.graph.increment_version(b["written"])
        return loss
