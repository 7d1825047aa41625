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


class LazyAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, lazy=False,
                 rowwise=False, stochastic_rounding=True, seed=None):
        """stochastic_rounding: bf16 weights and states are written back with stochastic rounding
        (fp32 ones are unaffected). seed: key of the rounding noise (drawn from torch's default
        generator when None)."""
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, lazy=lazy,
                                      rowwise=rowwise, stochastic_rounding=stochastic_rounding))
        self.seed = int(torch.randint(0, 2**62, (1,)).item()) if seed is None else int(seed)

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
                     P_arr=ops.ptr_array(b["P"]), M_arr=ops.ptr_array(b["M"]), V_arr=ops.ptr_array(b["V"]))
        plan = plans[gi] = {"key": key, "members": members, "batches": list(batches.values())}
        return plan

    @torch.no_grad()
    def step(self, closure=None):
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
            # every step counter in one call, and one host read for all of them (the
            # counters are CPU tensors, as torch.optim.AdamW keeps them)
            counters = [self.state[p]["step"] for p in live]
            torch._foreach_add_(counters, 1)
            try:
                step_of = torch.stack(counters).tolist()
            except RuntimeError:  # counters loaded onto different devices
                step_of = [float(c) for c in counters]
            plan = self._launch_plan(gi, group, live)
            for b in plan["batches"]:
                dim, held, rp, gp, counts, steps = b["dim"], [], [], [], [], []
                for j, i in enumerate(b["pos"]):
                    p = live[i]
                    sparse = getattr(p, "sparse_grad", None)
                    if sparse is not None:
                        if not group["lazy"]:
                            raise ValueError("sparse row gradients need lazy=True")
                        rows, g = sparse
                        rows = rows if rows.dtype == torch.int64 else rows.long()
                        g = g if g.dtype == torch.float32 else g.float()
                    else:
                        g = p.grad if p.grad.dtype == torch.float32 else p.grad.float()
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
                                       ops.i64_array(counts), steps, b["stream_ids"], lr=group["lr"],
                                       betas=group["betas"], eps=group["eps"],
                                       weight_decay=group["weight_decay"], rowwise=b["rowwise"], lazy=b["lazy"],
                                       stochastic_rounding=group.get("stochastic_rounding", True), seed=self.seed)
                # the kernel wrote through raw pointers: move the version counters as torch's
                # own in-place ops would (autograd's saved-tensor checks and caches keyed on
                # them then see the update) (p itself: p.data has a version counter of its own)
                torch.autograd.graph.increment_version(b["written"])
        return loss
