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

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        index = {id(p): i for i, p in enumerate(p for g in self.param_groups for p in g["params"])}
        for group in self.param_groups:
            live = [p for p in group["params"]
                    if p.grad is not None or getattr(p, "sparse_grad", None) is not None]
            for p in live:
                if not self.state[p]:
                    self.init_state(self.state[p], p, group)
            # every step counter in one call, and one host read for all of them (the
            # counters are CPU tensors, as torch.optim.AdamW keeps them)
            counters = [self.state[p]["step"] for p in live]
            if counters:
                torch._foreach_add_(counters, 1)
                try:
                    step_of = torch.stack(counters).tolist()
                except RuntimeError:  # counters loaded onto different devices
                    step_of = [float(c) for c in counters]
            batches = {}
            for p, step in zip(live, step_of if counters else ()):
                sparse = getattr(p, "sparse_grad", None)
                state = self.state[p]
                n = p.shape[0] if p.dim() >= 1 else 1
                rowwise = state["exp_avg_sq"].dim() == 1 and p.dim() >= 2
                # the reference's lazy branches need rows (p.dim() >= 2); others are plain AdamW
                lazy = bool(group["lazy"]) and p.dim() >= 2
                if sparse is not None:
                    if not group["lazy"]:
                        raise ValueError("sparse row gradients need lazy=True")
                    rows, g = sparse
                    rows = rows if rows.dtype == torch.int64 else rows.long()
                    g = g if g.dtype == torch.float32 else g.float()
                else:
                    g = p.grad if p.grad.dtype == torch.float32 else p.grad.float()
                    rows = torch.arange(n, device=p.device)  # all-zero rows skip in the kernel
                P = self._as_rows(p.data, n)
                M = self._as_rows(state["exp_avg"], n)
                V = state["exp_avg_sq"] if rowwise else self._as_rows(state["exp_avg_sq"], n)
                key = (P.dtype, P.shape[1], rowwise, lazy, V.dtype)
                b = batches.setdefault(key, {"params": [], "exp_avgs": [], "exp_avg_sqs": [], "rows": [],
                                             "grads": [], "steps": [], "stream_ids": [], "written": []})
                b["written"] += [p, state["exp_avg"], state["exp_avg_sq"]]
                b["params"].append(P)
                b["exp_avgs"].append(M)
                b["exp_avg_sqs"].append(V)
                b["rows"].append(rows)
                b["grads"].append(g if g.dim() == 2 and g.shape[0] == rows.numel() else g.reshape(rows.numel(), -1))
                b["steps"].append(int(step))
                b["stream_ids"].append(index[id(p)] % 65536)
            for (_, _, rowwise, lazy, _), b in batches.items():
                ops.sparse_adam(b["params"], b["exp_avgs"], b["exp_avg_sqs"], b["rows"], b["grads"],
                                b["steps"], b["stream_ids"], lr=group["lr"], betas=group["betas"],
                                eps=group["eps"], weight_decay=group["weight_decay"], rowwise=rowwise,
                                lazy=lazy, stochastic_rounding=group.get("stochastic_rounding", True),
                                seed=self.seed)
                # the kernel wrote through raw pointers: move the version counters as torch's
                # own in-place ops would (autograd's saved-tensor checks and caches keyed on
                # them -- the engram's stacked key/value weight -- then see the update)
                # (p itself: p.data has a version counter of its own)
                torch.autograd.graph.increment_version(b["written"])
        return loss
