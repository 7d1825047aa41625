"""The serving plugin's row-table seam on one GPU (the surface of micro_engram_vllm/tp.py).

vLLM's engram layers get their tables as row shards (MicroEngram.shard_rows) and a lookup
function installed as `row_lookup_fn` (micro_engram_vllm/model.py:173-193). On one GPU the
shard of every table is the whole table, so the masked lookup of tp.py:20-39 -- rows this rank
owns, zeros for the others, then a sum over ranks -- is a plain gather: here the me_gather
kernel, which already reads a row id outside its table as a zero row. More than one rank would
need the all-reduce of the masked rows, which this single-GPU build does not run: such a
lookup raises.
"""
import torch

from . import ops
from .module import check_loaded


def _world_one(engram):
    _rank, world, starts, _pers = engram.row_info
    if world != 1 or any(starts):
        raise NotImplementedError(
            f"[micro_engram] tp_lookup over {world} tensor-parallel ranks needs the all-reduce of "
            "the masked rows, which this single-GPU build does not provide")


def _tables(engram):
    """The rows the lookup reads: the UVA views of host-offloaded shards when the server made
    them (row_views), else the shards."""
    return engram.__dict__.get("row_views") or engram.row_shards


def tp_memory(engram, idx):
    """The concatenated memory vectors [N, n_tables * dim] for the hashed ids `idx`: what
    torch.cat(tp_lookup(...)(engram, idx), -1) gives, without the per-table split."""
    _world_one(engram)
    tables = _tables(engram)
    if torch.is_grad_enabled() and any(t.requires_grad for t in tables):
        # trainable rows: the differentiable row lookup (the same gather, with table gradients)
        from .rows import _RowLookup, _table_offsets

        return _RowLookup.apply(engram._stacked_idx(idx), _table_offsets(engram), *tables)
    return ops.gather(engram._stacked_idx(idx), [t.detach() for t in tables])


def tp_lookup(all_reduce):
    """A MicroEngram.row_lookup_fn (tp.py:17-39): per-table rows [*idx shape, dim] for the
    hashed ids. `all_reduce` would sum the ranks' masked rows; with one rank there is nothing to
    sum and it is never called."""

    def lookup(engram, idx):
        mem = tp_memory(engram, idx)
        shape = tuple(idx[0].shape)
        return list(mem.reshape(*shape, -1).split(engram.engram_dim, dim=-1))

    lookup.all_reduce = all_reduce
    lookup.memory = tp_memory  # MicroEngram takes the concatenated buffer from here directly
    return lookup


def load_rows(engram, sd, where, complete=True):
    """Load an engram state dict with whole tables (`tables.<k>.weight`) into a row-sharded
    engram (tp.py:42-77): each table is copied into this rank's shard (on one GPU, all of it),
    the rest goes through the module's own loading (scales converted by its state-dict hook).
    complete=False accepts part of an engram (tensors streamed in several calls) and reports
    nothing missing. Returns the set of table indices loaded."""
    rest = dict(sd)
    _rank, _world, starts, _pers = engram.row_info
    loaded = set()
    for k, shard in enumerate(engram.row_shards):
        full = rest.pop(f"tables.{k}.weight", None)
        if full is None:
            continue
        want = (engram.table_rows[k], engram.engram_dim)
        if tuple(full.shape) != want:
            raise ValueError(f"[micro_engram] {where}: table {k} is {tuple(full.shape)}, the engram's "
                             f"table {k} is {want}")
        first = starts[k]
        with torch.no_grad():
            shard.copy_(full[first:first + shard.shape[0]])
        loaded.add(k)
    stray = [name for name in rest if name.startswith("tables.")]
    if stray:
        raise ValueError(f"[micro_engram] {where}: tensors for tables the engram does not have: {stray[:5]}")
    if complete:
        absent = sorted(set(range(len(engram.row_shards))) - loaded)
        if absent:
            raise ValueError(f"[micro_engram] {where}: no rows given for tables {absent}")
        check_loaded(engram, rest, where)
    elif rest:
        if "mults" in rest and not torch.equal(rest["mults"].to(engram.mults.device).long(),
                                               engram.mults.long()):
            raise ValueError(f"[micro_engram] {where}: saved hash multipliers disagree with the engram's "
                             "seed (the seed is wrong for these weights)")
        result = engram.load_state_dict(rest, strict=False)
        if result.unexpected_keys:
            raise ValueError(f"[micro_engram] {where}: tensors the engram does not have: "
                             f"{result.unexpected_keys[:10]}")
    return loaded
