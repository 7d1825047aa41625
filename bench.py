"""Engram forward throughput on one MI355X: the Gemma-31B-scale prefill.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload: one engram with orders {2,3,4}, 8 heads x 64 dims, bf16 tables of {1,572,864;
4,194,304; 4,194,304} rows (10.2 GB, resident in HBM), hidden 5376 bf16, one packed sequence of
8192 Zipf(1.1) tokens over a 262,144 vocab with documents of U[64, 2048] tokens. A step is one
forward (fused hash + row gather, then the K/V projection + scalar_sqrt gate + residual add),
all inputs already in HBM. Prints one JSON line:

  value         forward tokens/s over the K timed steps: one replay of a HIP graph of the K
                steps, wall clock, synchronised, after ~0.25 s of untimed replays of the same
                graph (an idle part needs ~0.1-0.2 s of load to reach its sustained clock; without
                them a 20-step replay reads ~8 % slow). Step k runs on prefill batch k % 16 of 16
                distinct seeded batches of this shape, so a step's gather meets caches that
                hold other batches' rows
  roofline      the gather kernel (the metric's HBM figure): algorithmic bytes per launch /
                its mean duration, against 8 TB/s. The duration: the gather's launches over the
                16 batches captured as a HIP graph, replayed between HIP events on the replay
                stream (the rocprofv3 kernel trace of this script's step sequence agrees).
                copy_1gib_gbs: a 1 GiB device copy, the known-size kernel that calibrates the
                HBM byte counters; copy_same_size: a device copy of the gather's output size
                (25 MB read + 25 MB written), the cost of the same bytes with no hashing;
                copy_same_size_nt: the same copy by a non-temporal 16-byte copy kernel (the
                fastest sequential copy of these bytes measured here); random_rows_same_size:
                the gather's access shape (random 128-byte rows of the same tables, written
                concatenated in token order) with row ids from integer arithmetic, so no
                dependent load precedes the row reads -- what random row reads of this size
                sustain; gather_over_random_rows = its time / the gather's
  roofline_gate the K/V projection + gate + residual kernels: 4 * M * d FLOP per token / their
                mean duration (graph replay, as above), against 2.5 PFLOP/s dense bf16
  serving_decode  a decode step of 256 one-token sequences on the same engram (hash_prev +
                inject, the calls of the vLLM decoder layer), graph replay over 16 distinct steps;
                its roofline: the step's algorithmic bytes (both projection weights, the tokens'
                table rows, ids, hidden in and out) / its duration, against 8 TB/s
  roofline_update  the training-side sparse update of a batch of this shape once its gradients
                exist (segment sums of the 196,608 lookups' gradient rows + row-wise Adam with
                stochastic rounding on the touched rows), algorithmic bytes / duration (graph
                replay) over 16 distinct batches; the key plan the sums read (unique keys,
                their rows and segment bounds, the tables' bounds) is made in the forward from
                the per-table row ids (me_dedup_tables, as the row lookup calls it) and is timed
                beside it (key_plan_ms; with_key_plan_frac counts all three)
  training_step  one training step of a second engram of the same shape with row-sharded
                tables (sparse row gradients): forward with gradients, backward from a fixed
                output gradient, clip (a host read, as the reference's trainer does), the row
                tables' lazy row-wise Adam step and the dense weights' AdamW step; wall clock
                over synchronised steps
  tiny_forward  the tiny fp32 forward (orders {2,3}, 16 tables of 65,536 rows, hidden 1024,
                2048 tokens): tokens/s, gather HBM and projection fp32 MFMA rooflines
  two_engram_canon  two Gemma-scale engrams with a 15 % canon map, 8 x 8192 tokens, chained:
                tokens/s and the gather's HBM roofline
  cpu_baseline  the reference path restated in torch-CPU ops (the oracle) on the same batch:
                hash on all tokens, lookup + inject on a sample, medians of 5 runs
  cpu_baseline_configs  the same restatement for the other workloads, each beside the GPU
                figure in its unit (gpu_value): tiny_forward (the whole fp32 forward),
                serving_decode (hash_prev + lookup + inject of one 256-token step),
                two_engram_canon (both engrams' hashes on all tokens, the chained lookups and
                injects on a sample), sparse_update (torch.unique + index_add_ + each table's
                row-wise Adam with stochastic rounding, one batch's 196,608 lookups)
"""
import argparse
import ctypes
import gc
import json
import os
import sys
import time

import numpy as np
import torch

from micro_engram_fork_amd import ops, rows, synthetic
from micro_engram_fork_amd.optim import LazyAdamW

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the baseline sample")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="seconds of untimed replays before each timed one (0 under a profiler that "
                         "counts every dispatch)")
    return ap.parse_args()


# HBM bytes per launch of the gather kernel on this workload: rocprofv3 --pmc FETCH_SIZE (12,433.1
# KiB per dispatch, x2.0) and WRITE_SIZE (24,600.7 KiB, x1.0), the factors being what the two
# counters read for this script's device copy of the gather's output size. A counter run cannot
# share a process with the timing, so the figure is a measured constant, re-measured when the
# kernel or its inputs change (the canon map's lines are in it; the paced row loads).
GATHER_TRAFFIC_BYTES = 50_654_105
CYCLE = 16  # distinct prefill batches the timed steps cycle through


def gather_bytes_per_token(eng, esize):
    """Algorithmic bytes of the fused hash + gather per token: every table row read and written
    once, plus the token id, its position and its canon entry (8 bytes each; the module reads
    the canon map on every call, identity or not)."""
    n_t = len(eng.table_rows)
    return n_t * eng.engram_dim * esize * 2 + 24


def update_batches(eng, dev, n_batches):
    """The training-side sparse update of n prefill batches of the workload's shape: each
    batch's 196,608 (token, table) lookups with fp32 gradients N(0, 1e-3), as keys into the
    concatenated tables (token-major, the order of the row lookup's backward)."""
    offs = [0]
    for r in eng.table_rows:
        offs.append(offs[-1] + r)
    off_t = torch.tensor(offs[:-1], device=dev)[:, None]
    out = []
    for s in range(n_batches):
        ids, pos = synthetic.prefill_ids(seed=s, device=dev)
        idx = torch.stack(eng.hash_ids(ids, pos)).reshape(len(eng.tables), -1)
        keys = (idx + off_t).t().reshape(-1).contiguous()
        grads = synthetic.lookup_grads(keys.numel(), eng.engram_dim, seed=s, device=dev)
        uniq, _inv, count, plan = ops.dedup_keys(keys, offs[-1])
        gsum = ops.dedup_sums(plan, count, grads)
        n_uniq = int(count.item())
        bounds = torch.searchsorted(uniq[:n_uniq], torch.tensor(offs, device=dev)).tolist()
        rows = [uniq[bounds[k]:bounds[k + 1]] - offs[k] for k in range(len(eng.tables))]
        sums = [gsum[bounds[k]:bounds[k + 1]] for k in range(len(eng.tables))]
        out.append((keys, grads, rows, sums, n_uniq, plan, count, idx))
    return out, offs[-1]


def key_bound_offsets(eng):
    """First key of every table in the concatenated key space, and the total (len n_tables + 1)."""
    offs = [0]
    for r in eng.table_rows:
        offs.append(offs[-1] + r)
    return offs


def update_bytes(n_lookups, n_uniq, dim, esize):
    """Algorithmic bytes of one sparse update, in three parts.
    Key plan (in the forward, from the per-table row ids): read the int64 row ids; write the
    unique keys and their int64 rows, the sorted positions (4 B per lookup) and two 4-byte segment
    bounds per unique key. Segment sums (the backward): read the fp32 gradient rows and their sorted
    positions, the segment bounds; write the summed fp32 rows. Row-wise Adam per unique row:
    weight and first moment read and written (esize each), the fp32 second moment read and
    written, the summed gradient and the row id read (784 B for 64 bf16)."""
    keys = n_lookups * 8 + n_uniq * 8 + n_uniq * 8 + n_lookups * 4 + n_uniq * 8
    sums = n_lookups * (4 * dim + 4) + n_uniq * (8 + 4 * dim)
    adam = n_uniq * (4 * dim * esize + 8 + 4 * dim + 8)
    return keys, sums, adam


def training_step_ms(dev, batches, steps, warmup):
    """Mean wall-clock ms of one training step on a second engram of the workload's shape with
    row-sharded tables: forward with gradients (hash, differentiable row lookup, gate), backward
    from a fixed output gradient (gate backward, weight GEMMs, dedup of the row gradients), the
    tables' clip (norm, in-place scaling, a host read of the norm), the lazy row-wise Adam step
    of the tables and the AdamW step of the dense key / value weights and scales, all with
    stochastic rounding (the reference trainer's two optimizers, train/loop.py:299-302)."""
    eng = synthetic.build_engram("gemma", dev, seed=1)
    eng.shard_rows(0, 1, device=dev)
    rt = rows.RowTables([("model.layers.0.micro_engram.", eng)], lr=5e-3, lazy=True, rowwise=True,
                        sparse_grads=True, seed=2024)
    dense = [eng.key.weight, eng.value.weight, eng.q_scale, eng.k_scale]
    dense_opt = LazyAdamW(dense, lr=5e-3, lazy=False, seed=2025)
    gen = torch.Generator(device=dev).manual_seed(7)
    gout = torch.randn(batches[0][2].shape, generator=gen, device=dev).to(torch.bfloat16) * 1e-3

    def step(k):
        ids, pos, hidden = batches[k % CYCLE]
        h = hidden.detach().requires_grad_(True)
        eng(h, ids, pos).backward(gout)
        rt.clip(1.0)
        rt.step(5e-3)
        dense_opt.step()
        dense_opt.zero_grad(set_to_none=True)

    for k in range(warmup):
        step(k)
    # read the gate statistics once, as a trainer's log step does (the first fold of a process
    # also loads its reduction kernels, ~10 ms once); fewer than 32 timed steps then fold none
    eng.pop_gate_stats()
    # The process's long-lived Python objects (torch, the modules, ~270 k of them) are moved out
    # of the collector's reach for the timed steps, as a training loop does after its set-up
    # (gc.freeze): a full collection over them takes ~80 ms, and one landing inside 30 steps of
    # ~1.5 ms read as 4 ms per step. Young-generation collections still run.
    gc.collect()
    gc.freeze()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(steps):
        step(warmup + k)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    gc.unfreeze()
    del rt, eng
    torch.cuda.empty_cache()
    return ms


def cpu_model():
    """The host CPU's model name (first 'model name' of /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def calib_lib():
    """The benchmark's calibration kernels (micro_engram_fork_amd/csrc/calib), through ctypes."""
    from micro_engram_fork_amd._build import CALIB_LIB_PATH

    lib = ctypes.CDLL(CALIB_LIB_PATH)
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    lib.me_calib_copy_nt.argtypes = [P, P, I64, ctypes.c_int, P]
    lib.me_calib_random_rows.argtypes = [P, P, ctypes.c_int, P, I64, ctypes.c_uint32, P]
    return lib


def calib_ok(status):
    if status != 0:
        raise RuntimeError(f"calibration kernel launch failed ({status})")


def _oracle():
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle

    return oracle


def cpu_threads():
    """torch intra-op threads for the CPU baselines: the host cores this process may use."""
    threads = int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    return threads


def median_s(fn, runs=5):
    """Median wall-clock seconds of `runs` calls of fn after one warm-up call."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


class CpuEngram:
    """An engram's tensors copied to host memory, for the torch-CPU restatement of the
    reference path (the oracle's functions): tables, key / value weights, scale deltas, hash
    constants."""

    def __init__(self, eng):
        self.tables = [t.weight.detach().cpu() for t in eng.tables]
        self.wk, self.wv = eng.key.weight.detach().cpu(), eng.value.weight.detach().cpu()
        self.dq, self.dk = eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu()
        self.mults, self.canon = eng.mults.cpu(), eng.canon.cpu()
        self.orders, self.rows, self.pad_id = eng._table_orders, eng.table_rows, eng.pad_id

    def hash_ids(self, ids, pos):
        return _oracle().hash_ids_torch(ids, self.mults, self.orders, self.rows, self.canon,
                                        self.pad_id, position_ids=pos)

    def hash_prev(self, ids):
        return _oracle().hash_prev_torch(ids, self.mults, self.orders, self.rows, self.canon,
                                         self.pad_id)

    def inject(self, hidden, idx):
        """lookup + cat + inject (module.py:146-154, 228-261) of hidden [n, d] with the row ids
        idx [n_tables, n]."""
        oracle = _oracle()
        mem = oracle.lookup_torch(self.tables, list(idx))
        return oracle.inject(hidden, mem, self.wk, self.wv, "scalar_sqrt", self.dq, self.dk)


def cpu_baseline(eng, ids, pos, hidden, target_s, runs=5, cpu_eng=None):
    """The reference path restated op for op in torch on the CPU (the oracle): hash_ids as
    torch tensor ops (module.py:183-205) on the whole batch, then F.embedding lookups + inject
    (module.py:146-154, 228-261) on a token sample; each timed as the median of `runs` runs
    after one warm-up, with torch's intra-op threads = the host cores this process may use."""
    oracle = _oracle()
    threads = cpu_threads()
    ce = cpu_eng or CpuEngram(eng)
    tables, wk, wv, dq, dk = ce.tables, ce.wk, ce.wv, ce.dq, ce.dk
    ids_c, pos_c = ids.cpu(), pos.cpu()
    mults, canon = ce.mults, ce.canon
    h_all = hidden.reshape(-1, hidden.shape[-1]).cpu()
    T = h_all.shape[0]
    median_s_ = lambda fn: median_s(fn, runs)

    hash_out = {}

    def hash_all():
        hash_out["idx"] = oracle.hash_ids_torch(ids_c, mults, eng._table_orders, eng.table_rows,
                                                canon, eng.pad_id, position_ids=pos_c)

    hash_s_per_tok = median_s_(hash_all) / T
    idx = hash_out["idx"].reshape(len(tables), -1)

    def run(sample):
        mem = oracle.lookup_torch(tables, [i[sample] for i in idx])
        return oracle.inject(h_all[sample], mem, wk, wv, "scalar_sqrt", dq, dk)

    rng = np.random.Generator(np.random.PCG64(0))
    probe = torch.from_numpy(np.sort(rng.choice(T, 128, replace=False)))
    run(probe)
    t0 = time.perf_counter()
    run(probe)
    per_tok = (time.perf_counter() - t0) / probe.numel()
    n = int(min(T, max(128, target_s / max(per_tok, 1e-9) / (runs + 1))))
    sample = torch.from_numpy(np.sort(rng.choice(T, n, replace=False)))
    per_tok = median_s_(lambda: run(sample)) / n + hash_s_per_tok
    return {"value": 1.0 / per_tok, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"hash_ids as torch-CPU ops on all {T} tokens, then lookup + inject on {n} of "
                      f"them; each the median of {runs} runs after 1 warm-up; per-token times "
                      f"added"}


def _baseline(value, unit, threads, sample, **extra):
    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": sample, **extra}


def cpu_baseline_tiny(eng, batch, runs=5):
    """The tiny fp32 forward restated in torch-CPU ops: hash_ids + lookup + inject of all its
    tokens (module.py:183-205, 146-154, 228-261), the median of `runs` runs."""
    threads = cpu_threads()
    ce = CpuEngram(eng)
    ids, pos, hidden = (t.cpu() for t in batch)
    h = hidden.reshape(-1, hidden.shape[-1])
    T = h.shape[0]
    sec = median_s(lambda: ce.inject(h, ce.hash_ids(ids, pos).reshape(len(ce.tables), -1)), runs)
    return _baseline(T / sec, "tokens/s", threads,
                     f"the whole forward of all {T} tokens; median of {runs} runs after 1 warm-up",
                     ms_per_forward=sec * 1e3)


def cpu_baseline_decode(ce, ids, hidden, runs=5):
    """A serving decode step restated in torch-CPU ops: hash_prev + lookup + inject
    (module.py:207-226, 146-154, 228-261) of its tokens on the host copy of the tables."""
    threads = cpu_threads()
    ids, hidden = ids.cpu(), hidden.cpu()
    sec = median_s(lambda: ce.inject(hidden, ce.hash_prev(ids)), runs)
    n = ids.shape[0]
    return _baseline(n / sec, "tokens/s", threads,
                     f"one whole decode step of {n} tokens; median of {runs} runs after 1 warm-up",
                     step_ms=sec * 1e3)


def cpu_baseline_two_engram(engs, ids, pos, hidden, target_s, runs=5):
    """The two-engram chain restated in torch-CPU ops: both engrams' hash_ids on all tokens, then
    lookup + inject of the first and of the second on its output for a token sample (inject is
    per token, so a sample is the chain on those tokens); per-token times added."""
    threads = cpu_threads()
    ces = [CpuEngram(e) for e in engs]
    ids_c, pos_c = ids.cpu(), pos.cpu()
    h_all = hidden.reshape(-1, hidden.shape[-1]).cpu()
    T = h_all.shape[0]
    idx = {}

    def hash_both():
        idx[0] = ces[0].hash_ids(ids_c, pos_c).reshape(len(ces[0].tables), -1)
        idx[1] = ces[1].hash_ids(ids_c, pos_c).reshape(len(ces[1].tables), -1)

    hash_s_per_tok = median_s(hash_both, runs) / T

    def chain(sample):
        out = ces[0].inject(h_all[sample], idx[0][:, sample])
        return ces[1].inject(out, idx[1][:, sample])

    rng = np.random.Generator(np.random.PCG64(1))
    probe = torch.from_numpy(np.sort(rng.choice(T, 64, replace=False)))
    chain(probe)
    t0 = time.perf_counter()
    chain(probe)
    per_tok = (time.perf_counter() - t0) / probe.numel()
    n = int(min(T, max(64, target_s / max(per_tok, 1e-9) / (runs + 1))))
    sample = torch.from_numpy(np.sort(rng.choice(T, n, replace=False)))
    per_tok = median_s(lambda: chain(sample), runs) / n + hash_s_per_tok
    return _baseline(1.0 / per_tok, "tokens/s", threads,
                     f"both engrams' hash_ids on all {T} tokens, then the two lookups + injects "
                     f"chained on {n} of them; each the median of {runs} runs after 1 warm-up; "
                     f"per-token times added")


def cpu_baseline_update(ce, keys, grads, offsets, runs=5):
    """The sparse update of one batch restated in torch-CPU ops: torch.unique + index_add_ of the
    lookups' gradient rows (rows.py:81, 117-118), then each table's lazy row-wise Adam step with
    stochastic bf16 rounding on its touched rows (optim.py:65-133, noise from torch.randint as
    optim.py:40 draws it). Runs on (and updates) the host copy of the tables."""
    oracle = _oracle()
    threads = cpu_threads()
    keys, grads = keys.cpu(), grads.cpu()
    D = grads.shape[1]
    m = [torch.zeros_like(t) for t in ce.tables]
    v = [torch.zeros(t.shape[0], dtype=torch.float32) for t in ce.tables]
    offs = torch.tensor(offsets, dtype=torch.int64)
    noise = lambda rows, which: torch.randint(0, 1 << 16, (rows.numel(), D), dtype=torch.int32)

    def update():
        uniq, _inv, acc = oracle.dedup_torch(keys, grads)
        b = torch.searchsorted(uniq, offs).tolist()
        for k, table in enumerate(ce.tables):
            oracle.sparse_adam_step(table, m[k], v[k], uniq[b[k]:b[k + 1]] - offsets[k],
                                    acc[b[k]:b[k + 1]], 1, 5e-3, noise=noise)

    sec = median_s(update, runs)
    n = keys.numel()
    return _baseline(n / sec, "lookups/s", threads,
                     f"dedup + row-wise Adam (SR) of all {n} lookups of one batch; median of {runs} "
                     f"runs after 1 warm-up", ms_per_update=sec * 1e3)


SETTLE_S = 0.25  # sustained replays before a timed one (the part's clock settles in ~0.1-0.2 s)
_SETTLE = [SETTLE_S]  # the run's setting (--settle caps every settle)


def settle(graph, seconds=None):
    """Replays `graph` back to back for about `seconds` (untimed, synchronised at the end). An
    MI355X that has idled runs its first milliseconds of work measurably slower than under
    sustained load (a 20-step replay right after a pause: ~290-305 us per step; after 0.2 s of
    replays: ~275 us, the same as a 50-step replay), so a timed replay is taken at the
    sustained operating point a serving loop runs at."""
    seconds = _SETTLE[0] if seconds is None else min(seconds, _SETTLE[0])
    t0 = time.perf_counter()
    while True:
        graph.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def replay_ms(fns, reps):
    """Mean duration in ms of one call of the sequence `fns`: `reps` rounds of the calls
    captured in one HIP graph and replayed between two HIP events on the replay stream
    (consecutive kernels of a graph start back to back, so the events add nothing per call),
    after the graph has settled the part's clock. Returns the mean per call of the sequence
    (total / (reps * len(fns)))."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in fns:
            fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(reps):
                for fn in fns:
                    fn()
        settle(graph, 0.1)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(side)
        graph.replay()
        end.record(side)
        torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * len(fns))


def graph_step_ms(step, n_steps):
    """Wall-clock ms per call of step(k), k = 0 .. n_steps-1 captured as one HIP graph and
    replayed once (synchronised on both sides), after an eager warm-up of each call and the
    graph's settle replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for k in range(n_steps):
            step(k)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for k in range(n_steps):
                step(k)
        settle(graph, 0.1)
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    del graph
    return wall / n_steps * 1e3


def measure_tiny(dev, steps=32, cycle=4, cpu=False):
    """The tiny fp32 forward: one engram, orders {2,3}, 16 tables of 65,536 x 64 fp32, hidden
    1024 fp32, one document of 2048 uniform ids over 32,000; `cycle` distinct seeded batches.
    Forward tokens/s, the gather's HBM roofline and the projection's fp32 MFMA roofline."""
    eng = synthetic.build_engram("tiny", dev, seed=0).eval()
    batches = [tuple(t.to(dev) for t in synthetic.tiny_inputs(seed=s)) for s in range(cycle)]
    T = batches[0][0].numel()
    mems = [None] * cycle

    def gather(k):
        ids, pos, _ = batches[k % cycle]
        mems[k % cycle] = eng.hashed_memory(ids, pos, dev)

    def gate(k):
        eng.gate_residual(batches[k % cycle][2], mems[k % cycle])

    with torch.inference_mode():
        ms = graph_step_ms(lambda k: (gather(k), gate(k)), steps)
        gather_ms = replay_ms([(lambda k=k: gather(k)) for k in range(cycle)], 4)
        gate_ms = replay_ms([(lambda k=k: gate(k)) for k in range(cycle)], 4)
    M = len(eng.table_rows) * eng.engram_dim
    d = batches[0][2].shape[-1]
    gbytes = gather_bytes_per_token(eng, 4) * T
    flop = 4.0 * M * d * T
    out = {
        "workload": "tiny_forward: 1 engram, orders {2,3}, 16 fp32 tables of 65536 x 64, hidden 1024 "
                    "fp32, 1 x 2048 uniform ids over 32000, one document, scalar_sqrt gate",
        "tokens_per_s": T / (ms * 1e-3), "ms_per_step": ms, "dtype": "f32",
        "gather": {"mean_ms": gather_ms, "bytes_per_launch": gbytes,
                   "achieved_gbs": gbytes / (gather_ms * 1e-3) / 1e9,
                   "frac": gbytes / (gather_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "gate": {"mean_ms": gate_ms, "flop_per_launch": flop,
                 "achieved_tflops": flop / (gate_ms * 1e-3) / 1e12, "peak_tflops": F32_PEAK_TFLOPS,
                 "frac": flop / (gate_ms * 1e-3) / 1e12 / F32_PEAK_TFLOPS},
    }
    if cpu:
        with torch.inference_mode():
            out["cpu_baseline"] = cpu_baseline_tiny(eng, batches[0])
        out["cpu_baseline"]["gpu_value"] = out["tokens_per_s"]
    del eng, batches, mems
    torch.cuda.empty_cache()
    return out


def measure_two_engram(dev, steps=3, cpu=False, cpu_seconds=10.0):
    """Two Gemma-scale engrams (layers 0 and 29: seeds 0 and 290,203) with a canon map merging
    15 % of the ids, prefill batch 8 x 8192 packed Zipf tokens, hidden 5376 bf16: the hidden
    state through the first engram, then the second. Forward tokens/s of the chain and the
    gather's HBM roofline (canon entry read per token)."""
    rng = np.random.Generator(np.random.PCG64(29))
    canon = synthetic.canon_map(rng, synthetic.GEMMA_VOCAB)
    engs = [synthetic.build_engram("gemma", dev, seed=s, canon=canon).eval()
            for s in (0, synthetic.LAYER29_SEED)]
    ids, pos = synthetic.prefill_ids(seed=3, batch=8, device=dev)
    gen = torch.Generator(device=dev).manual_seed(4)
    hidden = torch.randn(8, 8192, synthetic.GEMMA_DIM, generator=gen, device=dev).to(torch.bfloat16)
    T = ids.numel()
    state = {}

    def chain(k):
        h = hidden
        for eng in engs:
            h = eng(h, ids, pos)
        state["out"] = h

    def gather(k):
        state["mem"] = engs[k % 2].hashed_memory(ids, pos, dev)

    with torch.inference_mode():
        ms = graph_step_ms(chain, steps)
        gather_ms = replay_ms([(lambda k=k: gather(k)) for k in range(2)], 2)
    gbytes = gather_bytes_per_token(engs[0], 2) * T
    out = {
        "workload": "two_engram_canon: engrams of layers 0 and 29 (seeds 0, 290203), Gemma-scale "
                    "tables each, canon map merging 15% of 262144 ids, batch 8 x 8192 packed Zipf(1.1), "
                    "hidden 5376 bf16, chained",
        "tokens_per_s": T / (ms * 1e-3), "ms_per_step": ms, "tokens_per_step": T, "dtype": "bf16",
        "gather": {"mean_ms": gather_ms, "bytes_per_launch": gbytes,
                   "achieved_gbs": gbytes / (gather_ms * 1e-3) / 1e9,
                   "frac": gbytes / (gather_ms * 1e-3) / 1e9 / HBM_PEAK_GBS},
    }
    if cpu:
        with torch.inference_mode():
            out["cpu_baseline"] = cpu_baseline_two_engram(engs, ids, pos, hidden, cpu_seconds)
        out["cpu_baseline"]["gpu_value"] = out["tokens_per_s"]
    del engs, hidden, state
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    _SETTLE[0] = max(args.settle, 0.0)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the engram path here has no multi-GPU mode "
              f"(asked for --gpus {args.gpus}). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    eng = synthetic.build_engram("gemma", dev, seed=0).eval()
    # CYCLE distinct prefill batches of the workload's shape (seeds 0..15): step k uses batch
    # k % CYCLE, so every step's gather reads rows the previous steps have not left in the
    # caches (~400 MB of rows over the cycle, more than the 256 MB last-level cache), as
    # consecutive prefill batches do
    batches = []
    for s in range(CYCLE):
        ids, pos = synthetic.prefill_ids(seed=s, device=dev)
        gen = torch.Generator(device=dev).manual_seed(s + 1)
        hidden = torch.randn(ids.shape[0], ids.shape[1], synthetic.GEMMA_DIM, generator=gen,
                             device=dev).to(torch.bfloat16)
        batches.append((ids, pos, hidden))
    T = batches[0][0].numel()
    stream = torch.cuda.current_stream(dev)
    mems = [None] * CYCLE

    def gather(k):
        ids, pos, _ = batches[k % CYCLE]
        mems[k % CYCLE] = eng.hashed_memory(ids, pos, dev)

    def gate(k):
        eng.gate_residual(batches[k % CYCLE][2], mems[k % CYCLE])

    def step(k):
        gather(k)
        gate(k)

    with torch.inference_mode():
        for k in range(args.warmup):
            step(k)
        torch.cuda.synchronize()
        # The K steps are captured once as a HIP graph (the serving idiom: every op is graph
        # safe, no host synchronisation, shapes fixed) and the timed region is one replay of
        # it, synchronised on both sides, after untimed replays have brought the part to its
        # sustained clock (settle).
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for k in range(args.steps):
                    step(k)
            settle(graph)
            t0 = time.perf_counter()
            graph.replay()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
        del graph

        # Kernel durations: each kernel alone, over the same cycle of batches, replayed as a
        # graph between HIP events on the replay stream (the launches of a step sequence, as
        # the rocprofv3 kernel trace of this script shows, agree with these within a few %)
        gather_ms = replay_ms([(lambda k=k: gather(k)) for k in range(CYCLE)], 2)
        gate_ms = replay_ms([(lambda k=k: gate(k)) for k in range(CYCLE)], 2)

        # Serving decode on the same engram: 256 sequences x 1 token with 0-3 history tokens,
        # hash_prev + inject as the vLLM decoder layer calls them, over 16 distinct steps
        dsteps = []
        for s in range(CYCLE):
            dids, dhidden = synthetic.decode_inputs(seed=s)
            dsteps.append((dids.to(dev), dhidden.to(dev)))

        def decode(k):
            dids, dhidden = dsteps[k % CYCLE]
            eng.inject(dhidden, eng.hash_prev(dids))

        decode_ms = replay_ms([(lambda k=k: decode(k)) for k in range(CYCLE)], 2)
        decode_tokens = dsteps[0][0].shape[0]
        decode_cpu_input = dsteps[0]
        del dsteps

        # A plain device copy of the gather's output size (each launch on other buffers, as the
        # gather meets rows no earlier launch read): what moving the same bytes costs on this
        # part with no hashing and no random reads
        gbytes_out = T * len(eng.tables) * eng.engram_dim * eng.tables[0].weight.element_size()
        ring = torch.empty(2 * CYCLE * gbytes_out, dtype=torch.uint8, device=dev)
        views = [(ring[2 * k * gbytes_out:(2 * k + 1) * gbytes_out],
                  ring[(2 * k + 1) * gbytes_out:(2 * k + 2) * gbytes_out]) for k in range(CYCLE)]
        copy_same_ms = replay_ms([(lambda k=k: views[k][1].copy_(views[k][0])) for k in range(CYCLE)], 2)
        # the same bytes through the calibration kernels: a non-temporal 16-byte copy (its two
        # best launch shapes), and the gather's access shape -- random 128-byte rows of these
        # tables, written concatenated in token order -- with row ids from integer arithmetic
        # instead of the hash (no dependent load in front of the row reads)
        calib = calib_lib()
        sid = lambda: ops.stream_of(dev)  # the capturing stream, read at each call
        copy_nt_ms = min(replay_ms([(lambda k=k: calib_ok(calib.me_calib_copy_nt(
            views[k][0].data_ptr(), views[k][1].data_ptr(), gbytes_out, u, sid()))) for k in range(CYCLE)], 2)
            for u in (3, 12))
        tptrs = (ctypes.c_void_p * len(eng.tables))(*[t.weight.data_ptr() for t in eng.tables])
        trows = (ctypes.c_int64 * len(eng.tables))(*eng.table_rows)
        random_rows_ms = replay_ms([(lambda k=k: calib_ok(calib.me_calib_random_rows(
            tptrs, trows, len(eng.tables), views[k][1].data_ptr(), T, 77 * k + 1, sid())))
            for k in range(CYCLE)], 2)
        del views, ring

        # The sparse update (dedup + row-wise Adam with stochastic rounding) of the same
        # batch shape, over the same cycle of distinct batches; it writes the tables, so it
        # runs after the forward measurements.
        ubatches, key_bound = update_batches(eng, dev, CYCLE)
        tables = [t.weight.detach() for t in eng.tables]
        exp_avgs = [torch.zeros_like(t) for t in tables]
        exp_avg_sqs = [torch.zeros(t.shape[0], device=dev) for t in tables]
        streams = list(range(len(tables)))

        def dedup_keys(k):  # the row lookup's key plan: per-table row ids, no inverse
            ops.dedup_tables(ubatches[k % CYCLE][7], eng.table_rows, inverse=False)

        def dedup_sums(k):
            _, grads, _, _, _, plan, count, _ = ubatches[k % CYCLE]
            ops.dedup_sums(plan, count, grads)

        def adam(k):
            _, _, rows, sums, _, _, _, _ = ubatches[k % CYCLE]
            ops.sparse_adam(tables, exp_avgs, exp_avg_sqs, rows, sums, [1] * len(tables),
                            streams, lr=5e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0,
                            rowwise=True, lazy=True, stochastic_rounding=True, seed=2024)

        keys_ms = replay_ms([(lambda k=k: dedup_keys(k)) for k in range(CYCLE)], 2)
        sums_ms = replay_ms([(lambda k=k: dedup_sums(k)) for k in range(CYCLE)], 2)
        adam_ms = replay_ms([(lambda k=k: adam(k)) for k in range(CYCLE)], 2)
        n_lookups = ubatches[0][0].numel()
        n_uniq = float(np.mean([u[4] for u in ubatches]))
        update_cpu_input = (ubatches[0][0].cpu(), ubatches[0][1].cpu())
        del ubatches, exp_avgs, exp_avg_sqs
    train_ms = training_step_ms(dev, batches, steps=30, warmup=10)
    cpu = not args.no_cpu_baseline
    tiny = measure_tiny(dev, cpu=cpu)
    two = measure_two_engram(dev, cpu=cpu, cpu_seconds=args.cpu_seconds)
    with torch.inference_mode():
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        copy_ms = replay_ms([lambda: dst.copy_(src)], 5)
        del src, dst

    esize = eng.tables[0].weight.element_size()
    gbytes = gather_bytes_per_token(eng, esize) * T
    gather_gbs = gbytes / (gather_ms * 1e-3) / 1e9
    copy_gbs = 2.0 * (1 << 30) / (copy_ms * 1e-3) / 1e9
    M = len(eng.table_rows) * eng.engram_dim
    d = synthetic.GEMMA_DIM
    gate_flop = 4.0 * M * d * T
    gate_tflops = gate_flop / (gate_ms * 1e-3) / 1e12

    # decode step: algorithmic bytes = both projection weights + the 256 tokens' table rows, ids,
    # hidden read and output written (the weights dominate: 33 MB)
    n_dec = decode_tokens
    decode_bytes = (2 * d * M * esize + n_dec * len(eng.table_rows) * eng.engram_dim * esize
                    + n_dec * 4 * 4 + 2 * n_dec * d * esize)
    decode_gbs = decode_bytes / (decode_ms * 1e-3) / 1e9

    keys_b, sums_b, adam_b = update_bytes(n_lookups, n_uniq, eng.engram_dim, esize)
    update_gbs = (sums_b + adam_b) / ((sums_ms + adam_ms) * 1e-3) / 1e9
    result = {
        "metric": "Engram fwd tokens/sec @8192-token prefill on 1 GPU; gather HBM GB/s vs peak",
        "value": T * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: {CYCLE} seeded prefill batches cycled (Zipf ids, packed documents, "
                "hidden N(0,1)), random N(0,0.02) tables and dense weights",
        "config": {
            "workload": "gemma_prefill: 1 engram, orders {2,3,4}, 8 heads x 64, bf16 tables "
                        "{2:1572864, 3:4194304, 4:4194304} rows, hidden 5376, batch 1 x 8192 packed "
                        "Zipf(1.1) over 262144, scalar_sqrt gate",
            "tokens_per_step": T,
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "hash+gather (lookup_kernel)",
            "bound": "hbm",
            "achieved": gather_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gather_gbs / HBM_PEAK_GBS,
            "traffic": GATHER_TRAFFIC_BYTES,
            "bytes_per_launch": gbytes,
            "mean_ms": gather_ms,
            "copy_1gib_gbs": copy_gbs,
            "copy_same_size_ms": copy_same_ms,
            "copy_same_size_gbs": 2.0 * gbytes_out / (copy_same_ms * 1e-3) / 1e9,
            "copy_same_size_nt_ms": copy_nt_ms,
            "copy_same_size_nt_gbs": 2.0 * gbytes_out / (copy_nt_ms * 1e-3) / 1e9,
            "random_rows_same_size_ms": random_rows_ms,
            "random_rows_same_size_gbs": 2.0 * gbytes_out / (random_rows_ms * 1e-3) / 1e9,
            "gather_over_random_rows": random_rows_ms / gather_ms,
        },
        "roofline_gate": {
            "kernel": "K/V projection + gate + residual (gate224_kernel key + value passes on 256 x 224 "
                      "tiles, alpha)",
            "bound": "mfma",
            "achieved": gate_tflops,
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gate_tflops / BF16_PEAK_TFLOPS,
            "flop_per_launch": gate_flop,
            "mean_ms": gate_ms,
        },
        "roofline_update": {
            "kernel": "sparse update after the backward: segment sums of the gradient rows + "
                      "row-wise Adam with stochastic rounding (the key plan -- unique keys, "
                      "their rows, segment bounds, table bounds, from the per-table row ids -- "
                      "runs in the training forward, after the gate's launches on the same "
                      "stream; its time is key_plan_ms)",
            "bound": "hbm",
            "achieved": update_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": update_gbs / HBM_PEAK_GBS,
            "lookups": n_lookups,
            "unique_rows_mean": n_uniq,
            "sums_ms": sums_ms,
            "sums_gbs": sums_b / (sums_ms * 1e-3) / 1e9,
            "key_plan_ms": keys_ms,
            "key_plan_gbs": keys_b / (keys_ms * 1e-3) / 1e9,
            "with_key_plan_frac": (keys_b + sums_b + adam_b) / ((keys_ms + sums_ms + adam_ms) * 1e-3)
                                  / 1e9 / HBM_PEAK_GBS,
            "adam_ms": adam_ms,
            "adam_gbs": adam_b / (adam_ms * 1e-3) / 1e9,
        },
        "training_step": {
            "workload": "a second engram of the same shape, row-sharded tables: forward with "
                        "gradients + backward + clip + lazy row-wise Adam (SR) on 8192 tokens",
            "ms_per_step": train_ms,
            "tokens_per_s": T / (train_ms * 1e-3),
        },
        "serving_decode": {
            "workload": "the same engram, 256 sequences x 1 token (0-3 history tokens, [256, 4] "
                        "int32 ids with -1), hidden 5376 bf16: hash_prev + inject per step",
            "step_us": decode_ms * 1e3,
            "tokens_per_s": decode_tokens / (decode_ms * 1e-3),
            "roofline": {"bound": "hbm", "bytes_per_step": decode_bytes, "achieved": decode_gbs,
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": decode_gbs / HBM_PEAK_GBS},
        },
        "tiny_forward": tiny,
        "two_engram_canon": two,
        "timing": "value: wall clock around one replay of a HIP graph of the K steps; kernel "
                  "durations: per-kernel graph replays over the 16 batches between HIP events",
        "cpu_baseline": None,
    }
    if cpu:
        ids, pos, hidden = batches[0]
        with torch.inference_mode():
            ce = CpuEngram(eng)
            result["cpu_baseline"] = cpu_baseline(eng, ids, pos, hidden, args.cpu_seconds, cpu_eng=ce)
            # the other configurations' CPU restatements, each beside the GPU figure in its unit
            dec = cpu_baseline_decode(ce, *decode_cpu_input)
            dec["gpu_value"] = decode_tokens / (decode_ms * 1e-3)
            upd = cpu_baseline_update(ce, *update_cpu_input, key_bound_offsets(eng))
            upd["gpu_value"] = n_lookups / ((keys_ms + sums_ms + adam_ms) * 1e-3)
            del ce
        result["cpu_baseline_configs"] = {
            "tiny_forward": tiny.pop("cpu_baseline"),
            "serving_decode": dec,
            "two_engram_canon": two.pop("cpu_baseline"),
            "sparse_update": upd,
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
