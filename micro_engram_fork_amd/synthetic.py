"""Seeded synthetic workloads of the Engram lookup path, shared by the benchmark and the tests.

RNGs: numpy PCG64 for token ids, document lengths and canon maps; torch generators for
tensors. Every builder is deterministic in its seed.

Workloads (unit of work in brackets):
  tiny_forward        [1 forward]  one engram, orders {2,3}, 65,536 rows x 16 tables, 8 heads x
                      64 dims, fp32; hidden [1, 2048, 1024] ~N(0,1); ids uniform over 32,000;
                      one document
  gemma_prefill       [1 forward]  orders {2,3,4} with {1,572,864; 4,194,304; 4,194,304} rows,
                      8 heads x 64 dims, bf16 tables (10.2 GB); hidden [1, 8192, 5376] bf16;
                      Zipf(1.1) ids over 262,144; packed documents of U[64, 2048] tokens
  serving_decode      [1 step]     the gemma tables; 256 sequences x 1 token with 0-3 history
                      tokens ([256, 4] int32, -1 = missing); hidden [256, 5376] bf16
  two_engram_canon    [1 forward]  two gemma-size engrams (layers 0 and 29), 15% canon merge,
                      batch 8 x 8192 packed Zipf ids
  sparse_update       [dedup + 1 rowwise_adam step]  the gemma_prefill batch's 196,608 lookups
                      with fp32 gradients ~N(0, 1e-3)
"""
import numpy as np
import torch

GEMMA_ORDERS = (2, 3, 4)
GEMMA_SIZES = {2: 1_572_864, 3: 4_194_304, 4: 4_194_304}
GEMMA_VOCAB = 262_144
GEMMA_DIM = 5376
LAYER29_SEED = 10007 * 29  # default seed of the engram at layer 29


def zipf_ids(rng, n, vocab, s=1.1):
    """n ids with P(rank r) ~ r^-s over `vocab`, ranks mapped to ids by a seeded permutation."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    p = ranks ** -s
    p /= p.sum()
    perm = rng.permutation(vocab)
    return perm[rng.choice(vocab, size=n, p=p)]


def packed_positions(rng, total, lo=64, hi=2048):
    """position_ids of documents with lengths U[lo, hi] packed into `total` tokens (the last
    one truncated); positions restart at 0 at each document start."""
    pos = np.empty(total, dtype=np.int64)
    t = 0
    while t < total:
        n = min(int(rng.integers(lo, hi + 1)), total - t)
        pos[t:t + n] = np.arange(n)
        t += n
    return pos


def canon_map(rng, vocab, frac=0.15):
    """An idempotent token-merge map: a random `frac` of ids map onto ids that are not merged
    (so canon[canon] == canon, the validity rule of micro_engram/runconfig.py:91-100)."""
    perm = rng.permutation(vocab)
    n_merge = int(round(frac * vocab))
    merged, keep = perm[:n_merge], perm[n_merge:]
    canon = np.arange(vocab, dtype=np.int64)
    canon[merged] = keep[rng.integers(0, keep.size, size=n_merge)]
    return canon


def fill_tables(engram, std=0.02, seed=0):
    """Re-initialise every table N(0, std) on its own device, seeded (in chunks: fast on a GPU
    for 10 GB of tables)."""
    gen_dev = None
    with torch.no_grad():
        for k, table in enumerate(engram.tables):
            w = table.weight
            gen = torch.Generator(device=w.device).manual_seed(seed * 1000 + k)
            gen_dev = w.device
            chunk = 1 << 22
            for a in range(0, w.shape[0], chunk):
                w[a:a + chunk].normal_(0.0, std, generator=gen)
    return gen_dev


def fill_dense(engram, seed=0, std=0.02, scale_std=0.1):
    """Random key/value weights (value non-zero, so the output is non-trivial) and small
    random scale deltas."""
    gen = torch.Generator().manual_seed(seed + 7)
    with torch.no_grad():
        for lin in (engram.key, engram.value):
            w = torch.randn(lin.weight.shape, generator=gen) * std
            lin.weight.copy_(w.to(lin.weight.dtype))
        if engram.gate == "scalar_sqrt":
            engram.q_scale.copy_((torch.randn(engram.q_scale.shape, generator=gen) * scale_std))
            engram.k_scale.copy_((torch.randn(engram.k_scale.shape, generator=gen) * scale_std))


def build_engram(kind, device, seed=0, dtype=None, gate="scalar_sqrt", canon=None):
    """A MicroEngram of one of the workload shapes, with random tables and dense weights."""
    from .module import MicroEngram

    if kind == "tiny":
        eng = MicroEngram(model_dim=1024, table_size=65_536, engram_dim=64, num_heads=8,
                          orders=(2, 3), vocab_size=32_000, seed=seed, gate=gate,
                          build_tables=False)
        dtype = dtype or torch.float32
    elif kind == "gemma":
        eng = MicroEngram(model_dim=GEMMA_DIM, table_size=GEMMA_SIZES[2], engram_dim=64,
                          num_heads=8, orders=GEMMA_ORDERS, table_sizes=GEMMA_SIZES,
                          vocab_size=GEMMA_VOCAB, seed=seed, gate=gate, canon=canon,
                          build_tables=False)
        dtype = dtype or torch.bfloat16
    else:
        raise ValueError(kind)
    # tables are created directly on the device (10 GB would not fit the host comfortably)
    eng.tables = torch.nn.ModuleList(
        torch.nn.Embedding(rows, eng.engram_dim, device=device, dtype=dtype) for rows in eng.table_rows)
    eng.to(device=device, dtype=dtype)
    fill_tables(eng, seed=seed)
    fill_dense(eng, seed=seed)
    return eng


def tiny_inputs(seed=0, device="cpu"):
    rng = np.random.Generator(np.random.PCG64(seed))
    T = 2048
    ids = torch.from_numpy(rng.integers(0, 32_000, size=(1, T))).to(device)
    pos = torch.arange(T, device=device).unsqueeze(0)
    gen = torch.Generator().manual_seed(seed + 1)
    hidden = torch.randn(1, T, 1024, generator=gen).to(device)
    return ids, pos, hidden


def prefill_ids(seed=0, batch=1, seq=8192, device="cpu"):
    """Zipf(1.1) ids over the gemma vocab [batch, seq] and the positions of packed documents."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ids = np.stack([zipf_ids(rng, seq, GEMMA_VOCAB) for _ in range(batch)])
    pos = np.stack([packed_positions(rng, seq) for _ in range(batch)])
    return torch.from_numpy(ids).to(device), torch.from_numpy(pos).to(device)


def prefill_inputs(seed=0, batch=1, seq=8192, device="cpu", dim=GEMMA_DIM, dtype=torch.bfloat16):
    """prefill_ids plus hidden ~N(0,1) [batch, seq, dim]."""
    ids, pos = prefill_ids(seed, batch, seq, device)
    gen = torch.Generator().manual_seed(seed + 1)
    hidden = torch.randn(batch, seq, dim, generator=gen).to(dtype)
    return ids, pos, hidden.to(device)


def decode_inputs(seed=0, n_seq=256, max_order=4, device="cpu", dim=GEMMA_DIM,
                  dtype=torch.bfloat16):
    """[n_seq, max_order] int32 ids (column i = token i steps back, -1 = none) with 0-3 history
    tokens per sequence, and hidden [n_seq, dim]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ids = zipf_ids(rng, n_seq * max_order, GEMMA_VOCAB).reshape(n_seq, max_order)
    hist = rng.integers(0, max_order, size=n_seq)  # tokens of history: 0..max_order-1
    hist[: n_seq // 2] = max_order - 1           # half the batch has the full history
    cols = np.arange(max_order)[None, :]
    ids = np.where(cols <= hist[:, None], ids, -1).astype(np.int32)
    gen = torch.Generator().manual_seed(seed + 1)
    hidden = torch.randn(n_seq, dim, generator=gen).to(dtype)
    return torch.from_numpy(ids).to(device), hidden.to(device)


def lookup_grads(n_lookups, dim, seed=0, device="cpu", std=1e-3):
    gen = torch.Generator(device=device).manual_seed(seed + 3)
    return torch.randn(n_lookups, dim, generator=gen, device=device) * std
