"""Writes the small golden fixtures under tests/golden/ from the oracle.

The reference's own tests hold no numeric vectors (they compare implementations), so these
fixtures are the oracle's outputs on seeded inputs, written once and checked in: they catch a
regression of the oracle itself and give the GPU tests fixed known answers.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def hash_small():
    rng = np.random.Generator(np.random.PCG64(2024))
    V = 1000
    orders = [2, 2, 3, 3, 4, 4]
    rows = [257, 257, 401, 401, 97, 97]
    mults = oracle.make_mults(290_203, len(orders), 4)
    canon = np.arange(V)
    merge = rng.choice(V, size=100, replace=False)
    canon[merge[:50]] = merge[50:]
    ids = rng.integers(-2, V + 2, size=(2, 40))
    pos = np.stack([np.concatenate([np.arange(13), np.arange(27)]),
                    np.concatenate([np.arange(5), np.arange(30), np.arange(5)])])
    idx = oracle.hash_ids(ids, mults, orders, rows, canon, 3, position_ids=pos)
    prev_ids = rng.integers(-1, V, size=(25, 4))
    prev_idx = oracle.hash_prev(prev_ids, mults, orders, rows, canon, 3)
    np.savez_compressed(os.path.join(HERE, "hash_small.npz"), ids=ids, pos=pos, canon=canon,
                        mults=mults, orders=np.array(orders), rows=np.array(rows), pad_id=3,
                        idx=idx, prev_ids=prev_ids, prev_idx=prev_idx)


def dedup_small():
    rng = np.random.Generator(np.random.PCG64(77))
    keys = rng.integers(0, 40, size=300)
    grads = rng.standard_normal((300, 8)).astype(np.float32)
    uniq, inv, acc = oracle.dedup(keys, grads)
    np.savez_compressed(os.path.join(HERE, "dedup_small.npz"), keys=keys, grads=grads, uniq=uniq,
                        inv=inv, acc=acc)


def inject_small():
    gen = torch.Generator().manual_seed(5)
    N, d, M = 12, 32, 16
    hidden = torch.randn(N, d, generator=gen) * 30
    mem = torch.randn(N, M, generator=gen) * 0.02
    wk = torch.randn(d, M, generator=gen) * 0.2
    wv = torch.randn(d, M, generator=gen) * 0.2
    dq = torch.randn(d, generator=gen) * 0.1
    dk = torch.randn(d, generator=gen) * 0.1
    out, alpha = oracle.inject(hidden, mem, wk, wv, "scalar_sqrt", dq, dk, return_alpha=True)
    np.savez_compressed(os.path.join(HERE, "inject_small.npz"), hidden=hidden.numpy(),
                        mem=mem.numpy(), wk=wk.numpy(), wv=wv.numpy(), dq=dq.numpy(),
                        dk=dk.numpy(), out=out.numpy(), alpha=alpha.numpy())


if __name__ == "__main__":
    hash_small()
    dedup_small()
    inject_small()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
