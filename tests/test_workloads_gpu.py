"""Full-size workloads on the GPU against the oracle, on sampled tokens.

Two engrams with a token-merge map: the engrams of layers 0 and 29 (seeds 0 and 10007 * 29),
orders {2,3,4} with {1,572,864; 4,194,304; 4,194,304} rows, 8 heads x 64 bf16, a canon map
merging 15 % of the 262,144 ids, a prefill batch of 8 x 8192 packed Zipf tokens, hidden 5376
bf16. The hidden state goes through the first engram, then the second (the decoder layers in
between are not part of this path). Tolerance: the bf16 bound of test_gate_gpu.py on the final
output against the oracle's two-step chain (each step rounded to bf16 like the GPU's).
"""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16_ulp(x):
    x = x.abs().float().clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(x)) - 7)


def _oracle_step(eng, h, ids, pos, sample):
    """The oracle's inject of `eng` on the sampled tokens' hidden rows h (row ids from the oracle's
    hash of the whole batch, rows read from the engram's tables)."""
    idx = oracle.hash_ids(ids.numpy(), eng.mults.cpu().numpy(), eng._table_orders, eng.table_rows,
                          eng.canon.cpu().numpy(), eng.pad_id, position_ids=pos.numpy())
    idx = torch.from_numpy(idx.reshape(len(eng.tables), -1)[:, sample]).to(DEV)
    mem = torch.cat([t.weight[idx[k]] for k, t in enumerate(eng.tables)], dim=-1).cpu()
    return oracle.inject(h, mem, eng.key.weight.detach().cpu(), eng.value.weight.detach().cpu(),
                         "scalar_sqrt", eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu())


def test_two_engram_canon_prefill_sampled():
    rng = np.random.Generator(np.random.PCG64(29))
    canon = synthetic.canon_map(rng, synthetic.GEMMA_VOCAB)
    ids, pos = synthetic.prefill_ids(seed=3, batch=8)
    gen = torch.Generator().manual_seed(4)
    hidden = torch.randn(8, 8192, synthetic.GEMMA_DIM, generator=gen).to(torch.bfloat16)
    engs = [synthetic.build_engram("gemma", DEV, seed=s, canon=canon).eval()
            for s in (0, synthetic.LAYER29_SEED)]
    assert not engs[0].identity_canon() and not engs[1].identity_canon()
    with torch.no_grad():
        h = hidden.to(DEV)
        for eng in engs:
            h = eng(h, ids.to(DEV), pos.to(DEV))
    torch.cuda.synchronize()
    sample = np.sort(np.random.Generator(np.random.PCG64(5)).choice(8 * 8192, 384, replace=False))
    got = h.reshape(-1, h.shape[-1])[torch.from_numpy(sample).to(DEV)].float().cpu()
    ref = hidden.reshape(-1, hidden.shape[-1])[sample]
    for eng in engs:
        ref = _oracle_step(eng, ref, ids, pos, sample)
    ref, h0 = ref.float(), hidden.reshape(-1, hidden.shape[-1])[sample].float()
    err = (got - ref).abs()
    # two bf16 residual roundings: one ulp of each, plus 2^-6 of the total update
    bound = 2 * _bf16_ulp(torch.maximum(got.abs(), ref.abs())) + 2.0 ** -6 * (ref - h0).abs()
    assert not (err > bound).any(), f"max err {float(err.max()):.3g}"
    assert (err.max(dim=-1).values <= 1e-2 * h0.norm(dim=-1)).all()
    del engs, h
    torch.cuda.empty_cache()
