"""Full-size workloads on the GPU against the oracle, every token.

Two engrams with a token-merge map: the engrams of layers 0 and 29 (seeds 0 and 10007 * 29),
orders {2,3,4} with {1,572,864; 4,194,304; 4,194,304} rows, 8 heads x 64 bf16, a canon map
merging 15 % of the 262,144 ids, a prefill batch of 8 x 8192 packed Zipf tokens, hidden 5376
bf16. The hidden state goes through the first engram, then the second (the decoder layers in
between are not part of this path). Tolerance, on every element: after the first engram the bf16
bound of test_gate_gpu.py (one ulp of the output plus 2^-6 of the added update); after the
second, one ulp of each step's output plus 2^-6 of each step's update (a one-ulp difference of
the intermediate carries into the final value, which can sit in a smaller binade).
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
    """The oracle's inject of `eng` on the hidden rows h of the tokens `sample` (row ids from the
    oracle's hash of the whole batch, rows read from the engram's tables)."""
    idx = oracle.hash_ids(ids.numpy(), eng.mults.cpu().numpy(), eng._table_orders, eng.table_rows,
                          eng.canon.cpu().numpy(), eng.pad_id, position_ids=pos.numpy())
    idx = torch.from_numpy(idx.reshape(len(eng.tables), -1)[:, sample]).to(DEV)
    mem = torch.cat([t.weight[idx[k]] for k, t in enumerate(eng.tables)], dim=-1).cpu()
    return oracle.inject(h, mem, eng.key.weight.detach().cpu(), eng.value.weight.detach().cpu(),
                         "scalar_sqrt", eng.q_scale.detach().cpu(), eng.k_scale.detach().cpu())


def test_two_engram_canon_prefill_full():
    rng = np.random.Generator(np.random.PCG64(29))
    canon = synthetic.canon_map(rng, synthetic.GEMMA_VOCAB)
    ids, pos = synthetic.prefill_ids(seed=3, batch=8)
    gen = torch.Generator().manual_seed(4)
    hidden = torch.randn(8, 8192, synthetic.GEMMA_DIM, generator=gen).to(torch.bfloat16)
    engs = [synthetic.build_engram("gemma", DEV, seed=s, canon=canon).eval()
            for s in (0, synthetic.LAYER29_SEED)]
    assert not torch.equal(engs[0].canon.cpu(), torch.arange(engs[0].canon.numel()))
    with torch.no_grad():
        h1 = engs[0](hidden.to(DEV), ids.to(DEV), pos.to(DEV))
        h2 = engs[1](h1, ids.to(DEV), pos.to(DEV))
    torch.cuda.synchronize()
    sample = np.arange(8 * 8192)
    h0 = hidden.reshape(-1, hidden.shape[-1])
    r1 = _oracle_step(engs[0], h0, ids, pos, sample)
    r2 = _oracle_step(engs[1], r1, ids, pos, sample).float()
    r1, h0 = r1.float(), h0.float()
    g1 = h1.reshape(-1, h1.shape[-1]).float().cpu()
    g2 = h2.reshape(-1, h2.shape[-1]).float().cpu()
    ulp1 = _bf16_ulp(torch.maximum(g1.abs(), r1.abs()))
    err1 = (g1 - r1).abs()
    assert not (err1 > ulp1 + 2.0 ** -6 * (r1 - h0).abs()).any(), f"step 1 max err {float(err1.max()):.3g}"
    err2 = (g2 - r2).abs()
    bound = ulp1 + _bf16_ulp(torch.maximum(g2.abs(), r2.abs())) + 2.0 ** -6 * ((r1 - h0).abs() + (r2 - r1).abs())
    assert not (err2 > bound).any(), f"max err {float(err2.max()):.3g}"
    assert (err2.max(dim=-1).values <= 1e-2 * h0.norm(dim=-1)).all()
    del engs, h1, h2
    torch.cuda.empty_cache()
