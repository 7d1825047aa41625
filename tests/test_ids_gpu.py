"""The serving-side kernels on the GPU against the oracle: fill_engram_ids (and the fused media
mask) and mask_media bit-exact, and the end-to-end property of test_vllm_ids.py:100-132 --
a request served in chunks and decode steps through fill_engram_ids + hash_prev + inject gives
the training forward's output."""
import numpy as np
import pytest
import torch

import oracle
from micro_engram_fork_amd import MicroEngram
from micro_engram_fork_amd.ids import fill_engram_ids, mask_media
from test_oracle_ids import CASES, SLOTS, histories, make_step, run_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_gpu(step, dtypes=None, media=None):
    dt = dtypes or {}
    out = torch.full((step["num_tokens"] + 10, step["width"]), 777, dtype=torch.int32, device=DEV)
    t = {k: torch.from_numpy(np.asarray(step[k])).to(dt.get(k, torch.from_numpy(np.asarray(step[k])).dtype)).to(DEV)
         for k in ("input_ids", "positions", "idx_mapping", "query_start_loc", "all_token_ids")}
    keep = None
    if media is not None:
        keep = torch.full((out.shape[0],), True, device=DEV)
        media = torch.tensor(media, device=DEV)
    fill_engram_ids(out, t["input_ids"], t["positions"], t["idx_mapping"], t["query_start_loc"],
                    t["all_token_ids"], step["num_reqs"], step["num_tokens"], step["num_tokens_padded"],
                    media_ids=media, keep=keep)
    return out.cpu().numpy(), None if keep is None else keep.cpu().numpy()


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("width", [3, 4, 1])
def test_fill_cases_bit_exact(name, width):
    step = make_step(CASES[name], histories(), SLOTS, width)
    got, _ = run_gpu(step)
    assert np.array_equal(got, run_oracle(step))


def _random_step(seed, n_reqs=200, max_len=4096, width=4):
    rng = np.random.Generator(np.random.PCG64(seed))
    hist = {r: list(rng.integers(0, 262_144, max_len)) for r in range(n_reqs)}
    slots = {r: s for r, s in enumerate(rng.permutation(n_reqs + 7)[:n_reqs])}
    chunks = []
    for r in range(n_reqs):
        if rng.random() < 0.7:  # decode step at a random position (0 and 1 included)
            chunks.append((r, int(rng.integers(0, 50)) if r % 10 == 0 else int(rng.integers(0, max_len - 1)), 1))
        else:  # a prefill chunk, from the start or after a prefix-cache hit / earlier chunk
            start = 0 if rng.random() < 0.5 else int(rng.integers(1, max_len - 400))
            chunks.append((r, start, int(rng.integers(1, 300))))
    return make_step(chunks, hist, slots, width, rows=n_reqs + 7, max_len=max_len)


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("wide", [False, True])
def test_fill_random_serving_batch(seed, wide):
    step = _random_step(seed)
    dtypes = {k: torch.int64 for k in ("input_ids", "positions", "idx_mapping", "query_start_loc",
                                       "all_token_ids")} if wide else None
    got, _ = run_gpu(step, dtypes)
    assert np.array_equal(got, run_oracle(step))


def test_fill_with_media_mask_fused():
    step = _random_step(3, n_reqs=40)
    media = [int(step["input_ids"][5]), int(step["input_ids"][77]), 123456]
    got, keep = run_gpu(step, media=media)
    ref = run_oracle(step)
    padded = step["num_tokens_padded"]
    want_ids, want_keep = oracle.mask_media(ref[:padded], media)
    assert np.array_equal(got[:padded], want_ids) and np.array_equal(got[padded:], ref[padded:])
    assert np.array_equal(keep[:padded], want_keep)
    assert (~keep[:padded]).sum() > 0


def test_fill_zero_tokens_and_empty_requests():
    out = torch.full((6, 3), 777, dtype=torch.int32, device=DEV)
    z = torch.zeros(0, dtype=torch.int32, device=DEV)
    fill_engram_ids(out, z, z.long(), z, torch.zeros(1, dtype=torch.int32, device=DEV),
                    torch.zeros((1, 4), dtype=torch.int32, device=DEV), 0, 0, 4)
    assert (out[:4] == -1).all() and (out[4:] == 777).all()
    # requests with no tokens this step sit between others in query_start_loc
    h = histories()
    step = make_step([(0, 40, 1), (1, 37, 0), (2, 5, 3), (3, 0, 0)], h, SLOTS)
    got, _ = run_gpu(step)
    assert np.array_equal(got, run_oracle(step))


def test_mask_media_op():
    rng = np.random.Generator(np.random.PCG64(9))
    ids = rng.integers(-1, 50, (333, 4)).astype(np.int32)
    media = [3, 7, -1]
    got, keep = mask_media(torch.from_numpy(ids).to(DEV), torch.tensor(media, device=DEV))
    want, want_keep = oracle.mask_media(ids, media)
    assert np.array_equal(got.cpu().numpy(), want) and np.array_equal(keep.cpu().numpy(), want_keep)
    assert got.dtype == torch.int32 and keep.dtype == torch.bool


@pytest.mark.parametrize("gate,orders,sizes,width", [
    ("scalar", (2, 3), None, 3), ("scalar_sqrt", (2, 3), None, 3),
    ("scalar_sqrt", (2, 3, 4), {2: 257, 3: 401, 4: 97}, 4)])
def test_chunked_serving_equals_training_forward(gate, orders, sizes, width):
    # test_vllm_ids.py:100-132: chunked prefill then decode steps, fed through the persistent
    # id buffer, give the training forward's output token for token
    torch.manual_seed(0)
    eng = MicroEngram(model_dim=16, table_size=257, engram_dim=4, num_heads=2, orders=orders,
                      vocab_size=1000, pad_id=0, gate=gate, table_sizes=sizes)
    with torch.no_grad():
        eng.value.weight.normal_()
        canon = torch.arange(1000)
        canon[11], canon[501] = 10, 500
        eng.canon.copy_(canon)
    eng = eng.to(DEV).eval()
    seq = torch.tensor(histories()[0][:30])
    seq[4], seq[17] = 11, 501
    hidden = (torch.randn(30, 16) * 30).to(DEV)
    with torch.inference_mode():
        train = eng(hidden.unsqueeze(0), seq.unsqueeze(0).to(DEV))[0]
        served = []
        for chunk in [(0, 0, 13), (0, 13, 9)] + [(0, p, 1) for p in range(22, 30)]:
            step = make_step([chunk], {0: seq.tolist()}, {0: 3}, width)
            got, _ = run_gpu(step)
            _, start, cnt = chunk
            ids = torch.from_numpy(got[:cnt]).to(DEV)
            served.append(eng.inject(hidden[start:start + cnt], eng.hash_prev(ids)))
    assert torch.allclose(torch.cat(served), train, atol=1e-5)
