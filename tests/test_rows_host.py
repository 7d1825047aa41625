"""Host-side logic of the row tables (CPU): the norm spans of RowTables.clip."""
import torch

from micro_engram_fork_amd.rows import _spans


def test_spans_merge_adjacent_slices_only():
    # slices that tile one buffer in order become one view; anything else stays apart, and the
    # squared sum over the spans is the squared sum over the parts
    buf = torch.arange(40, dtype=torch.float32).reshape(20, 2)
    other = torch.ones(4, 2)
    parts = [buf[0:3], buf[3:7], buf[7:20], other, buf[0:2], buf[5:8]]
    spans = _spans(parts)
    assert [s.numel() for s in spans] == [40, 8, 4, 6]
    assert spans[0].data_ptr() == buf.data_ptr() and spans[0].dim() == 1
    assert torch.equal(spans[0], buf.reshape(-1))
    assert float(sum(s.pow(2).sum() for s in spans)) == float(sum(p.pow(2).sum() for p in parts))


def test_spans_keep_other_dtypes_and_gaps_apart():
    buf = torch.zeros(10, dtype=torch.float32)
    parts = [buf[0:4], buf[5:9], torch.zeros(3, dtype=torch.bfloat16)]
    assert [s.numel() for s in _spans(parts)] == [4, 4, 3]


def test_spans_never_extend_a_strided_span():
    # a strided (non-contiguous) gradient followed by a contiguous one that starts where the
    # strided view's last element would end if it were dense: they stay apart, so the clip's
    # norm and scaling touch exactly the gradients' own elements
    buf = torch.arange(40, dtype=torch.float32)
    strided = buf[:20].view(5, 4)[:, :2]          # 10 elements, not contiguous
    after = buf[10:14]                            # starts at strided.data_ptr() + 10 * 4
    assert not strided.is_contiguous()
    assert strided.data_ptr() + strided.numel() * 4 == after.data_ptr()
    spans = _spans([strided, after])
    assert len(spans) == 2
    assert torch.equal(spans[0], strided) and torch.equal(spans[1], after)
    # a contiguous 1-D span followed by its neighbour still merges
    merged = _spans([buf[:6], buf[6:9]])
    assert len(merged) == 1 and torch.equal(merged[0], buf[:9])


def test_optimizer_load_keeps_the_row_wise_second_moment_fp32():
    # torch.optim's load casts floating state to the parameter's dtype; the row-wise second
    # moment of a bf16 table keeps its fp32 values (1 + 1e-4 is not a bf16 number)
    from micro_engram_fork_amd.optim import LazyAdamW
    table = torch.nn.Parameter(torch.zeros(5, 4, dtype=torch.bfloat16))
    bias = torch.nn.Parameter(torch.zeros(3, dtype=torch.bfloat16))
    opt = LazyAdamW([table, bias], lazy=True, rowwise=True, seed=1)
    for p in (table, bias):
        st = opt.state[p]
        LazyAdamW.init_state(st, p, opt.param_groups[0])
        st["step"] = torch.tensor(3.0)
        st["exp_avg_sq"] += 1.0001
    loaded = LazyAdamW([table, bias], lazy=True, rowwise=True, seed=1)
    loaded.load_state_dict(opt.state_dict())
    row = loaded.state[table]
    assert row["exp_avg_sq"].dtype == torch.float32 and row["exp_avg_sq"].shape == (5,)
    assert torch.equal(row["exp_avg_sq"], opt.state[table]["exp_avg_sq"])
    assert row["exp_avg_sq"] is not opt.state[table]["exp_avg_sq"]
    assert row["exp_avg"].dtype == torch.bfloat16 and float(row["step"]) == 3.0
    assert loaded.state[bias]["exp_avg_sq"].dtype == torch.bfloat16  # elementwise: torch's cast
