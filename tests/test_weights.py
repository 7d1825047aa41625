"""On-disk formats on the CPU: every format the engram can be saved in reads back into an equal
engram; tensor names with and without decoder layers; micro_engram_config.json parsing; the
token-merge map check; row-table checkpoints with optimizer state.

Modelled on the reference's own checks: test_rows.py:192-263 (DCP save/load, optimizer state,
lazy <-> rowwise conversion, resume from a checkpoint without row sharding), test_multi.py:146-323
(configs, several engrams, shared files) and runconfig.py:91-100 (canon).
"""
import json
import os

import numpy as np
import pytest
import torch

from micro_engram_fork_amd import MicroEngram, check_loaded, engram_from_spec
from micro_engram_fork_amd.rows import ROWS_DIR, ROWS_OPTIM_DIR, RowTables
from micro_engram_fork_amd.optim import LazyAdamW
from micro_engram_fork_amd import weights as W

D, N, E = 32, 61, 8


def _engram(seed=3, orders=(2, 3), canon=None, sizes=None):
    torch.manual_seed(seed)
    eng = MicroEngram(model_dim=D, table_size=N, engram_dim=E, num_heads=2, orders=orders, vocab_size=50,
                      gate="scalar_sqrt", seed=seed, canon=canon, table_sizes=sizes)
    with torch.no_grad():
        for t in eng.tables:
            t.weight.normal_(0, 0.1)
        eng.key.weight.normal_(0, 0.1)
        eng.value.weight.normal_(0, 0.1)
        eng.q_scale.fill_(0.25)
        eng.k_scale.normal_(0, 0.05)
    return eng


def _spec(eng, layer=0):
    return {"layer": layer, "table_size": N, "table_sizes": None, "engram_dim": E, "num_heads": 2,
            "orders": list(eng.orders), "gate": eng.gate, "seed": eng.seed, "pad_id": 0}


def _same(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    return sa.keys() == sb.keys() and all(torch.equal(sa[k], sb[k]) for k in sa)


CANON = np.arange(50)
CANON[[7, 9, 11]] = [3, 3, 5]


@pytest.mark.parametrize("fmt,name,layer", [("pt", "micro_engram.pt", None),
                                            ("pt", "full.pt", 4),
                                            ("safetensors", "e.safetensors", None),
                                            ("safetensors", "e.safetensors", 4),
                                            ("safetensors_dir", "merged", 4),
                                            ("dcp", "pytorch_model_fsdp_0", 4)])
def test_round_trip_every_format(tmp_path, fmt, name, layer):
    eng = _engram(canon=CANON)
    path = W.save_engram_weights(eng, str(tmp_path / name), layer=layer, fmt=fmt)
    sd = W.load_engram_weights(str(tmp_path / name), layer=layer)
    assert {"tables.0.weight", "key.weight", "value.weight", "q_scale", "k_scale", "mults", "canon"} <= set(sd)
    # files hold the scale itself, fp32 (module.py:166-172), not the delta the module keeps
    assert sd["q_scale"].dtype == torch.float32 and torch.equal(sd["q_scale"], torch.full((D,), 1.25))
    fresh = engram_from_spec(_spec(eng), D, 50, canon=sd["canon"])
    assert not torch.equal(fresh.tables[0].weight, eng.tables[0].weight)
    check_loaded(fresh, sd, path)
    assert _same(fresh, eng)  # the scales as stored (1 + delta) agree exactly
    # the module keeps the delta: back from the file it is (1 + delta) - 1 in fp32, as in the
    # reference's loader (module.py:174-181); 0.25 survives exactly, a random delta to rounding
    assert torch.equal(fresh.q_scale, eng.q_scale)
    assert torch.equal(fresh.k_scale, (eng.k_scale.float() + 1) - 1)
    if layer is not None:
        assert W.engram_layers_in(str(tmp_path / name)) == [layer]


def test_full_names_select_the_layer(tmp_path):
    # one file with the engrams of layers 0 and 29 (test_multi.py:310-323)
    a, b = _engram(seed=1), _engram(seed=2)
    sd = {W.full_name(0, k): v for k, v in a.state_dict().items()}
    sd.update({W.full_name(29, k, prefix="model.layers"): v for k, v in b.state_dict().items()})
    both = str(tmp_path / "both.pt")
    torch.save(sd, both)
    assert W.engram_layers_in(both) == [0, 29]
    got = W.load_engram_weights(both, layer=29, need_layer=True)
    assert torch.equal(got["tables.0.weight"], b.tables[0].weight)
    got0 = W.load_engram_weights(both, layer=0, need_layer=True)
    assert torch.equal(got0["tables.0.weight"], a.tables[0].weight)
    # local names shared by several engrams: refused, not silently the same tensors
    local = str(tmp_path / "local.pt")
    torch.save({"tables.0.weight": torch.zeros(4, 2), "value.weight": torch.zeros(2, 2)}, local)
    with pytest.raises(ValueError, match="several engrams"):
        W.load_engram_weights(local, layer=29, need_layer=True)
    assert "tables.0.weight" in W.load_engram_weights(local, layer=29)  # alone it still loads


def test_fsdp_wrapped_names_in_dcp(tmp_path):
    # an FSDP checkpoint of the whole model (test_rows.py:248-257): extra prefixes, the wrapper
    # module in the name, other tensors that are not the engram's
    import torch.distributed.checkpoint as dcp

    eng = _engram()
    pre = "base_model.model.model.language_model.layers.3._checkpoint_wrapped_module.micro_engram."
    sd = {pre + k: v for k, v in eng.state_dict().items()}
    sd["base_model.model.model.language_model.layers.3.mlp.up_proj.weight"] = torch.randn(4, 4)
    folder = str(tmp_path / "checkpoint-7" / "pytorch_model_fsdp_0")
    dcp.save(sd, checkpoint_id=folder, no_dist=True)
    got = W.load_engram_weights(folder, layer=3)
    assert "mlp.up_proj.weight" not in got and not any("up_proj" in k for k in got)
    assert torch.equal(got["tables.1.weight"], eng.tables[1].weight)
    assert W.load_engram_weights(folder, layer=5) == {}
    assert W.layer_of_key(pre + "tables.0.weight") == 3
    assert W.local_name(pre + "tables.0.weight") == "tables.0.weight"
    assert W.local_name("model.layers.3.mlp.up_proj.weight") is None


class Payload:
    """An arbitrary pickled object: a weights_only load must refuse it."""


def test_weights_only_loading(tmp_path):
    # .pt files are read with weights_only=True: a pickled object is refused, not executed
    bad = str(tmp_path / "bad.pt")
    torch.save({"tables.0.weight": torch.zeros(2, 2), "obj": Payload()}, bad)
    with pytest.raises(Exception, match="[Ww]eights only|weights_only|Unsupported global"):
        W.load_engram_weights(bad)


def test_engram_specs_forms():
    # an old config: one engram at the top level, no "engrams", no "seed" (test_multi.py:275-278)
    legacy = {"table_size": 1000, "engram_dim": 64, "num_heads": 4, "weights": "micro_engram.pt"}
    (s,) = W.engram_specs(legacy, "/x/micro_engram_config.json")
    assert s["layer"] == 0 and s["seed"] == 0 and s["orders"] == (2, 3) and s["gate"] == "scalar"
    assert s["weights"] == "/x/micro_engram.pt"
    # the multi-engram form: entries inherit the top level, string table_sizes keys become ints
    conf = {"table_size": 1000, "engram_dim": 64, "num_heads": 4, "gate": "scalar_sqrt",
            "engrams": [{"layer": 0, "seed": 0, "weights": "../runA/checkpoint-10"},
                        {"layer": 29, "seed": 290203, "orders": [2, 3, 4],
                         "table_sizes": {"2": 5, "3": 7, "4": 0}, "weights": None}]}
    a, b = W.engram_specs(conf, "/runs/B/checkpoint-3/micro_engram_config.json")
    assert os.path.normpath(a["weights"]) == "/runs/B/runA/checkpoint-10" and a["gate"] == "scalar_sqrt"
    assert b["layer"] == 29 and b["seed"] == 290203 and b["orders"] == (2, 3, 4)
    assert b["table_sizes"] == {2: 5, 3: 7, 4: None} and b["weights"] is None
    assert W.default_seed(29) == 290203
    with pytest.raises(ValueError, match="more than one engram in a layer"):
        W.engram_specs({"engrams": [{"layer": 2}, {"layer": 2}]})
    assert W.norm_table_sizes(None) is None


def test_resolve_engram_source(tmp_path):
    eng = _engram()
    out = tmp_path / "out"
    for step, complete in ((5, True), (10, True), (12, False)):
        ck = out / f"checkpoint-{step}"
        os.makedirs(ck)
        if complete:
            (ck / "trainer_state.json").write_text("{}")
        W.save_engram_weights(eng, str(ck / "pytorch_model_fsdp_0"), layer=0)
        (ck / W.CONFIG_NAME).write_text(json.dumps({**_spec(eng), "weights": "pytorch_model_fsdp_0"}))
    assert W.latest_checkpoint(str(out)).endswith("checkpoint-10")  # 12 is not complete
    weights, spec = W.resolve_engram_source(str(out), 0)
    assert weights.endswith("checkpoint-10/pytorch_model_fsdp_0") and spec["seed"] == eng.seed
    # the config file itself, and bare weights (no settings)
    w2, s2 = W.resolve_engram_source(str(out / "checkpoint-5" / W.CONFIG_NAME), 0)
    assert w2.endswith("checkpoint-5/pytorch_model_fsdp_0") and s2["layer"] == 0
    w3, s3 = W.resolve_engram_source(str(out / "checkpoint-5" / "pytorch_model_fsdp_0"), 0)
    assert s3 is None and w3.endswith("pytorch_model_fsdp_0")
    with pytest.raises(ValueError, match="no engram at layer 7"):
        W.resolve_engram_source(str(out / "checkpoint-5"), 7)
    # end to end: config + weights -> an equal engram (the weights of a checkpoint folder)
    got = W.load_engram(str(out), 0, D, 50)
    assert _same(got, eng)


def test_check_canon():
    good = torch.tensor(CANON)
    assert torch.equal(W.check_canon(good, 50), good)
    with pytest.raises(ValueError, match="length"):
        W.check_canon(good[:10], 50)
    bad = good.clone()
    bad[4] = 50
    with pytest.raises(ValueError, match="outside"):
        W.check_canon(bad, 50)
    chain = good.clone()
    chain[3] = 1  # 7 -> 3 -> 1: not idempotent
    with pytest.raises(ValueError, match="idempotent"):
        W.check_canon(chain, 50)


def _rows_engram(seed=3, requires_grad=True):
    eng = _engram(seed=seed)
    eng.shard_rows(0, 1, requires_grad=requires_grad)
    return eng


PREFIX = "model.language_model.layers.3.micro_engram."


def _fill_state(rt, seed):
    g = torch.Generator().manual_seed(seed)
    for p in rt.params():
        st = rt.optimizer.state[p]
        LazyAdamW.init_state(st, p, rt.optimizer.param_groups[0])
        st["exp_avg"].copy_(torch.randn(st["exp_avg"].shape, generator=g))
        st["exp_avg_sq"].copy_(torch.rand(st["exp_avg_sq"].shape, generator=g))
        st["step"] = torch.tensor(3.0)


def test_row_tables_checkpoint_round_trip(tmp_path):
    src = _rows_engram()
    rt = RowTables([(PREFIX, src)], lazy=True)
    _fill_state(rt, 1)
    folder, ofolder = str(tmp_path / ROWS_DIR), str(tmp_path / ROWS_OPTIM_DIR)
    rt.save(folder, ofolder)
    # the folder is a complete engram the normal loaders read (scales as 1 + delta)
    sd = W.load_engram_weights(folder, layer=3)
    assert all(torch.equal(sd[f"tables.{k}.weight"], p) for k, p in enumerate(src.row_shards))
    assert torch.equal(sd["key.weight"], src.key.weight) and torch.allclose(sd["q_scale"], torch.full((D,), 1.25))
    assert "mults" in sd and "canon" in sd
    # resume into fresh rows: tables and optimizer state come back
    dst = _rows_engram(seed=3)
    with torch.no_grad():
        for p in dst.row_shards:
            p.zero_()
    rt2 = RowTables([(PREFIX, dst)], lazy=True)
    n, ok = rt2.load(folder, ofolder)
    assert n == 4 and ok and rt2.converted == 0
    assert all(torch.equal(a, b) for a, b in zip(dst.row_shards, src.row_shards))
    for a, b in zip(src.row_shards, dst.row_shards):
        sa, sb = rt.optimizer.state[a], rt2.optimizer.state[b]
        assert torch.equal(sa["exp_avg"], sb["exp_avg"]) and torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"])
        assert float(sb["step"]) == 3.0
    # lazy (per value) -> rowwise (per row): the row mean, exactly what rowwise would hold
    rw = _rows_engram()
    rt3 = RowTables([(PREFIX, rw)], lazy=True, rowwise=True)
    n, ok = rt3.load(folder, ofolder)
    assert ok and rt3.converted == 4
    for a, b in zip(src.row_shards, rw.row_shards):
        want = rt.optimizer.state[a]["exp_avg_sq"].mean(dim=1)
        assert rt3.optimizer.state[b]["exp_avg_sq"].shape == (a.shape[0],)
        assert torch.allclose(rt3.optimizer.state[b]["exp_avg_sq"], want)
    # rowwise -> lazy: every value gets its row's moment
    rw_dir = tmp_path / "rw"
    rt3.save(str(rw_dir / ROWS_DIR), str(rw_dir / ROWS_OPTIM_DIR))
    lz = _rows_engram()
    rt4 = RowTables([(PREFIX, lz)], lazy=True)
    rt4.load(str(rw_dir / ROWS_DIR), str(rw_dir / ROWS_OPTIM_DIR))
    for a, b in zip(rw.row_shards, lz.row_shards):
        v = rt4.optimizer.state[b]["exp_avg_sq"]
        assert v.shape == b.shape and torch.equal(v[:, 0], rt3.optimizer.state[a]["exp_avg_sq"])
    assert rt4.converted == 4


def test_row_tables_load_errors_and_plain_checkpoint(tmp_path):
    import torch.distributed.checkpoint as dcp

    full = _engram()
    old = str(tmp_path / "plain" / "pytorch_model_fsdp_0")
    wrapped = "base_model.model.model.language_model.layers.3._checkpoint_wrapped_module.micro_engram."
    dcp.save({wrapped + k: v for k, v in full.state_dict().items()}, checkpoint_id=old, no_dist=True)
    # resume from a run without row sharding: rows from the model checkpoint, Adam starts over
    sw = _rows_engram(seed=3)
    with torch.no_grad():
        for p in sw.row_shards:
            p.zero_()
    n, ok = RowTables([(PREFIX, sw)], lazy=True).load(old, str(tmp_path / "plain" / ROWS_OPTIM_DIR))
    assert n == 4 and not ok
    assert all(torch.equal(p, t.weight) for p, t in zip(sw.row_shards, full.tables))
    # other table sizes cannot resume
    other = MicroEngram(model_dim=D, table_size=N + 2, engram_dim=E, num_heads=2, vocab_size=50,
                        gate="scalar_sqrt", seed=3)
    other.shard_rows(0, 1)
    with pytest.raises(ValueError, match="rows"):
        RowTables([(PREFIX, other)], lazy=True).load(old)
    # a prefix whose layer has no tables in the folder
    eng = _engram()
    folder = str(tmp_path / "l3")
    dcp.save({"model.layers.3.micro_engram." + k: v for k, v in eng.state_dict().items()},
             checkpoint_id=folder, no_dist=True)
    with pytest.raises(ValueError, match="holds no tables.0.weight"):
        RowTables([("model.language_model.layers.9.micro_engram.", _rows_engram())], lazy=True).load(folder)
