"""The drop-in boundary on the host (no GPU): the vLLM decoder layer's two calls trace as one
graph under torch.compile(fullgraph=True) (micro_engram_vllm/model.py:45-50, tp.py:5-7 ask for
torch.compile and CUDA graphs), for the plain engram, the plugin's tp_lookup wiring and a
replaced `lookup`; every import INTEGRATION.md shows resolves; and the ops' eager shortcut
hands dispatch modes and tensor subclasses to the registered ops."""
import os
import re

import pytest
import torch

from micro_engram_fork_amd import MicroEngram, ops
from micro_engram_fork_amd.tp import tp_lookup

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
N, DIM = 48, 64


def _engram():
    return MicroEngram(DIM, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3, 4),
                       vocab_size=1000, gate="scalar_sqrt").to(torch.bfloat16).eval()


def _trace(layer, *args):
    """The graphs dynamo hands to the backend for layer(*args) with fullgraph=True (the backend
    records them and returns a stand-in, so no kernel runs)."""
    graphs = []

    def record(gm, example_inputs):
        graphs.append(gm)
        return lambda *a: (torch.zeros(N, DIM, dtype=torch.bfloat16),)

    torch._dynamo.reset()
    with torch.no_grad():
        torch.compile(layer, backend=record, fullgraph=True)(*args)
    torch._dynamo.reset()
    return graphs


def _targets(gm):
    return [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]


def _inputs():
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(-1, 1000, (N, 4), generator=g, dtype=torch.int32)
    hidden = torch.randn(N, DIM, generator=g).to(torch.bfloat16)
    keep = torch.arange(N) % 5 != 0
    return hidden, ids, keep


def test_decode_layer_traces_as_one_graph():
    eng = _engram()
    graphs = _trace(lambda h, ids, keep: eng.inject(h, eng.hash_prev(ids), keep), *_inputs())
    assert len(graphs) == 1
    ops_seen = [t for t in _targets(graphs[0]) if t.startswith("micro_engram_amd")]
    assert ops_seen == ["micro_engram_amd.hash_prev.default", "micro_engram_amd.gather.default",
                        "micro_engram_amd.gate_residual_rows.default"]


def test_tp_lookup_wiring_traces_as_one_graph():
    eng = _engram()
    eng.shard_rows(0, 1, dtype=torch.bfloat16, requires_grad=False, empty=True)
    eng.row_lookup_fn = tp_lookup(lambda x: x)
    graphs = _trace(lambda h, ids, keep: eng.inject(h, eng.hash_prev(ids), keep), *_inputs())
    assert len(graphs) == 1
    assert "micro_engram_amd.gather.default" in _targets(graphs[0])


def test_replaced_lookup_is_what_inject_reads():
    # the reference's own test replaces lookup on the instance (test_zero_order.py:84-88); the
    # rows it returns must be what the gate reads, traced or not
    eng = _engram()
    marker = [torch.full((N, 8), 0.5, dtype=torch.bfloat16) for _ in range(6)]
    eng.lookup = lambda _idx: marker
    assert eng._lookup_replaced()
    graphs = _trace(lambda h, ids, keep: eng.inject(h, eng.hash_prev(ids), keep), *_inputs())
    assert len(graphs) == 1
    targets = _targets(graphs[0])
    assert "micro_engram_amd.gather.default" not in targets
    assert any("cat" in t for t in targets)

    class Sub(MicroEngram):
        def lookup(self, idx):
            return super().lookup(idx)

    sub = Sub(DIM, table_size=97, engram_dim=8, num_heads=2, orders=(2, 3), vocab_size=1000)
    assert sub._lookup_replaced() and not _engram()._lookup_replaced()


def _integration_imports():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    stmts = []
    for block in blocks:
        for m in re.finditer(r"^from (micro_engram_fork_amd[\w.]*) import (\([^)]*\)|[^\n]+)",
                             block, flags=re.M):
            names = [n.strip() for n in m.group(2).strip("()").replace("\n", " ").split(",")]
            stmts.append((m.group(1), [n for n in names if n]))
    return stmts


def test_every_import_in_the_integration_notes_resolves():
    import importlib

    stmts = _integration_imports()
    assert len(stmts) >= 6
    for module, names in stmts:
        mod = importlib.import_module(module)
        missing = [n for n in names if not hasattr(mod, n)]
        assert not missing, f"INTEGRATION.md imports {missing} from {module}, which has no such names"


def test_eager_shortcut_leaves_modes_and_subclasses_to_the_ops():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.utils._python_dispatch import TorchDispatchMode

    t = torch.zeros(2)
    p = torch.nn.Parameter(torch.zeros(2))
    assert ops._direct_call((t, [t, p], None, 3), {"accumulate": True})

    class Passthrough(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with Passthrough():
        assert not ops._direct_call((t,), {})
    with FakeTensorMode() as mode:
        fake = mode.from_tensor(t)
    assert not ops._direct_call((fake,), {})
    assert not ops._direct_call((t, [t, fake]), {})
    assert not ops._direct_call((), {"idx": fake})

    class Sub(torch.Tensor):
        pass

    assert not ops._direct_call((t.as_subclass(Sub),), {})


def test_dispatch_mode_sees_the_op():
    # with a dispatch mode active around an eager call, the call goes to the registered op, so
    # the mode sees micro_engram_amd::gather (which then refuses the CPU tensors, as every op does)
    from torch.utils._python_dispatch import TorchDispatchMode

    seen = []

    class Record(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            seen.append(str(func))
            return func(*args, **(kwargs or {}))

    idx = torch.zeros(2, 4, dtype=torch.int64)
    tables = [torch.zeros(5, 8), torch.zeros(5, 8)]
    with Record():
        with pytest.raises(RuntimeError, match="runs only on the GPU"):
            ops.gather(idx, tables)
    assert "micro_engram_amd.gather.default" in seen
