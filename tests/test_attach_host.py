"""The training / HF entry on the CPU (micro_engram/module.py:286-393): find_text_layers,
layer_device_dtype and attach_engram's hooks. The engram's own compute needs the GPU, so its
forward is replaced by a recorder here; what is checked is the wiring: the engram becomes the
layer's submodule, the ids of the model's forward reach it once per forward, and its result
replaces the layer's output (first element of a tuple output)."""
import pytest
import torch
import torch.nn as nn

from micro_engram_fork_amd import MicroEngram, attach_engram, find_text_layers, layer_device_dtype


class _Layer(nn.Module):
    def __init__(self, d, tuple_out):
        super().__init__()
        self.norm = nn.LayerNorm(d)
        self.tuple_out = tuple_out

    def forward(self, x):
        y = self.norm(x)
        return (y, "aux") if self.tuple_out else y


class _Text(nn.Module):
    def __init__(self, d, n, tuple_out):
        super().__init__()
        self.embed = nn.Embedding(100, d)
        self.layers = nn.ModuleList(_Layer(d, tuple_out) for _ in range(n))

    def forward(self, input_ids=None, position_ids=None):
        x = self.embed(input_ids)
        for layer in self.layers:
            x = layer(x)
            x = x[0] if isinstance(x, tuple) else x
        return x


class _Model(nn.Module):
    """A multimodal-looking model: a vision tower listed first, then the language model."""

    def __init__(self, d=8, tuple_out=False):
        super().__init__()
        self.vision_tower = nn.Module()
        self.vision_tower.layers = nn.ModuleList(nn.Linear(d, d) for _ in range(2))
        self.language_model = _Text(d, 3, tuple_out)

    def forward(self, input_ids=None, position_ids=None):
        return self.language_model(input_ids=input_ids, position_ids=position_ids)


def _engram(d=8):
    return MicroEngram(model_dim=d, table_size=31, engram_dim=4, num_heads=2, orders=(2, 3),
                       vocab_size=100, gate="scalar_sqrt")


def test_find_text_layers_prefers_language_model():
    m = _Model()
    name, layers = find_text_layers(m)
    assert name == "language_model.layers" and layers is m.language_model.layers
    plain = nn.Module()
    plain.vision_layers = nn.ModuleList([nn.Linear(2, 2)])
    plain.blocks = nn.Module()
    plain.blocks.layers = nn.ModuleList([nn.Linear(2, 2)])
    assert find_text_layers(plain)[0] == "blocks.layers"
    with pytest.raises(RuntimeError):
        find_text_layers(nn.Linear(2, 2))


def test_layer_device_dtype_skips_packed_weights():
    class Params4bit(nn.Parameter):  # stands for bitsandbytes' packed 4-bit weight class
        pass

    layer = nn.Module()
    layer.q = nn.Module()
    layer.q.weight = Params4bit(torch.zeros(4, dtype=torch.bfloat16), requires_grad=False)
    layer.norm = nn.LayerNorm(4).to(torch.float16)
    assert layer_device_dtype(layer) == (torch.device("cpu"), torch.float16)
    only_packed = nn.Module()
    only_packed.q = nn.Module()
    only_packed.q.weight = Params4bit(torch.zeros(4, dtype=torch.uint8), requires_grad=False)
    only_packed.q.compute_dtype = torch.float32
    assert layer_device_dtype(only_packed) == (torch.device("cpu"), torch.float32)
    del only_packed.q.compute_dtype
    assert layer_device_dtype(only_packed)[1] == torch.bfloat16
    with pytest.raises(RuntimeError):
        layer_device_dtype(nn.Module())


@pytest.mark.parametrize("tuple_out", [False, True])
def test_attach_engram_injects_once_per_forward(tuple_out):
    m = _Model(tuple_out=tuple_out)
    eng = _engram()
    calls = []

    def recorder(hidden, input_ids, position_ids=None):
        calls.append((input_ids, position_ids))
        return hidden + 1000.0

    eng.forward = recorder
    name, handles = attach_engram(m, eng, 1, dtype=torch.float32)
    assert name == "language_model.layers.1"
    assert m.language_model.layers[1].micro_engram is eng
    assert eng.key.weight.dtype == torch.float32 and eng.mults.dtype == torch.int64
    ids = torch.randint(0, 100, (2, 5))
    pos = torch.arange(5).expand(2, 5)
    out = m(input_ids=ids, position_ids=pos)
    assert len(calls) == 1 and calls[0][0] is ids and calls[0][1] is pos
    # the layer after the engram normalises, so compare the layer's own output instead
    with torch.no_grad():
        x = m.language_model.embed(ids)
        x0 = m.language_model.layers[0].norm(x)
        y1 = m.language_model.layers[1](x0)
    y1 = y1[0] if tuple_out else y1
    assert torch.allclose(y1, m.language_model.layers[1].norm(x0) + 1000.0)
    assert len(calls) == 2  # the direct call above injected too (the hook is on the layer)
    for h in handles:
        h.remove()
    m(input_ids=ids, position_ids=pos)
    assert len(calls) == 2 and out.shape == (2, 5, 8)


def test_attach_engram_with_get_ids_and_layer_dtype():
    m = _Model().to(torch.float64)
    eng = _engram()
    seen = []
    eng.forward = lambda h, i, p=None: (seen.append((i, p)), h)[1]
    ids, pos = torch.zeros(1, 3, dtype=torch.long), torch.arange(3)[None]
    _name, handles = attach_engram(m, eng, 0, get_ids=lambda: (ids, pos))
    assert len(handles) == 1  # no pre-hook on the model when the ids come from get_ids
    assert eng.key.weight.dtype == torch.float64  # the layer's dtype
    m(input_ids=torch.ones(1, 3, dtype=torch.long))
    assert len(seen) == 1 and seen[0][0] is ids and seen[0][1] is pos
