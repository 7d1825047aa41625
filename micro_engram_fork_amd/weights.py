"""Engram weights on disk: reading the files a trained engram is kept in, and writing them.

What is on disk is fixed by the reference (micro_engram/weights.py:112-202, runconfig.py:40-67,
module.py:166-181); how it is read here is this package's own:

  * an engram tensor is named either locally ("tables.0.weight", "key.weight", "q_scale",
    "mults", "canon", ...) or by its place in a model, "<...>.layers.<L>.micro_engram.<local>",
    possibly with FSDP's "_checkpoint_wrapped_module." before "micro_engram" -- EngramKey
    parses both;
  * the scales are stored as the scale itself (1 + the module's delta, fp32); MicroEngram's
    state-dict hooks convert;
  * four containers hold the tensors -- a torch.save'd dict (.pt, read with weights_only=True,
    so nothing in the file runs; nested dicts flatten with dots), one .safetensors file, a
    folder of .safetensors files (a merged or assembled model), and a torch.distributed
    checkpoint folder (a ".metadata" file: a trainer's pytorch_model_fsdp_0 or a
    micro_engram_rows folder), read in this process without a process group. Each is a
    TensorSource: list the names, read the ones wanted.

micro_engram_config.json describes a run's engrams (layer, sizes, orders, gate, seed, canon,
weights); engram_specs turns it into one settings dict per engram for engram_from_spec, and
resolve_engram_source finds the config and weights of a layer from a config file, a checkpoint
folder, a training output folder or the weights themselves.
"""
import glob
import json
import os
import re

import torch

from .module import SEED_STRIDE, default_seed  # noqa: F401  (the seed rule, weights.py:157)

CONFIG_NAME = "micro_engram_config.json"
ENGRAM_FILE = "micro_engram.safetensors"  # an assembled model's engram file
MODULE_NAME = "micro_engram"

# ".layers.<L>." then an optional FSDP wrapper, then the engram module
_PLACED = re.compile(r"(?:^|\.)layers\.(?P<layer>\d+)\.(?:_checkpoint_wrapped_module\.)?"
                     + MODULE_NAME + r"\.(?P<local>.+)$")
_CHECKPOINT = re.compile(r"^checkpoint-(\d+)$")

# settings an engram entry of the config may carry (the rest of a config is not the engram's)
SPEC_KEYS = ("layer", "table_size", "table_sizes", "engram_dim", "num_heads", "orders", "gate",
             "seed", "pad_id", "token_merge", "canon_path", "frozen", "init_from")


# ------------------------------------------------------------------------------ names
class EngramKey:
    """A parsed tensor name: `local` is the name inside the engram, `layer` the decoder layer
    (None for local names and for names under a bare "micro_engram." prefix)."""

    __slots__ = ("layer", "local")

    def __init__(self, layer, local):
        self.layer, self.local = layer, local

    @classmethod
    def parse(cls, name):
        """The EngramKey of `name`, or None for tensors that are not an engram's."""
        m = _PLACED.search(name)
        if m is not None:
            return cls(int(m.group("layer")), m.group("local"))
        head = MODULE_NAME + "."
        if name.startswith(head):
            return cls(None, name[len(head):])
        mid = "." + head
        if mid in name:
            return cls(None, name.split(mid, 1)[1])
        return None

    def belongs_to(self, layer):
        """Whether the tensor is part of decoder `layer`'s engram: any engram when layer is None;
        a name without a layer fits every layer."""
        return layer is None or self.layer is None or self.layer == layer


def local_name(name):
    """Name of an engram tensor inside the engram, or None when `name` is not one."""
    key = EngramKey.parse(name)
    return None if key is None else key.local


def layer_of_key(name):
    """Decoder layer of a full engram tensor name, or None."""
    key = EngramKey.parse(name)
    return None if key is None else key.layer


def full_name(layer, local, prefix="model.language_model.layers"):
    """The name the tensor `local` of decoder `layer`'s engram has inside a model."""
    return f"{prefix}.{int(layer)}.{MODULE_NAME}.{local}"


# ------------------------------------------------------------------------------ containers
class TensorSource:
    """A weights container: names() lists every tensor name in it, read(names) returns
    {name: CPU tensor} for the ones asked for."""

    def __init__(self, path):
        self.path = path

    def names(self):
        raise NotImplementedError

    def read(self, names):
        raise NotImplementedError


class _DcpSource(TensorSource):
    def _meta(self):
        import torch.distributed.checkpoint as dcp

        return dcp.FileSystemReader(self.path).read_metadata().state_dict_metadata

    def names(self):
        from torch.distributed.checkpoint.metadata import TensorStorageMetadata

        return [k for k, m in self._meta().items() if isinstance(m, TensorStorageMetadata)]

    def read(self, names):
        import torch.distributed.checkpoint as dcp

        meta = self._meta()
        out = {k: torch.empty(tuple(meta[k].size), dtype=meta[k].properties.dtype) for k in names}
        if out:
            dcp.load(out, storage_reader=dcp.FileSystemReader(self.path), no_dist=True)
        return out


class _SafetensorsSource(TensorSource):
    def __init__(self, path, files):
        super().__init__(path)
        self.files = files

    def _index(self):
        from safetensors import safe_open

        where = {}
        for f in self.files:
            with safe_open(f, framework="pt", device="cpu") as fh:
                for k in fh.keys():
                    where[k] = f
        return where

    def names(self):
        return list(self._index())

    def read(self, names):
        from safetensors import safe_open

        by_file = {}
        index = self._index()
        for k in names:
            by_file.setdefault(index[k], []).append(k)
        out = {}
        for f, ks in by_file.items():
            with safe_open(f, framework="pt", device="cpu") as fh:
                out.update({k: fh.get_tensor(k) for k in ks})
        return out


class _PtSource(TensorSource):
    def _flat(self):
        if getattr(self, "_loaded", None) is not None:
            return self._loaded
        tree = torch.load(self.path, map_location="cpu", weights_only=True)
        flat, todo = {}, [("", tree)]
        while todo:
            prefix, node = todo.pop()
            for k, v in node.items():
                if isinstance(v, dict):
                    todo.append((f"{prefix}{k}.", v))
                elif torch.is_tensor(v):
                    flat[f"{prefix}{k}"] = v
        self._loaded = flat
        return flat

    def names(self):
        return list(self._flat())

    def read(self, names):
        flat = self._flat()
        return {k: flat[k] for k in names}


def open_source(path):
    """The TensorSource for `path`: a DCP folder (it has .metadata), a folder of .safetensors, a
    .safetensors file, or anything else as a torch.save'd dict."""
    path = os.path.abspath(path)
    if os.path.isdir(path):
        if os.path.isfile(os.path.join(path, ".metadata")):
            return _DcpSource(path)
        return _SafetensorsSource(path, sorted(glob.glob(os.path.join(path, "*.safetensors"))))
    if path.endswith(".safetensors"):
        return _SafetensorsSource(path, [path])
    return _PtSource(path)


def is_dcp_folder(path):
    return os.path.isdir(path) and os.path.isfile(os.path.join(path, ".metadata"))


# ------------------------------------------------------------------------------ reading
def load_engram_weights(path, layer=None, need_layer=False):
    """{local name: CPU tensor} of the engram stored at `path`, only decoder `layer`'s engram when
    a layer is given. A file of plain local names (no "micro_engram." anywhere, like
    micro_engram.pt) is the engram itself; if it may be shared by several engrams
    (need_layer with a layer given), it cannot tell which layer it is for and is refused."""
    src = open_source(path)
    names = src.names()
    wanted = {}
    for name in names:
        key = EngramKey.parse(name)
        if key is not None and key.belongs_to(layer):
            wanted[name] = key.local
    if wanted:
        return {wanted[k]: v for k, v in src.read(list(wanted)).items()}
    if os.path.isdir(src.path):
        return {}  # a checkpoint or model folder without this engram
    # a single file with nothing named as an engram tensor holds the engram under local names
    if need_layer and layer is not None and any(n.startswith("tables.") for n in names):
        raise ValueError(
            f"[micro_engram] {path} names its tensors without a decoder layer ({names[0]}, ...), and "
            f"several engrams read it: there is no telling which tensors are layer {layer}'s. Save "
            f"each engram to its own file, or under full names (...layers.{layer}.micro_engram.*)")
    return src.read(names)


def engram_layers_in(path):
    """The decoder layers, sorted, that have engram tensors at `path`."""
    layers = set()
    for name in open_source(path).names():
        key = EngramKey.parse(name)
        if key is not None and key.layer is not None:
            layers.add(key.layer)
    return sorted(layers)


# ------------------------------------------------------------------------------ writing
def engram_state(engram):
    """The engram's tensors under local names on the CPU, scales as 1 + delta in fp32; a
    row-sharded engram on one GPU gives its shards (each a whole table) as the tables."""
    state = {k: v.detach().cpu() for k, v in engram.state_dict().items()}
    for k, shard in enumerate(getattr(engram, "row_shards", None) or []):
        state[f"tables.{k}.weight"] = shard.detach().cpu()
    return state


_WRITERS = {}


def _writer(fmt):
    def register(fn):
        _WRITERS[fmt] = fn
        return fn

    return register


@_writer("pt")
def _write_pt(state, path):
    torch.save(state, path)
    return path


@_writer("safetensors")
def _write_safetensors(state, path):
    from safetensors.torch import save_file

    save_file({k: v.contiguous() for k, v in state.items()}, path)
    return path


@_writer("safetensors_dir")
def _write_safetensors_dir(state, path):
    os.makedirs(path, exist_ok=True)
    return _write_safetensors(state, os.path.join(path, ENGRAM_FILE))


@_writer("dcp")
def _write_dcp(state, path):
    import torch.distributed.checkpoint as dcp

    dcp.save(state, checkpoint_id=path, no_dist=True)
    return path


def save_engram_weights(engram, path, layer=None, fmt=None, prefix="model.language_model.layers"):
    """Write the engram where load_engram_weights (and the reference's loaders) read it back.
    fmt: "pt", "safetensors", "safetensors_dir" (a folder with micro_engram.safetensors) or "dcp";
    by default from the suffix of `path` (none: a DCP folder). With `layer` the tensors get full
    names, so one file can hold several engrams; the two folder formats are model checkpoints and
    need it. Returns the path written."""
    if fmt is None:
        fmt = {".pt": "pt", ".safetensors": "safetensors"}.get(os.path.splitext(path)[1], "dcp")
    if fmt not in _WRITERS:
        raise ValueError(f"[micro_engram] no writer for weights format {fmt!r} (have {sorted(_WRITERS)})")
    state = engram_state(engram)
    if layer is not None:
        state = {full_name(layer, k, prefix): v for k, v in state.items()}
    elif fmt in ("safetensors_dir", "dcp"):
        raise ValueError(f"[micro_engram] the {fmt} format is a model checkpoint: give the decoder layer")
    return _WRITERS[fmt](state, path)


# ------------------------------------------------------------------------------ configs
def norm_table_sizes(sizes):
    """Per-order table sizes with integer orders (JSON object keys are strings) and 0 as None;
    None when there are none."""
    if not sizes:
        return None
    return {int(order): int(rows) if rows else None for order, rows in dict(sizes).items()}


def _relative_to(conf_path, target):
    """`target` read relative to the folder of the config file (absolute paths unchanged)."""
    if not target or os.path.isabs(target) or not conf_path:
        return target or None
    return os.path.join(os.path.dirname(os.path.abspath(conf_path)), target)


def resolve_weights_path(conf, conf_path):
    """The config's top-level "weights", relative to the config's folder, or None."""
    return _relative_to(conf_path, conf.get("weights"))


def _normalise(spec):
    """Defaults of configs that predate a field: layer 0, orders (2, 3), the scalar gate, seed 0."""
    spec["layer"] = int(spec.get("layer") or 0)
    spec["orders"] = tuple(spec.get("orders") or (2, 3))
    spec["table_sizes"] = norm_table_sizes(spec.get("table_sizes"))
    spec["gate"] = spec.get("gate") or "scalar"
    spec["seed"] = 0 if spec.get("seed") is None else int(spec["seed"])
    return spec


def engram_specs(conf, conf_path=None):
    """Settings of each engram of a micro_engram_config.json: the entries of its "engrams" list,
    each taking the top-level value of any setting it leaves unset, or -- in configs from before
    several engrams -- one engram described by the top level itself. "weights" is per entry and
    read relative to the config's folder. Raises if two engrams share a layer."""
    shared = {k: conf.get(k) for k in SPEC_KEYS}
    entries = conf.get("engrams")
    if not entries:
        entries = [dict(shared, weights=conf.get("weights"))]
    specs = []
    for entry in entries:
        own = {k: v for k, v in entry.items() if v is not None}
        spec = _normalise({**shared, **own})
        spec["weights"] = _relative_to(conf_path, entry.get("weights"))
        specs.append(spec)
    layers = sorted(s["layer"] for s in specs)
    if len(set(layers)) < len(layers):
        raise ValueError(f"[micro_engram] the config puts more than one engram in a layer: layers {layers}")
    return specs


def latest_checkpoint(folder):
    """The checkpoint-N folder in `folder` with the largest N among the complete ones (the
    trainer writes trainer_state.json last), or None."""
    done = []
    for sub in glob.glob(os.path.join(folder, "checkpoint-*")):
        m = _CHECKPOINT.match(os.path.basename(sub))
        if m and os.path.isfile(os.path.join(sub, "trainer_state.json")):
            done.append((int(m.group(1)), sub))
    return max(done)[1] if done else None


def spec_for_layer(conf_path, layer):
    """Settings of decoder `layer`'s engram in the config file conf_path."""
    with open(conf_path) as f:
        specs = {s["layer"]: s for s in engram_specs(json.load(f), conf_path)}
    if layer not in specs:
        raise ValueError(f"[micro_engram] {conf_path} has no engram at layer {layer}; its engrams are at "
                         f"layers {sorted(specs)}")
    return specs[layer]


def resolve_engram_source(path, layer):
    """(weights path, settings or None) of decoder `layer`'s trained engram, from
      * a micro_engram_config.json file, or a folder that has one next to its weights;
      * a training output folder: its newest complete checkpoint-N (settings from that
        checkpoint's config, else the output folder's);
      * the weights themselves (settings unknown: None)."""
    path = os.path.abspath(path)
    config = path if path.endswith(".json") else os.path.join(path, CONFIG_NAME)
    folder_of_weights = os.path.isdir(path) and not is_dcp_folder(path)
    if folder_of_weights and not glob.glob(os.path.join(path, "*.safetensors")):
        newest = latest_checkpoint(path)
        if newest is not None:
            weights, spec = resolve_engram_source(newest, layer)
            if spec is None and os.path.isfile(config):
                spec = spec_for_layer(config, layer)
            return weights, spec
    if os.path.isfile(config):
        spec = spec_for_layer(config, layer)
        return (spec["weights"] or os.path.dirname(config)), spec
    return path, None


def check_canon(canon, vocab_size):
    """A token-merge map read from disk, checked as the reference's config loader checks it
    (runconfig.py:91-100): 1-D, vocab_size long, ids inside the vocabulary, idempotent
    (canon[canon] == canon: a canonical id maps to itself). Returns it as int64."""
    if not torch.is_tensor(canon) or canon.dim() != 1 or canon.numel() != vocab_size:
        raise ValueError(f"[micro_engram] a canon map is a 1-D tensor with one id per token: length "
                         f"{vocab_size} expected")
    canon = canon.long()
    if canon.numel() and (int(canon.min()) < 0 or int(canon.max()) >= vocab_size):
        raise ValueError(f"[micro_engram] the canon map points outside the vocabulary [0, {vocab_size})")
    if not torch.equal(canon[canon], canon):
        raise ValueError("[micro_engram] the canon map is not idempotent: some token maps to an id that "
                         "is not its own canonical id")
    return canon


def load_engram(path, layer, model_dim, vocab_size, device=None, dtype=None, pad_default=0):
    """A MicroEngram rebuilt from decoder `layer`'s trained engram at `path` (any form
    resolve_engram_source accepts): settings, the seed among them (it fixes every hash
    address), from the config; tensors loaded and checked against those settings; the canon map
    validated. Without a config the settings are unknown, and this raises."""
    from .module import check_loaded, engram_from_spec

    weights, spec = resolve_engram_source(path, layer)
    if spec is None:
        raise ValueError(f"[micro_engram] found no {CONFIG_NAME} for {path}: the engram's sizes, orders "
                         "and seed are unknown")
    state = load_engram_weights(weights, layer=layer, need_layer=True)
    canon = state.get("canon")
    engram = engram_from_spec(spec, model_dim, vocab_size, pad_default=pad_default,
                              canon=None if canon is None else check_canon(canon, vocab_size))
    check_loaded(engram, state, weights)
    if device is None and dtype is None:
        return engram
    return engram.to(device=device, dtype=dtype)
