"""Engram weights on disk: the files micro-engram writes, read back into a MicroEngram.

Tensors are named relative to the engram (tables.0.weight, key.weight, value.weight,
q_scale, k_scale, mults, canon), or with the full name of the model they sit in
(model.language_model.layers.29.micro_engram.tables.0.weight; FSDP inserts
_checkpoint_wrapped_module before micro_engram). The scales are stored as the scale itself
(1 + delta, fp32); MicroEngram's state-dict hooks convert (micro_engram/module.py:156-181).

Formats read (micro_engram/weights.py:112-142):
  *.pt                      torch.save of a dict (micro_engram.pt: local names; nested dicts
                            are flattened with dots). Read with weights_only=True: nothing in
                            the file is executed.
  *.safetensors             one file, full or local names
  folder of *.safetensors   a merged or assembled model (only engram tensors are read)
  DCP folder (.metadata)    torch.distributed.checkpoint, e.g. checkpoint-N/pytorch_model_fsdp_0
                            or micro_engram_rows; only the engram tensors are read, in one
                            process (no process group)
Formats written (save_engram_weights): the same four, so a trained engram leaves this package
in a form the reference's loaders read.

micro_engram_config.json (micro_engram/weights.py:152-246, runconfig.py:40-67) says which
engrams a run has (layer, sizes, orders, gate, seed, canon, weights path); engram_specs and
resolve_engram_source turn it into constructor arguments for engram_from_spec.
"""
import glob
import hashlib
import json
import os
import re

import torch

from .module import SEED_STRIDE, default_seed  # noqa: F401  (re-exported: weights.py:152-160)

TAG = "micro_engram."
CONFIG_NAME = "micro_engram_config.json"
ENGRAM_FILE = "micro_engram.safetensors"  # assemble_engram_model.py:37

# decoder layer of a full name: "...layers.<L>.[_checkpoint_wrapped_module.]micro_engram."
_LAYER_KEY = re.compile(r"(?:^|\.)layers\.(\d+)\.(?:_checkpoint_wrapped_module\.)?micro_engram\.")
_CHECKPOINT_DIR = re.compile(r"checkpoint-(\d+)$")
_SPEC_FIELDS = ("layer", "table_size", "table_sizes", "engram_dim", "num_heads", "orders", "gate",
                "seed", "pad_id", "token_merge", "canon_path", "frozen", "init_from")


# ----------------------------------------------------------------------------- tensor names
def local_name(key):
    """Name inside the engram ('tables.0.weight') of a full tensor name, or None when the key is
    not an engram tensor (weights.py:28-36)."""
    mark = "." + TAG
    if mark in key:
        return key.split(mark, 1)[1]
    return key[len(TAG):] if key.startswith(TAG) else None


def layer_of_key(key):
    """Decoder layer a full engram tensor name belongs to, or None (weights.py:39-45)."""
    m = _LAYER_KEY.search(key)
    return None if m is None else int(m.group(1))


def _is_wanted(key, layer):
    """An engram tensor of `layer` (of any layer when None; names without a layer always)."""
    if local_name(key) is None:
        return False
    found = layer_of_key(key)
    return layer is None or found is None or found == layer


def full_name(layer, local, prefix="model.language_model.layers"):
    """The name an engram tensor has inside a model: <prefix>.<layer>.micro_engram.<local>."""
    return f"{prefix}.{int(layer)}.{TAG}{local}"


def _flatten(tree, prefix=""):
    flat = {}
    for k, v in tree.items():
        if isinstance(v, dict):
            flat.update(_flatten(v, f"{prefix}{k}."))
        else:
            flat[f"{prefix}{k}"] = v
    return flat


def _localised(sd, layer):
    return {local_name(k): v for k, v in sd.items() if torch.is_tensor(v) and _is_wanted(k, layer)}


# ----------------------------------------------------------------------------- readers
def _is_dcp(path):
    return os.path.isdir(path) and os.path.isfile(os.path.join(path, ".metadata"))


def _safetensors_files(path):
    return sorted(glob.glob(os.path.join(path, "*.safetensors"))) if os.path.isdir(path) else [path]


def _read_dcp(folder, layer):
    """Only the engram tensors of a DCP checkpoint, read in this process (weights.py:59-73)."""
    import torch.distributed.checkpoint as dcp
    from torch.distributed.checkpoint.metadata import TensorStorageMetadata

    reader = dcp.FileSystemReader(folder)
    meta = reader.read_metadata().state_dict_metadata
    out = {k: torch.empty(tuple(m.size), dtype=m.properties.dtype) for k, m in meta.items()
           if isinstance(m, TensorStorageMetadata) and _is_wanted(k, layer)}
    if out:
        dcp.load(out, storage_reader=reader, no_dist=True)
    return _localised(out, layer)


def _read_safetensors(files, layer):
    from safetensors import safe_open

    out = {}
    for f in files:
        with safe_open(f, framework="pt", device="cpu") as fh:
            for k in fh.keys():
                if _is_wanted(k, layer):
                    out[local_name(k)] = fh.get_tensor(k)
    return out


def _unlayered(sd, path, layer, need_layer):
    """A file saved with local names carries no layer; shared by several engrams it would give
    each the same tensors, so that is an error when need_layer (weights.py:144-150)."""
    if need_layer and layer is not None and any(k.startswith("tables.") for k in sd):
        raise ValueError(f"[micro_engram] {path} is used by several engrams, but its tensor names have "
                         f"no layer number (e.g. {next(iter(sd))}), so it can't tell which is layer "
                         f"{layer}'s. Give each engram its own file, or keep the full names "
                         f"(...layers.{layer}.micro_engram.tables.0.weight)")
    return sd


def load_engram_weights(path, layer=None, need_layer=False):
    """{local name: CPU tensor} of the engram stored at `path` (a .pt, a .safetensors file, a
    folder of .safetensors, or a DCP folder); with `layer`, only that decoder layer's engram
    (weights.py:112-141)."""
    path = os.path.abspath(path)
    if _is_dcp(path):
        return _read_dcp(path, layer)
    if os.path.isdir(path):
        return _read_safetensors(_safetensors_files(path), layer)
    if path.endswith(".safetensors"):
        sd = _read_safetensors([path], layer)
        if sd:
            return sd
        from safetensors.torch import load_file

        return _unlayered(load_file(path), path, layer, need_layer)
    tree = torch.load(path, map_location="cpu", weights_only=True)
    flat = _flatten(tree)
    sd = _localised(flat, layer)
    if sd:
        return sd
    return _unlayered({k: v for k, v in flat.items() if torch.is_tensor(v)}, path, layer, need_layer)


def engram_layers_in(path):
    """Sorted decoder layers whose engram tensors are stored at `path` (weights.py:88-109)."""
    path = os.path.abspath(path)
    if _is_dcp(path):
        import torch.distributed.checkpoint as dcp

        keys = list(dcp.FileSystemReader(path).read_metadata().state_dict_metadata)
    elif os.path.isdir(path) or path.endswith(".safetensors"):
        from safetensors import safe_open

        keys = []
        for f in _safetensors_files(path):
            with safe_open(f, framework="pt", device="cpu") as fh:
                keys.extend(fh.keys())
    else:
        keys = list(_flatten(torch.load(path, map_location="cpu", weights_only=True)))
    return sorted({layer_of_key(k) for k in keys
                   if local_name(k) is not None and layer_of_key(k) is not None})


# ----------------------------------------------------------------------------- writers
def engram_state(engram):
    """The engram's tensors under their local names, on the CPU, scales as 1 + delta (fp32). A
    row-sharded engram on one GPU contributes its row shards as the tables."""
    sd = {k: v.detach().cpu() for k, v in engram.state_dict().items()}
    shards = getattr(engram, "row_shards", None)
    if shards is not None:
        for k, p in enumerate(shards):
            sd[f"tables.{k}.weight"] = p.detach().cpu()
    return sd


def save_engram_weights(engram, path, layer=None, fmt=None, prefix="model.language_model.layers"):
    """Write the engram in one of the formats load_engram_weights reads. fmt: "pt" (local names,
    like micro_engram.pt), "safetensors" (one file), "safetensors_dir" (a folder with
    micro_engram.safetensors) or "dcp" (a DCP folder); by default from the path's suffix (a path
    without one is a DCP folder). With `layer`, tensors get full names (several engrams can
    share one file); "safetensors_dir" and "dcp" need it, as model checkpoints have them."""
    if fmt is None:
        fmt = "pt" if path.endswith(".pt") else "safetensors" if path.endswith(".safetensors") else "dcp"
    sd = engram_state(engram)
    if layer is not None:
        sd = {full_name(layer, k, prefix): v for k, v in sd.items()}
    elif fmt in ("safetensors_dir", "dcp"):
        raise ValueError(f"[micro_engram] a {fmt} engram checkpoint needs the decoder layer (full names)")
    if fmt == "pt":
        torch.save(sd, path)
    elif fmt in ("safetensors", "safetensors_dir"):
        from safetensors.torch import save_file

        if fmt == "safetensors_dir":
            os.makedirs(path, exist_ok=True)
            path = os.path.join(path, ENGRAM_FILE)
        save_file({k: v.contiguous() for k, v in sd.items()}, path)
    elif fmt == "dcp":
        import torch.distributed.checkpoint as dcp

        dcp.save(sd, checkpoint_id=path, no_dist=True)
    else:
        raise ValueError(f"[micro_engram] unknown weights format {fmt!r}")
    return path


# ----------------------------------------------------------------------------- configs
def norm_table_sizes(sizes):
    """{order: rows or None} with integer orders (JSON keys are strings), or None
    (weights.py:162-166)."""
    if not sizes:
        return None
    return {int(order): (int(rows) if rows else None) for order, rows in dict(sizes).items()}


def resolve_weights_path(conf, conf_path):
    """The top-level "weights" of a config, relative to the config's folder, or None
    (weights.py:143-150)."""
    w = conf.get("weights")
    if not w:
        return None
    return w if os.path.isabs(w) else os.path.join(os.path.dirname(os.path.abspath(conf_path)), w)


def engram_specs(conf, conf_path=None):
    """One settings dict per engram of a micro_engram_config.json (weights.py:172-200): the
    "engrams" list, or the single engram described at the top level by older configs. Each
    entry inherits the top-level fields it leaves unset; layer defaults to 0, orders to (2, 3),
    gate to "scalar" and seed to 0 (configs from before seeds were recorded); "weights" is
    resolved against the config's folder. Two engrams in one layer are an error."""
    top = {k: conf.get(k) for k in _SPEC_FIELDS}
    entries = conf.get("engrams") or [{**top, "weights": conf.get("weights")}]
    specs = []
    for entry in entries:
        spec = dict(top)
        spec.update({k: v for k, v in entry.items() if v is not None or k == "weights"})
        spec["layer"] = int(spec.get("layer") or 0)
        spec["orders"] = tuple(spec.get("orders") or (2, 3))
        spec["table_sizes"] = norm_table_sizes(spec.get("table_sizes"))
        spec["gate"] = spec.get("gate") or "scalar"
        spec["seed"] = int(spec["seed"]) if spec.get("seed") is not None else 0
        w = entry.get("weights")
        if w and conf_path and not os.path.isabs(w):
            w = os.path.join(os.path.dirname(os.path.abspath(conf_path)), w)
        spec["weights"] = w or None
        specs.append(spec)
    layers = [s["layer"] for s in specs]
    if len(set(layers)) != len(layers):
        raise ValueError(f"[micro_engram] two engrams in the same layer: {layers}")
    return specs


def latest_checkpoint(folder):
    """The newest complete checkpoint-N in `folder` (trainer_state.json is written last), or
    None (weights.py:206-211)."""
    best = None
    for c in glob.glob(os.path.join(folder, "checkpoint-*")):
        m = _CHECKPOINT_DIR.search(c)
        if m and os.path.isfile(os.path.join(c, "trainer_state.json")):
            if best is None or int(m.group(1)) > best[0]:
                best = (int(m.group(1)), c)
    return None if best is None else best[1]


def spec_for_layer(conf_path, layer):
    """The settings of the engram at `layer` in the config at conf_path (weights.py:239-246)."""
    with open(conf_path) as f:
        specs = engram_specs(json.load(f), conf_path)
    for spec in specs:
        if spec["layer"] == layer:
            return spec
    raise ValueError(f"[micro_engram] {conf_path} has no engram at layer {layer} "
                     f"(it has layers {[s['layer'] for s in specs]})")


def resolve_engram_source(path, layer):
    """(weights path, settings or None) of the trained engram for decoder `layer`
    (weights.py:214-236). `path`: a micro_engram_config.json, a folder holding one (a
    checkpoint-N, an assembled model, or an output_dir whose newest checkpoint is used), or the
    weights themselves."""
    path = os.path.abspath(path)
    conf_path = path if path.endswith(".json") else os.path.join(path, CONFIG_NAME)
    if os.path.isdir(path) and not _is_dcp(path):
        has_conf = os.path.isfile(conf_path)
        has_weights = bool(glob.glob(os.path.join(path, "*.safetensors")))
        ckpt = None if has_weights else latest_checkpoint(path)
        if ckpt is not None:
            weights, spec = resolve_engram_source(ckpt, layer)
            if spec is None and has_conf:
                spec = spec_for_layer(conf_path, layer)
            return weights, spec
    if os.path.isfile(conf_path):
        spec = spec_for_layer(conf_path, layer)
        return spec["weights"] or os.path.dirname(conf_path), spec
    return path, None


def check_canon(canon, vocab_size):
    """A token-merge map read from disk, validated (runconfig.py:91-100): 1-D of vocab_size ids
    inside the vocabulary, and idempotent (canon[canon] == canon)."""
    if not torch.is_tensor(canon) or canon.dim() != 1 or canon.numel() != vocab_size:
        raise ValueError(f"[micro_engram] canon file must be a 1-D tensor of length {vocab_size}")
    canon = canon.long()
    if int(canon.min()) < 0 or int(canon.max()) >= vocab_size:
        raise ValueError("[micro_engram] canon file has ids outside the vocabulary")
    if not torch.equal(canon[canon], canon):
        raise ValueError("[micro_engram] canon map is not idempotent (a canonical id must map to itself)")
    return canon


# ----------------------------------------------------------------------------- base check
_FP_PROJ = re.compile(r"^(.*\.layers\.)(\d+)\.(self_attn\.[qkvo]_proj|mlp\.(?:gate|up|down)_proj)\.weight$")
_FP_ROWS = 64


def _model_weight_files(model_dir):
    index = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.isfile(index):
        with open(index) as f:
            return {k: os.path.join(model_dir, v) for k, v in json.load(f)["weight_map"].items()}
    from safetensors import safe_open

    files = {}
    for f in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        with safe_open(f, framework="pt", device="cpu") as fh:
            files.update({k: f for k in fh.keys()})
    return files


def base_fingerprint(model_dir):
    """16 hex digits identifying a base model's weights (weights.py:266-310): SHA-256 over the
    first 64 rows of the token embedding and of the attention / MLP projections of the first,
    middle and last decoder layer, each tagged by its role (not its name), dtype and shape. None
    without safetensors weights."""
    from safetensors import safe_open

    if not os.path.isdir(model_dir):
        return None
    files = {k: f for k, f in _model_weight_files(model_dir).items()
             if TAG not in k and "vision" not in k and "audio" not in k}
    if not files:
        return None
    roles = {"embed": k for k in files if k.endswith("embed_tokens.weight")}
    by_layer = {}
    for k in files:
        m = _FP_PROJ.match(k)
        if m:
            by_layer.setdefault(int(m.group(2)), {})[m.group(3)] = k
    if by_layer:
        ids = sorted(by_layer)
        for where, i in (("first", ids[0]), ("middle", ids[len(ids) // 2]), ("last", ids[-1])):
            roles.update({f"{where}.{r}": k for r, k in by_layer[i].items()})
    if not roles:
        return None
    h = hashlib.sha256()
    for role in sorted(roles):
        k = roles[role]
        with torch.device("cpu"), safe_open(files[k], framework="pt", device="cpu") as fh:
            t = fh.get_slice(k)[:_FP_ROWS].contiguous().cpu()
        h.update(role.encode())
        h.update(str((t.dtype, tuple(t.shape))).encode())
        h.update(t.view(torch.uint8).numpy().tobytes())
    return h.hexdigest()[:16]


def base_mismatch(conf, model_dir):
    """A warning text when the engram was trained on other base weights, else None
    (weights.py:313-328). It never raises: a failed check is reported as a warning."""
    want = conf.get("base_fingerprint")
    if not want:
        return None
    try:
        have = base_fingerprint(model_dir)
    except Exception as e:  # noqa: BLE001
        return f"could not check which base weights this engram was trained on ({type(e).__name__}: {e})"
    if have is None or have == want:
        return None
    return (f"this engram was trained on different base weights (trained on {conf.get('base_model', '?')}, "
            f"fingerprint {want}; this model: {have}). It still loads, but it injects into hidden "
            f"states it never saw: expect worse output unless this is really the same base.")


def load_engram(path, layer, model_dim, vocab_size, device=None, dtype=None, pad_default=0):
    """A MicroEngram for decoder `layer` rebuilt from a trained one at `path` (any form
    resolve_engram_source takes): its settings (seed included, which fixes every hash address)
    from the config, its tensors checked and loaded (check_loaded), the canon map validated.
    Without a config the settings cannot be known and this raises."""
    from .module import check_loaded, engram_from_spec

    weights, spec = resolve_engram_source(path, layer)
    if spec is None:
        raise ValueError(f"[micro_engram] {path}: no {CONFIG_NAME} found, so the engram's settings "
                         f"(sizes, orders, seed) are unknown")
    sd = load_engram_weights(weights, layer=layer, need_layer=True)
    canon = sd.get("canon")
    if canon is not None:
        canon = check_canon(canon, vocab_size)
    eng = engram_from_spec(spec, model_dim, vocab_size, pad_default=pad_default, canon=canon)
    check_loaded(eng, sd, weights)
    return eng.to(device=device, dtype=dtype) if (device is not None or dtype is not None) else eng
