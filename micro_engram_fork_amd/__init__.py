"""micro-engram's Engram lookup path on MI355X (gfx950): hand-written HIP kernels behind the
reference's MicroEngram module surface.

    from micro_engram_fork_amd import MicroEngram
    eng = MicroEngram(model_dim=5376, engram_dim=64, num_heads=8, orders=(2, 3, 4), ...).cuda()
    with torch.inference_mode():
        out = eng(hidden, input_ids, position_ids)

The compute lives in libmicro_engram_amd.so (C-ABI: include/micro_engram.h), built in-tree by
`python -m micro_engram_fork_amd._build`.
"""
from .module import (MicroEngram, attach_engram, check_loaded, default_seed,  # noqa: F401
                     engram_from_spec, find_text_layers, layer_device_dtype, resolve_order_sizes)

__all__ = ["MicroEngram", "attach_engram", "check_loaded", "default_seed", "engram_from_spec",
           "find_text_layers", "layer_device_dtype", "resolve_order_sizes"]
