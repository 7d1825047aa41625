"""The serving step's token-id matrix and media mask on the GPU: the surface of
micro_engram_vllm/ids.py, each call one HIP kernel (csrc/ids.hip).

fill_engram_ids runs before every model step (the runner's prepare_inputs); it reads no device
value back to the host, so it can run before each CUDA-graph replay. mask_media runs inside the
decoder layer's forward, so it is a registered custom op with a fake implementation.
"""
from typing import Optional, Tuple

import torch

from ._lib import ME_I32, ME_I64, call
from .ops import require_gpu, stream_of

_INT = {torch.int32: ME_I32, torch.int64: ME_I64}


def _int_code(t, what):
    try:
        return _INT[t.dtype]
    except KeyError:
        raise TypeError(f"[micro_engram] {what} must be int32 or int64, got {t.dtype}") from None


def _vec(t, n, what):
    if t.dim() != 1 or t.numel() < n:
        raise ValueError(f"[micro_engram] {what} must be 1-D with at least {n} entries, got {tuple(t.shape)}")
    return t if t.is_contiguous() else t.contiguous()


def fill_engram_ids(out: torch.Tensor, input_ids: torch.Tensor, positions: torch.Tensor,
                    idx_mapping: torch.Tensor, query_start_loc: torch.Tensor,
                    all_token_ids: torch.Tensor, num_reqs: int, num_tokens: int,
                    num_tokens_padded: int, media_ids: Optional[torch.Tensor] = None,
                    keep: Optional[torch.Tensor] = None) -> None:
    """out[t] = (token at t, token at t-1, ...), -1 where there is none, in place
    (micro_engram_vllm/ids.py:10-59); rows num_tokens..num_tokens_padded become -1.

    media_ids (optional): also apply mask_media (ids.py:62-70) in the same launch -- media ids
    in the written rows become -1, and `keep` (bool [>= num_tokens_padded], optional) gets
    False where the token itself is a media placeholder."""
    dev = require_gpu(out, input_ids, positions, idx_mapping, query_start_loc, all_token_ids,
                      media_ids, keep)
    if out.dim() != 2 or out.dtype != torch.int32 or out.stride(1) != 1:
        raise ValueError("[micro_engram] out must be a row-contiguous int32 [max_tokens, max_order] buffer")
    num_reqs, num_tokens, num_tokens_padded = int(num_reqs), int(num_tokens), int(num_tokens_padded)
    if not 0 <= num_tokens <= num_tokens_padded <= out.shape[0]:
        raise ValueError(f"[micro_engram] need 0 <= num_tokens ({num_tokens}) <= num_tokens_padded "
                         f"({num_tokens_padded}) <= out rows ({out.shape[0]})")
    ids = _vec(input_ids, num_tokens, "input_ids")
    pos = _vec(positions, num_tokens, "positions")
    imap = _vec(idx_mapping, num_reqs, "idx_mapping")
    qsl = _vec(query_start_loc, num_reqs + 1, "query_start_loc")
    if all_token_ids.dim() != 2:
        raise ValueError("[micro_engram] all_token_ids must be [max_num_reqs, max_model_len]")
    hist = all_token_ids if all_token_ids.stride(1) == 1 else all_token_ids.contiguous()
    n_media, media_ptr, media_code = 0, None, ME_I64
    if media_ids is not None:
        media = media_ids.reshape(-1).contiguous()
        n_media, media_ptr, media_code = media.numel(), media.data_ptr(), _int_code(media, "media_ids")
    keep_ptr = None
    if keep is not None:
        if keep.dtype not in (torch.bool, torch.uint8) or keep.numel() < num_tokens_padded or not keep.is_contiguous():
            raise ValueError("[micro_engram] keep must be a contiguous bool/uint8 buffer of >= num_tokens_padded")
        keep_ptr = keep.data_ptr()
    call("me_fill_engram_ids", out.data_ptr(), out.shape[0], out.stride(0), out.shape[1],
         ids.data_ptr(), _int_code(ids, "input_ids"), pos.data_ptr(), _int_code(pos, "positions"),
         imap.data_ptr(), _int_code(imap, "idx_mapping"), qsl.data_ptr(),
         _int_code(qsl, "query_start_loc"), hist.data_ptr(), _int_code(hist, "all_token_ids"),
         hist.shape[0], hist.shape[1], hist.stride(0), num_reqs, num_tokens, num_tokens_padded,
         media_ptr, media_code, n_media, keep_ptr, stream_of(dev))


@torch.library.custom_op("micro_engram_amd::mask_media", mutates_args=())
def mask_media(ids: torch.Tensor, media_ids: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(ids with media placeholder ids set to -1, keep [n] bool: False where the token itself is
    a media placeholder) (micro_engram_vllm/ids.py:62-70)."""
    dev = require_gpu(ids, media_ids)
    if ids.dim() != 2 or ids.stride(1) != 1:
        raise ValueError("[micro_engram] ids must be a row-contiguous [n, max_order] matrix")
    media = media_ids.reshape(-1).contiguous()
    n, width = ids.shape
    out = torch.empty((n, width), dtype=torch.int32, device=dev)
    keep = torch.empty(n, dtype=torch.bool, device=dev)
    call("me_mask_media", ids.data_ptr(), _int_code(ids, "ids"), n, width, ids.stride(0) if n else width,
         media.data_ptr() if media.numel() else None, _int_code(media, "media_ids"), media.numel(),
         out.data_ptr(), keep.data_ptr(), stream_of(dev))
    return (out if ids.dtype == torch.int32 else out.to(ids.dtype)), keep


@mask_media.register_fake
def _(ids, media_ids):
    return ids.new_empty(ids.shape), ids.new_empty(ids.shape[0], dtype=torch.bool)
