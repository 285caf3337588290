"""FP8 checkpoint format for the block-FP8 linear path.

A quantised linear weight is stored as two tensors (the layout FP8 checkpoints
on the Hugging Face Hub use for 128x128 block quantisation, e.g. DeepSeek-V3's
``quantization_config = {"quant_method": "fp8", "weight_block_size": [128, 128]}``):

    <prefix>.weight            float8_e4m3fn [N, K]
    <prefix>.weight_scale_inv  float32 [ceil(N/128), ceil(K/128)]

``weight_scale_inv`` is the per-block scale Bs that multiplies the fp8 values
back (W ~= Wq * Bs), i.e. exactly the (B, Bs) operands of
``w8a8_block_fp8_matmul``. Files are safetensors (no pickle).
"""
from __future__ import annotations

from pathlib import Path
from typing import Callable, Dict, Iterable, Tuple

import torch

SCALE_SUFFIX = "weight_scale_inv"
BLOCK = 128


def _scale_name(weight_name: str) -> str:
    assert weight_name.endswith("weight"), weight_name
    return weight_name[: -len("weight")] + SCALE_SUFFIX


def _default_select(name: str, t: torch.Tensor) -> bool:
    return (name.endswith(".weight") and t.dim() == 2 and t.is_floating_point()
            and t.dtype != torch.float8_e4m3fn and min(t.shape) >= BLOCK)


def quantize_state_dict(state_dict: Dict[str, torch.Tensor], device="cuda",
                        select: Callable[[str, torch.Tensor], bool] = _default_select
                        ) -> Dict[str, torch.Tensor]:
    """Quantise the selected 2-D weights with the GPU block quantiser
    (quantize_weight); other tensors are copied unchanged. Returns CPU tensors
    in the checkpoint layout above."""
    from . import quantize_weight
    out: Dict[str, torch.Tensor] = {}
    for name, t in state_dict.items():
        if select(name, t):
            w = t.to(device)
            if w.dtype not in (torch.float32, torch.bfloat16):
                w = w.float()
            q, s = quantize_weight(w)
            out[name] = q.cpu()
            out[_scale_name(name)] = s.cpu()
        else:
            out[name] = t.detach().cpu()
    return out


def fp8_linear_weights(state_dict: Dict[str, torch.Tensor]
                       ) -> Dict[str, Tuple[torch.Tensor, torch.Tensor]]:
    """The (Wq, Bs) pairs of a checkpoint dict, keyed by weight name, after
    checking dtypes and the 128x128 scale shape."""
    pairs = {}
    for name, t in state_dict.items():
        if not (name.endswith("weight") and t.dtype == torch.float8_e4m3fn):
            continue
        sname = _scale_name(name)
        if sname not in state_dict:
            raise ValueError(f"{name}: float8 weight without {sname}")
        s = state_dict[sname]
        N, K = t.shape
        want = (-(-N // BLOCK), -(-K // BLOCK))
        if s.dtype != torch.float32 or tuple(s.shape) != want:
            raise ValueError(f"{sname}: expected float32 {list(want)}, got {s.dtype} "
                             f"{list(s.shape)}")
        pairs[name] = (t, s)
    return pairs


def save_fp8_checkpoint(path, state_dict: Dict[str, torch.Tensor]) -> None:
    from safetensors.torch import save_file
    save_file({k: v.contiguous().cpu() for k, v in state_dict.items()}, str(path))


def load_fp8_checkpoint(paths, device="cpu") -> Dict[str, torch.Tensor]:
    """Load one or more safetensors files (e.g. the shards of a Hub FP8
    checkpoint) into one dict on ``device``."""
    from safetensors.torch import load_file
    if isinstance(paths, (str, Path)):
        paths = [paths]
    out: Dict[str, torch.Tensor] = {}
    for p in paths:
        out.update(load_file(str(p), device=str(device)))
    return out
