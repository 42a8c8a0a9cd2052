"""3-D RoPE table construction (host side, torch), as the reference builds it.

* ``get_1d_rotary_pos_embed`` -- ``deploy/xvideo/models/dit/rope.py:31-52``
  (``freqs = 1/theta^(arange(0, dim, 2)/dim)``, ``angle = pos * freqs``, pair-interleaved).
* ``rotary_pos_embed_3d`` -- the t|h|w concatenation of
  ``get_rotary_pos_embed_from_ids`` (``deploy/xvideo/models/dit/dit.py:896-934``)
  over tokens ordered t-major, then h, then w (``dit.py:906-915``).
* ``prepare_fused_rope`` -- half-width bf16 tables consumed by the kernels
  (``deploy/xvideo/models/dit/sgl_fused_ops.py:94-119``).

Tables are built once per forward and shared by every layer; they are tiny
(L x D/2 bf16) next to the per-layer Q/K/V traffic.
"""
from __future__ import annotations

from typing import Sequence, Tuple, Union

import torch


def get_1d_rotary_pos_embed(dim: int, pos: Union[torch.Tensor, int], theta: float = 10000.0
                            ) -> Tuple[torch.Tensor, torch.Tensor]:
    assert dim % 2 == 0, f"RoPE dimension must be even, got {dim}"
    if isinstance(pos, int):
        pos = torch.arange(pos).float()
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, device=pos.device)[: (dim // 2)].float() / dim))
    freqs = torch.outer(pos, freqs)
    return freqs.cos().repeat_interleave(2, dim=1), freqs.sin().repeat_interleave(2, dim=1)


def rotary_pos_embed_3d(frame_ids: torch.Tensor, height: int, width: int,
                        rope_dim_list: Sequence[int] = (44, 42, 42), theta: float = 10000.0
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Full-width fp32 (cos, sin) [L, D] with L = len(frame_ids) * height * width."""
    device = frame_ids.device
    t = frame_ids.to(torch.float32).repeat_interleave(height * width)
    hh, ww = torch.meshgrid(torch.arange(height, dtype=torch.float32, device=device),
                            torch.arange(width, dtype=torch.float32, device=device), indexing="ij")
    h = hh.reshape(-1).repeat(frame_ids.numel())
    w = ww.reshape(-1).repeat(frame_ids.numel())
    cos_list, sin_list = [], []
    for dim, p in zip(rope_dim_list, (t, h, w)):
        c, s = get_1d_rotary_pos_embed(dim, p, theta=theta)
        cos_list.append(c)
        sin_list.append(s)
    return torch.cat(cos_list, dim=1), torch.cat(sin_list, dim=1)


def prepare_fused_rope(cos: torch.Tensor, sin: torch.Tensor, head_dim: int, device=None
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Full-width [L, D] (or already half-width) tables -> bf16 half tables [L, D/2]."""
    while cos.dim() > 2:
        if cos.shape[0] != 1:
            raise RuntimeError(f"freqs_cis cos has non-singleton leading dim: {cos.shape}")
        cos, sin = cos.squeeze(0), sin.squeeze(0)
    if cos.shape[-1] == head_dim:
        cos, sin = cos[..., ::2], sin[..., ::2]
    if cos.shape[-1] != head_dim // 2:
        raise RuntimeError(f"freqs_cis width must be {head_dim} or {head_dim // 2}, got {cos.shape[-1]}")
    device = device if device is not None else cos.device
    return (cos.to(device=device, dtype=torch.bfloat16).contiguous(),
            sin.to(device=device, dtype=torch.bfloat16).contiguous())


def rope_3d_half_tables(num_frames: int, height: int, width: int,
                        rope_dim_list: Sequence[int] = (44, 42, 42), theta: float = 10000.0,
                        device=None, frame_ids: torch.Tensor = None
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 half tables [T*H*W, D/2] for the (t, h, w) grid, ready for the kernels."""
    if frame_ids is None:
        frame_ids = torch.arange(num_frames)
    cos, sin = rotary_pos_embed_3d(frame_ids, height, width, rope_dim_list, theta)
    return prepare_fused_rope(cos, sin, sum(rope_dim_list), device=device)
