"""3-D RoPE table construction (host side, torch), as the reference builds it.

* ``get_1d_rotary_pos_embed`` -- ``deploy/xvideo/models/dit/rope.py:31-52``
  (``freqs = 1/theta^(arange(0, dim, 2)/dim)``, ``angle = pos * freqs``, pair-interleaved).
* ``rotary_pos_embed_3d`` -- the t|h|w concatenation of
  ``get_rotary_pos_embed_from_ids`` (``deploy/xvideo/models/dit/dit.py:896-934``)
  over tokens ordered t-major, then h, then w (``dit.py:906-915``).
* ``source_id_rope`` / ``compose_rope`` -- the per-token role rotation (target,
  edit-condition ref video, extra ref image) added to the 3-D angles by angle
  addition (``dit.py:29-31,936-960,1146-1155``).
* ``visual_rope_half_tables`` -- the whole visual sequence of one forward,
  [current chunk | ref-video tokens], as ``dit.py:1093-1166`` assembles it.
* ``prepare_fused_rope`` -- half-width bf16 tables consumed by the kernels
  (``deploy/xvideo/models/dit/sgl_fused_ops.py:94-119``).

Tables are built once per forward and shared by every layer; they are tiny
(L x D/2 bf16) next to the per-layer Q/K/V traffic.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple, Union

import torch

# Role of a visual token in the joint sequence (dit.py:29-31).
SOURCE_ID_TARGET = 0.0
SOURCE_ID_EDIT_CONDITION = 1.0
SOURCE_ID_EXTRA_REF_IMAGE = 2.0


def get_1d_rotary_pos_embed(dim: int, pos: Union[torch.Tensor, int], theta: float = 10000.0
                            ) -> Tuple[torch.Tensor, torch.Tensor]:
    if dim % 2:
        raise ValueError(f"a rotary axis needs an even number of dims, got {dim}")
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


def source_id_rope(source_id: torch.Tensor, head_dim: int, role_dim: int = 128, theta: float = 256.0
                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Full-width fp32 (cos, sin) [..., head_dim] of the role rotation (``dit.py:936-960``).

    The first ``role_dim`` dims (clamped to [0, head_dim]) rotate by ``source_id * f_j`` with
    ``f_j = 1 / theta^(2j / role_dim)``; the remaining pairs are left unrotated (cos 1, sin 0).
    Source id 0 (target tokens) is the identity."""
    role_dim = max(0, min(int(role_dim), int(head_dim)))
    half = head_dim // 2
    cos_half = torch.ones(*source_id.shape, half, device=source_id.device, dtype=torch.float32)
    sin_half = torch.zeros_like(cos_half)
    inv_freq = 1.0 / (float(theta) ** (torch.arange(0, role_dim, 2, device=source_id.device,
                                                    dtype=torch.float32) / role_dim))
    angles = source_id.to(torch.float32).unsqueeze(-1) * inv_freq
    cos_half[..., : role_dim // 2] = torch.cos(angles)
    sin_half[..., : role_dim // 2] = torch.sin(angles)
    return cos_half.repeat_interleave(2, dim=-1), sin_half.repeat_interleave(2, dim=-1)


def compose_rope(cos_a: torch.Tensor, sin_a: torch.Tensor, cos_b: torch.Tensor, sin_b: torch.Tensor
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotation by angle a + b from the tables of a and b (``dit.py:1153-1154``), each product and
    sum rounded once in the tables' dtype."""
    return cos_a * cos_b - sin_a * sin_b, sin_a * cos_b + cos_a * sin_b


def _frame_ids(num_frames: int, temporal_ids: Optional[torch.Tensor]) -> torch.Tensor:
    if temporal_ids is None:
        return torch.arange(num_frames)
    ids = torch.as_tensor(temporal_ids, dtype=torch.long).cpu()
    if ids.dim() != 1 or ids.numel() != num_frames:
        raise ValueError(f"temporal ids must be 1-D with {num_frames} entries, got shape {tuple(ids.shape)}")
    return ids


def visual_rope_tables(current_shape: Tuple[int, int, int], ref_video_frames: Optional[int] = None,
                       temporal_ids: Optional[torch.Tensor] = None,
                       rope_dim_list: Sequence[int] = (16, 56, 56), theta: float = 256.0,
                       source_id_rope_dim: int = 128, source_id_rope_theta: float = 256.0,
                       ref_image_cache: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Full-width fp32 (cos, sin) [L, D] of one forward's visual sequence (``dit.py:1093-1155``).

    Tokens are the current chunk (``current_shape`` = (frames, h, w) after patching; role
    ``SOURCE_ID_EXTRA_REF_IMAGE`` when ``ref_image_cache``, else ``SOURCE_ID_TARGET``), then, if
    ``ref_video_frames`` is given, the ref-video tokens of the same spatial grid and the same
    temporal ids (role ``SOURCE_ID_EDIT_CONDITION``). The 3-D tables are rotated by each token's
    role angle. Defaults are the production model's (``deploy/xvideo/config.py:29-37``)."""
    frames, height, width = current_shape
    head_dim = sum(rope_dim_list)
    tokens = frames * height * width
    cur_id = SOURCE_ID_EXTRA_REF_IMAGE if ref_image_cache else SOURCE_ID_TARGET
    cos, sin = rotary_pos_embed_3d(_frame_ids(frames, temporal_ids), height, width, rope_dim_list, theta)
    ids = [torch.full((tokens,), cur_id, dtype=torch.float32)]
    if ref_video_frames is not None:
        c2, s2 = rotary_pos_embed_3d(_frame_ids(ref_video_frames, temporal_ids), height, width, rope_dim_list,
                                     theta)
        cos, sin = torch.cat([cos, c2]), torch.cat([sin, s2])
        ids.append(torch.full((c2.shape[0],), SOURCE_ID_EDIT_CONDITION, dtype=torch.float32))
    cos_r, sin_r = source_id_rope(torch.cat(ids), head_dim, source_id_rope_dim, source_id_rope_theta)
    return compose_rope(cos, sin, cos_r, sin_r)


def visual_rope_half_tables(current_shape: Tuple[int, int, int], ref_video_frames: Optional[int] = None,
                            device=None, **kwargs) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 half tables [L, D/2] of ``visual_rope_tables``, ready for the kernels."""
    cos, sin = visual_rope_tables(current_shape, ref_video_frames, **kwargs)
    return prepare_fused_rope(cos, sin, cos.shape[-1], device=device)


def prepare_fused_rope(cos: torch.Tensor, sin: torch.Tensor, head_dim: int, device=None
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Full-width [L, D] (or already half-width) tables -> bf16 half tables [L, D/2]."""
    while cos.dim() > 2:
        if cos.shape[0] != 1:
            raise RuntimeError(f"RoPE tables need a leading dimension of 1 to squeeze, got shape {tuple(cos.shape)}")
        cos, sin = cos.squeeze(0), sin.squeeze(0)
    if cos.shape[-1] == head_dim:
        cos, sin = cos[..., ::2], sin[..., ::2]
    if cos.shape[-1] != head_dim // 2:
        raise RuntimeError(f"RoPE table rows hold {cos.shape[-1]} values; a head of {head_dim} needs "
                           f"{head_dim} (full width) or {head_dim // 2} (half width)")
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
