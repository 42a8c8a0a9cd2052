"""The reference's CPU-runnable torch code path for the hot path, restated (torch, CPU).

TEST / CPU-BASELINE INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``. ``bench.py``
times these functions on the host cores as the reported CPU baseline.

* ``qkv_norm_rope_cache`` -- the reference's per-block sequence for one stream:
  ``rearrange(qkv, "B L (K H D) -> K B L H D")`` (``dit.py:409-411``), then the
  torch fallback of ``fused_qk_norm_rope_3d`` (``sgl_fused_ops.py:170-199``:
  fp32 RMSNorm, ``repeat_interleave`` tables, rotate-half, cast), with the
  pre-RoPE K kept (``return_k_pre_rope``) and V compacted for the cache
  (``dit.py:131-137,446-451``), written into a ring slot.
* ``fp8_linear`` -- ``_quantize_per_token_impl`` (``fp8_linear.py:38-43``) followed
  by fp32 dequantise-then-matmul + bias -> bf16, the benchmark's GEMM reference
  (row-wise ``torch._scaled_mm`` is not available on the CPU backend).
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = torch.finfo(FP8).max


def _rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    out = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (out * w.float()).to(dtype=x.dtype)


def qkv_norm_rope_cache(qkv: torch.Tensor, num_heads: int, eps: float, q_weight, k_weight,
                        cos_half, sin_half, cache_k: torch.Tensor, cache_v: torch.Tensor, slot: int):
    """qkv [L, 3*H*D] bf16; cos/sin half tables [L, D/2]; cache [S, L, H, D]. Returns (q, k)."""
    L = qkv.shape[0]
    D = qkv.shape[1] // (3 * num_heads)
    q, k, v = qkv.view(L, 3, num_heads, D).unbind(1)
    qn = _rmsnorm(q, q_weight, eps)
    kn = _rmsnorm(k, k_weight, eps)
    cos = cos_half.repeat_interleave(2, dim=-1).reshape(L, 1, D).float()
    sin = sin_half.repeat_interleave(2, dim=-1).reshape(L, 1, D).float()

    def apply(x):
        xf = x.float()
        pairs = xf.reshape(*x.shape[:-1], -1, 2)
        rotated = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)
        return (xf * cos + rotated * sin).to(dtype=x.dtype)

    q_out, k_out = apply(qn), apply(kn)
    cache_k[slot, :L].copy_(kn)
    cache_v[slot, :L].copy_(v.clone())
    return q_out, k_out


def quantize_per_token(x: torch.Tensor):
    absmax = x.abs().amax(dim=1, keepdim=True).float().clamp_min(1e-8)
    scale = absmax / FP8_MAX
    q = (x.float() / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return q, scale


def fp8_linear(x: torch.Tensor, w_q: torch.Tensor, w_s: torch.Tensor, bias: torch.Tensor):
    """x [M, K] bf16; w_q [N, K] e4m3fn; w_s [N] fp32; bias [N] bf16 -> bf16 [M, N]."""
    q, s = quantize_per_token(x)
    a = q.float() * s
    b = w_q.float() * w_s.reshape(-1, 1)
    return (a @ b.t() + bias.float()).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# One two-stream MMDiT block (MMDoubleStreamBlock.forward, dit.py:360-558), CPU
# ---------------------------------------------------------------------------
def quantize_per_token_rounding(x: torch.Tensor, exact_division: bool):
    """fp8_linear.py:38-43 (division) or per_token_quant_fp8_rocm.hip:72-77 (reciprocal)."""
    absmax = x.abs().amax(dim=1, keepdim=True).float().clamp_min(1e-8)
    scale = absmax / FP8_MAX
    v = x.float() / scale if exact_division else x.float() * (1.0 / scale)
    return v.clamp(-FP8_MAX, FP8_MAX).to(FP8), scale


def _fp8_linear_ref(x2d, w_q, w_s, bias, exact_division, gelu=False):
    q, s = quantize_per_token_rounding(x2d, exact_division)
    y = ((q.float() * s) @ (w_q.float() * w_s.reshape(-1, 1)).t() + bias.float()).to(torch.bfloat16)
    if gelu:  # F.gelu on the bf16 GEMM output (dit.py:87-89)
        y = torch.nn.functional.gelu(y.float(), approximate="tanh").to(torch.bfloat16)
    return y


def _layernorm_modulate_ref(x2d, shift, scale, eps):
    """fused_norm_scale_shift.cu:97-182 without affine weights: fp32, one rounding."""
    y = torch.nn.functional.layer_norm(x2d.float(), (x2d.shape[1],), eps=eps)
    return (y * (1 + scale.float()) + shift.float()).to(torch.bfloat16)


def _rope_half(x, cos_half, sin_half):
    """Interleaved-pair rotation with half tables [L, D/2] (fused_qknorm_rope_3d_kernel.cu:95-104)."""
    c = cos_half.float()[:, None, :]
    s = sin_half.float()[:, None, :]
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x0 * s + x1 * c
    return out


def _rms_two_round(x, w, eps):
    xf = x.float()
    n = (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    return (n.float() * w.float()).to(torch.bfloat16)


def double_stream_block(img, txt, vec, streams, heads, img_cos_half, img_sin_half, cached=(),
                        division_min_k=8192, eps=1e-6, skip_text_stream=False, write_only=False,
                        cache_tokens=None, cache_pre_rope=True, out_rows=None):
    """The quantised block chain on the CPU, with the reference's numerics at every step.

    img [L, E], txt [T, E], vec [1, E] bf16; ``streams`` = (img_w, txt_w) dicts with bf16
    ``mod_table`` [1, 6, E], ``q_norm``/``k_norm`` [D] and per linear ``<name>_q`` [N, K] e4m3fn,
    ``<name>_s`` [N] fp32, ``<name>_b`` [N] bf16 for qkv, proj, up, down; ``cached`` = list of
    (key [len, H, D] bf16, value [len, H, D] bf16, cos_full [len, D] f32, sin_full): a key
    stored before RoPE is rotated with its tables; with ``cos_full`` None it was stored rotated
    and is used as is (``_concat_kv_entries``, dit.py:216-271).

    Modes of ``MMDoubleStreamBlock.forward`` (dit.py:360-558): ``skip_text_stream`` attends
    over [cached | video] and leaves txt unchanged (dit.py:481-487,500-506); ``write_only``
    returns right after the cache write (dit.py:446-459); ``cache_tokens`` keeps the first
    tokens only (``kv_cache_write_seq_len``, dit.py:449-451); ``cache_pre_rope`` False keeps
    the rotated K (dit.py:432-433).
    ``out_rows`` = (img_rows, txt_rows) index tensors: every K / V row is still computed, but the
    attention and the row-local tail only for those output rows (the full-size check samples rows).
    Returns (img_out, txt_out, k_cache, v_cache) (img_out / txt_out: the selected rows).
    """
    L, E = img.shape
    T = txt.shape[0]
    D = E // heads
    n_cache = L if cache_tokens is None else int(cache_tokens)
    wi, wt = streams

    def modulation(w):
        # ModulateWan (dit.py:97-111): table + vec, six chunks
        return [c.squeeze(1) for c in (w["mod_table"].float() + vec.float().unsqueeze(1)).to(torch.bfloat16)
                .chunk(6, dim=1)]

    def qkv_proj(x, w, mod):
        xm = _layernorm_modulate_ref(x, mod[0], mod[1], eps)
        return _fp8_linear_ref(xm, w["qkv_q"], w["qkv_s"], w["qkv_b"], E >= division_min_k)

    mod_i = modulation(wi)
    qkv_i = qkv_proj(img, wi, mod_i).view(L, 3, heads, D)
    qi, ki, vi = qkv_i[:, 0], qkv_i[:, 1], qkv_i[:, 2]

    def norm1(x, wn):
        xf = x.float()
        return xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * wn.float()

    # video: q/k RMSNorm (one rounding) + RoPE; pre-RoPE K kept
    qh, kh = norm1(qi, wi["q_norm"]), norm1(ki, wi["k_norm"])
    q_img = _rope_half(qh, img_cos_half, img_sin_half).to(torch.bfloat16)
    k_img = _rope_half(kh, img_cos_half, img_sin_half).to(torch.bfloat16)
    k_cache = (kh.to(torch.bfloat16) if cache_pre_rope else k_img)[:n_cache]
    v_cache = vi[:n_cache].contiguous()
    if write_only:
        return img, txt, k_cache, v_cache

    if not skip_text_stream:
        mod_t = modulation(wt)
        # condition: two-rounding q/k RMSNorm, no RoPE (fused_joint_qkv_pack.cu:58-79)
        qkv_t = qkv_proj(txt, wt, mod_t).view(T, 3, heads, D)
        q_txt = _rms_two_round(qkv_t[:, 0], wt["q_norm"], eps)
        k_txt = _rms_two_round(qkv_t[:, 1], wt["k_norm"], eps)
    # cached chunks: pre-RoPE keys rotated with fp32 full-width tables (fused_joint_qkv_pack.cu:207-218)
    ck, cv = [], []
    for key, value, cos, sin in cached:
        if cos is None:
            ck.append(key)
        else:
            kf = key.float()
            c = cos.float()[:, None, 0::2]
            s = sin.float()[:, None, 0::2]
            out = torch.empty_like(kf)
            out[..., 0::2] = kf[..., 0::2] * c - kf[..., 1::2] * s
            out[..., 1::2] = kf[..., 0::2] * s + kf[..., 1::2] * c
            ck.append(out.to(torch.bfloat16))
        cv.append(value)
    if skip_text_stream:
        Q, K, V = q_img, torch.cat(ck + [k_img]), torch.cat(cv + [vi])
    else:
        Q = torch.cat([q_img, q_txt])
        K = torch.cat(ck + [k_img, k_txt])
        V = torch.cat(cv + [vi, qkv_t[:, 2]])
    ri = torch.arange(L) if out_rows is None else out_rows[0]
    rt = torch.arange(T) if out_rows is None else out_rows[1]
    sel = ri if skip_text_stream else torch.cat([ri, L + rt])
    Q = Q[sel]
    attn = torch.nn.functional.scaled_dot_product_attention(
        Q.float().transpose(0, 1)[None], K.float().transpose(0, 1)[None], V.float().transpose(0, 1)[None])
    attn = attn[0].transpose(0, 1).reshape(Q.shape[0], E).to(torch.bfloat16)
    n_i = ri.numel()

    def mlp_tail(x, w, mod, a):
        p = _fp8_linear_ref(a, w["proj_q"], w["proj_s"], w["proj_b"], E >= division_min_k)
        x = (x.float() + p.float() * mod[2].float()).to(torch.bfloat16)
        xm = _layernorm_modulate_ref(x, mod[3], mod[4], eps)
        h = _fp8_linear_ref(xm, w["up_q"], w["up_s"], w["up_b"], E >= division_min_k, gelu=True)
        d = _fp8_linear_ref(h, w["down_q"], w["down_s"], w["down_b"], h.shape[1] >= division_min_k)
        return (x.float() + d.float() * mod[5].float()).to(torch.bfloat16)

    img_out = mlp_tail(img[ri], wi, mod_i, attn[:n_i])
    txt_out = txt[rt] if skip_text_stream else mlp_tail(txt[rt], wt, mod_t, attn[n_i:])
    if out_rows is None and skip_text_stream:
        txt_out = txt
    return img_out, txt_out, k_cache, v_cache
