"""Quantised two-stream MMDiT block chain on the gfx950 kernels.

Counterpart of the reference's ``MMDoubleStreamBlock.forward``
(``deploy/xvideo/models/dit/dit.py:360-558``) with FP8 installed on both streams
(``dit.py:57-90``) and the streaming KV cache kept as a pre-RoPE ring:

per stream (video "img", condition "txt"), with ``mod = table + vec`` split into
(shift1, scale1, gate1, shift2, scale2, gate2) (``ModulateWan``, ``dit.py:97-111``):

* adaLN LayerNorm + modulation emitting the QKV input in FP8
  (``fused_norm_scale_shift_fp8``: ``fused_layernorm_modulate``
  ``sgl_fused_ops.py:46-91`` fused with the ``Fp8Linear`` quantiser);
* QKV FP8 GEMM (``fp8_scaled_mm``, ``fp8_linear.py:114-141``);
* the joint attention operands Q = [video | condition], K, V = [cached | video |
  condition] (``fused_joint_qkv_pack``, ``dit.py:489-496``) are written in place by
  their producers, so no row is copied twice:
  - video stream: QKV split + q/k RMSNorm + 3-D RoPE in one pass, roped q/k and V
    into the joint buffers, pre-RoPE K and V into a ring slot
    (``fused_qkv_norm_rope_cache``, replacing ``dit.py:409-451`` +
    ``_write_layer_kv_cache`` ``dit.py:867-882``);
  - cached chunks: pre-RoPE K rotated on read straight out of their ring slots
    with fp32 full-width tables into the head of the joint K / V
    (``fused_cached_kv_pack_out``, ``_concat_kv_entries`` ``dit.py:216-271``);
  - condition stream: the two-rounding q/k RMSNorm into the tails
    (``fused_text_qkv_pack``);
* attention: the gfx950 flash-attention kernel (``sdpa_attention``), non-causal, no
  mask, default scale 1/sqrt(D) -- the reference's ``_sdpa_attention``
  (``dit.py:154-167``) read in the token-major joint layout without transposes
  (``attention_backend="torch_sdpa"`` runs the reference's own call instead);
* out-proj FP8 GEMM with the gated residual (``fused_add_gate``, ``dit.py:525-528``)
  in its epilogue (``fp8_scaled_mm_gated_residual``);
* adaLN + FP8 quant -> FFN-up FP8 GEMM with the GELU-tanh epilogue -> quant ->
  FFN-down FP8 GEMM with the gated residual in its epilogue, in place on the
  stream (``dit.py:508-513,529-538``).

The condition stream runs on a second HIP stream (default priority) between the points
where the two streams meet -- its QKV and pack beside the video QKV, norm/RoPE and
cached pack; its projection and FFN beside the video FFN -- joined before attention and
before returning; the results are those of the serial chain, bit for bit.

Activation quantiser rounding per K follows the reference's ROCm path
(``fp8_linear.py:57-74``): reciprocal-multiply below K = 8192, division above.
Weights are random-initialised with the benchmark distributions (there are no
checkpoints here): Linear weights N(0, 0.02), biases N(0, 0.01), q/k norm weights
N(1, 0.1), modulation table N(0, 1)/sqrt(hidden) (``ModulateWan.__init__``).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import (fp8_qkv_norm_rope_cache, fused_cached_kv_pack_out, fused_norm_scale_shift_fp8,
               fused_qkv_norm_rope_cache, fused_text_qkv_pack, sdpa_attention)
from .fp8_linear import Fp8Linear, exact_division_for

NORM_EPS = 1e-6            # dit.py:35
NUM_MODULATION_CHUNKS = 6  # dit.py:37


@dataclass
class StreamWeights:
    """One stream's parameters (bf16 originals kept for reference checks)."""
    mod_table: torch.Tensor       # [1, 6, E] bf16
    q_norm: torch.Tensor          # [D] bf16
    k_norm: torch.Tensor          # [D] bf16
    linears: dict                 # name -> nn.Linear (bf16): qkv, proj, up, down
    qkv: Fp8Linear = None
    proj: Fp8Linear = None
    up: Fp8Linear = None
    down: Fp8Linear = None


def random_stream_weights(hidden: int, heads: int, mlp_hidden: int, generator: torch.Generator,
                          device) -> StreamWeights:
    """Random-init weights of one stream with the benchmark distributions (drawn on the CPU)."""
    D = hidden // heads

    def linear(k_in, k_out):
        lin = nn.Linear(k_in, k_out, bias=True)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(k_out, k_in, generator=generator) * 0.02)
            lin.bias.copy_(torch.randn(k_out, generator=generator) * 0.01)
        return lin.to(torch.bfloat16).to(device)

    table = (torch.randn(1, NUM_MODULATION_CHUNKS, hidden, generator=generator) / hidden ** 0.5)
    w = StreamWeights(
        mod_table=table.to(torch.bfloat16).to(device),
        q_norm=(1 + 0.1 * torch.randn(D, generator=generator)).to(torch.bfloat16).to(device),
        k_norm=(1 + 0.1 * torch.randn(D, generator=generator)).to(torch.bfloat16).to(device),
        linears={"qkv": linear(hidden, 3 * hidden), "proj": linear(hidden, hidden),
                 "up": linear(hidden, mlp_hidden), "down": linear(mlp_hidden, hidden)})
    return w


class KVRing:
    """Bounded KV-state cache: pre-RoPE K and V of up to ``slots`` chunks, ``[slots, capacity, H, D]``
    bf16 each, caller-owned and written in place (the reference keeps the same content in a dict of
    per-chunk tensors, ``dit.py:715-894``)."""

    def __init__(self, slots: int, capacity: int, heads: int, head_dim: int, device):
        self.k = torch.zeros(slots, capacity, heads, head_dim, dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)
        self.lengths = [0] * slots
        # per slot: K stored before RoPE (kv_cache_pre_rope=True) or rotated (the reference's default)
        self.pre_rope = [True] * slots
        # per slot: bumped on every write through the block (kernels write through raw pointers,
        # which torch's version counters do not see); in-place torch ops bump ``k._version``
        self.generation = [0] * slots

    def touch(self, slot: int) -> None:
        """Record that ``slot`` was rewritten outside torch's view (e.g. by a kernel)."""
        self.generation[slot] += 1

    def key(self, slot: int) -> torch.Tensor:
        return self.k[slot, : self.lengths[slot]][None]

    def value(self, slot: int) -> torch.Tensor:
        return self.v[slot, : self.lengths[slot]][None]


@dataclass
class CachedChunk:
    """A cached chunk to attend to: its ring slot and, for a K stored before RoPE, the fp32
    full-width RoPE tables ``[len, D]`` of its window-relative positions (``dit.py:1196-1217``).
    A slot holding rotated K (written with ``kv_cache_pre_rope=False``) takes no tables and is
    copied as is, as ``_concat_kv_entries`` concatenates such entries (``dit.py:258-271``)."""
    slot: int
    cos: Optional[torch.Tensor] = None
    sin: Optional[torch.Tensor] = None


@dataclass
class JointKV:
    """One layer's joint attention K / V buffers ``[1, cached + video + condition, H, D]`` kept
    across calls: the cached rows (chunks read from the ring, rotated on read) are assembled on
    the first call and reused while the cached chunks are unchanged (same ring slots, lengths,
    storage mode, slot generations, ring version and RoPE tables). The reference memoises the
    same assembly across the denoising steps of a chunk (``dit.py:1168-1217``,
    ``_assemble_layer_kv_cache_cached`` ``dit.py:801-816``) and copies it into the joint
    buffers on every call (``fused_joint_qkv_pack``, ``dit.py:489-496``); here the rows stay
    where the attention reads them and only the video and condition rows are rewritten. The
    stamp holds the ring and every RoPE table it names (compared by identity), so these stay
    alive while the JointKV does and a table rebuilt at a recycled address never matches."""
    k: Optional[torch.Tensor] = None
    v: Optional[torch.Tensor] = None
    stamp: Optional[tuple] = None

    def invalidate(self) -> None:
        self.stamp = None


class _Same:
    """A stamp entry that holds a strong reference to an object and compares by identity.

    Holding the reference keeps the object (a ring, a RoPE table) alive for as long as the stamp
    is, so its address cannot be handed to a new tensor with other contents while a stamp that
    names it exists; comparing by ``is`` then tells a rebuilt table from the original even where
    address, shape, strides and version counter all agree."""

    __slots__ = ("obj",)

    def __init__(self, obj):
        self.obj = obj

    def __eq__(self, other):
        return isinstance(other, _Same) and other.obj is self.obj

    def __hash__(self):
        return id(self.obj)

    def __repr__(self):
        return f"_Same({type(self.obj).__name__}@{id(self.obj):#x})"


def _tensor_key(t: Optional[torch.Tensor]):
    if t is None:
        return None
    return (_Same(t), t.data_ptr(), tuple(t.shape), tuple(t.stride()), str(t.dtype), t._version)


def cached_rows_stamp(ring: Optional[KVRing], cached: Sequence[CachedChunk]) -> tuple:
    """Everything the assembled cached rows depend on; equal stamps mean equal rows. The stamp
    holds the ring, its K / V tensors and every table it names (compared by identity), so a
    table freed and rebuilt with other values at the same address never matches."""
    if not cached:
        return ()
    return (_Same(ring), _Same(ring.k), _Same(ring.v), ring.k.data_ptr(), ring.k._version, ring.v._version,
            tuple((c.slot, ring.lengths[c.slot], ring.pre_rope[c.slot], ring.generation[c.slot],
                   _tensor_key(c.cos), _tensor_key(c.sin)) for c in cached))


def _adjacent_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Rows of a followed by rows of b: a view when b's rows follow a's in one contiguous buffer
    (chunks cut from one table of every cached token, as the reference builds ``cached_freqs_cis``,
    ``dit.py:1196-1217``), else a copy."""
    if (a.is_contiguous() and b.is_contiguous() and a.dtype == b.dtype and a.device == b.device
            and a.dim() == 2 and b.dim() == 2 and a.shape[1] == b.shape[1]
            and b.data_ptr() == a.data_ptr() + a.numel() * a.element_size()
            and a.untyped_storage().data_ptr() == b.untyped_storage().data_ptr()):
        return a.as_strided((a.shape[0] + b.shape[0], a.shape[1]), (a.shape[1], 1))
    return torch.cat([a, b])


class QuantizedDoubleStreamBlock:
    """The quantised chain of one two-stream MMDiT block (see the module docstring)."""

    def __init__(self, hidden: int, heads: int, mlp_hidden: int, device, generator: torch.Generator,
                 quant_rounding: str = "reference_rocm", overlap_streams: bool = True,
                 attention_backend: str = "hip", fuse_qkv: bool = True):
        if attention_backend not in ("hip", "torch_sdpa"):
            raise ValueError(f"attention_backend must be 'hip' or 'torch_sdpa', not {attention_backend!r}")
        # "hip": this library's attention kernel on the token-major joint operands; "torch_sdpa": the
        # reference's own call, F.scaled_dot_product_attention on transposed views (dit.py:154-167)
        self.attention_backend = attention_backend
        self.hidden, self.heads, self.mlp_hidden = hidden, heads, mlp_hidden
        self.head_dim = hidden // heads
        self.quant_rounding = quant_rounding
        # the condition stream's kernels run on a second (default-priority) HIP stream, beside the
        # video stream's, between the points where the two streams meet (joint attention operands,
        # attention output); results do not depend on it
        self.overlap_streams = overlap_streams
        # the video stream's QKV projection and its q/k norm, RoPE and ring write as one op
        # (fp8_qkv_norm_rope_cache); False: the GEMM, then fused_qkv_norm_rope_cache on its output
        # (the same bits)
        self.fuse_qkv = fuse_qkv
        self.img = random_stream_weights(hidden, heads, mlp_hidden, generator, device)
        self.txt = random_stream_weights(hidden, heads, mlp_hidden, generator, device)
        for w in (self.img, self.txt):
            w.qkv = Fp8Linear.from_linear(w.linears["qkv"], quant_rounding=quant_rounding)
            w.proj = Fp8Linear.from_linear(w.linears["proj"], quant_rounding=quant_rounding)
            w.up = Fp8Linear.from_linear(w.linears["up"], gelu_tanh=True, quant_rounding=quant_rounding)
            w.down = Fp8Linear.from_linear(w.linears["down"], quant_rounding=quant_rounding)

    # -- pieces -------------------------------------------------------------
    @staticmethod
    def modulation(w: StreamWeights, vec: torch.Tensor) -> List[torch.Tensor]:
        """ModulateWan.forward (dit.py:103-106): [1, 6, E] + vec -> six [1, E] rows."""
        return [c.squeeze(1) for c in (w.mod_table + vec.unsqueeze(1)).chunk(NUM_MODULATION_CHUNKS, dim=1)]

    def norm_quant(self, x2d: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, k_in: int):
        """LayerNorm + (1 + scale) + shift, quantised per token for the next Fp8Linear."""
        M = x2d.shape[0]
        q = torch.empty(M, x2d.shape[1], dtype=torch.float8_e4m3fn, device=x2d.device)
        s = torch.empty(M, 1, dtype=torch.float32, device=x2d.device)
        fused_norm_scale_shift_fp8(x2d, None, None, scale, shift, "layer", NORM_EPS, q, s, None,
                                   exact_division_for(k_in, self.quant_rounding))
        return q, s

    def attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Attention on [B, S, H, D] operands (dit.py:154-167): [B, S, H, D] out."""
        if self.attention_backend == "torch_sdpa":
            out = torch.nn.functional.scaled_dot_product_attention(
                q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=False)
            return out.transpose(1, 2)
        return sdpa_attention(q, k, v)

    # -- argument checks ----------------------------------------------------
    @staticmethod
    def check_cache_args(L: int, ring: Optional[KVRing], write_slot: Optional[int], cached: Sequence[CachedChunk],
                         cache_tokens: int) -> None:
        """Reject cache arguments that would make the chain read or write the wrong rows."""
        if (ring is None) and (write_slot is not None or cached):
            raise ValueError("write_slot and cached chunks need a KV ring")
        if write_slot is not None:
            if not 0 <= write_slot < len(ring.lengths):
                raise ValueError(f"write_slot {write_slot} is not a slot of the ring ({len(ring.lengths)} slots)")
            if not 0 <= cache_tokens <= L:
                raise ValueError(f"kv_cache_write_seq_len {cache_tokens} is outside [0, {L}]")
            if cache_tokens > ring.k.shape[1]:
                raise ValueError(f"{cache_tokens} tokens do not fit a ring slot of {ring.k.shape[1]}")
        slots = [c.slot for c in cached]
        if len(set(slots)) != len(slots):
            raise ValueError(f"a ring slot is attended twice: {slots}")
        if write_slot is not None and write_slot in slots:
            # the write would overwrite the chunk before it is read
            raise ValueError(f"write_slot {write_slot} is also a cached slot; the chunk would be overwritten "
                             "before attention reads it")
        for c in cached:
            if not 0 <= c.slot < len(ring.lengths):
                raise ValueError(f"cached slot {c.slot} is not a slot of the ring")
            n = ring.lengths[c.slot]
            if n <= 0:
                raise ValueError(f"cached slot {c.slot} is empty")
            if ring.pre_rope[c.slot]:
                if c.cos is None or c.sin is None:
                    raise ValueError(f"cached slot {c.slot} holds K before RoPE and needs its cos/sin tables")
                for name, t in (("cos", c.cos), ("sin", c.sin)):
                    if t.dim() != 2 or t.shape[0] != n:
                        raise ValueError(f"cached slot {c.slot} holds {n} tokens but its {name} table has "
                                         f"shape {tuple(t.shape)}; expected [{n}, head_dim]")
            elif c.cos is not None or c.sin is not None:
                raise ValueError(f"cached slot {c.slot} holds rotated K; it takes no RoPE tables")

    _side_streams = {}  # one second stream per device, shared by every block

    @classmethod
    def _side_stream(cls, device) -> torch.cuda.Stream:
        dev = torch.device(device)
        key = dev.index if dev.index is not None else torch.cuda.current_device()
        if key not in cls._side_streams:
            cls._side_streams[key] = torch.cuda.Stream(device=key)
        return cls._side_streams[key]

    # -- forward ------------------------------------------------------------
    def _cached_into(self, ring: KVRing, cached: Sequence[CachedChunk], k: torch.Tensor, v: torch.Tensor) -> None:
        """Cached chunks into the head of the joint K / V: runs of pre-RoPE slots rotated on read, two
        at a time (``fused_cached_kv_pack_out``); rotated slots copied as they are."""
        off, i = 0, 0
        while i < len(cached):
            c0 = cached[i]
            n0 = ring.lengths[c0.slot]
            if not ring.pre_rope[c0.slot]:
                k[0, off:off + n0].copy_(ring.k[c0.slot, :n0])
                v[0, off:off + n0].copy_(ring.v[c0.slot, :n0])
                off, i = off + n0, i + 1
                continue
            pair = i + 1 < len(cached) and ring.pre_rope[cached[i + 1].slot]
            seg = cached[i:i + 2] if pair else [c0]
            n = sum(ring.lengths[c.slot] for c in seg)
            cos = _adjacent_rows(c0.cos, seg[1].cos) if pair else c0.cos
            sin = _adjacent_rows(c0.sin, seg[1].sin) if pair else c0.sin
            k1 = ring.key(seg[1].slot) if pair else None
            v1 = ring.value(seg[1].slot) if pair else None
            fused_cached_kv_pack_out(ring.key(c0.slot), ring.value(c0.slot), k1, v1, cos, sin,
                                     k[:, off:off + n], v[:, off:off + n])
            off, i = off + n, i + len(seg)

    def _video_qkv(self, q8, s8, cos, sin, q_out, k_out, ring_k, ring_v, slot, v_out, n_cache, pre_rope):
        """The video stream's QKV projection with its q/k RMSNorm, RoPE and ring write
        (``dit.py:409-451``): fp8_qkv_norm_rope_cache when fused, else the GEMM and then
        fused_qkv_norm_rope_cache on its output. Returns None (fused) or the QKV rows."""
        w, H = self.img.qkv, self.heads
        if self.fuse_qkv:
            fp8_qkv_norm_rope_cache(q8, w.weight_fp8, s8, w.weight_scale, w.bias, H, NORM_EPS, self.img.q_norm,
                                    self.img.k_norm, cos, sin, q_out, k_out, ring_k, ring_v, slot, 0, v_out=v_out,
                                    cache_tokens=n_cache, cache_pre_rope=pre_rope)
            return None
        qkv = w.gemm(q8, s8)
        fused_qkv_norm_rope_cache(qkv, H, NORM_EPS, self.img.q_norm, self.img.k_norm, cos, sin, q_out, k_out, ring_k,
                                  ring_v, slot, 0, v_out=v_out, cache_tokens=n_cache, cache_pre_rope=pre_rope)
        return qkv

    def forward(self, img: torch.Tensor, txt: torch.Tensor, vec: torch.Tensor, img_cos: torch.Tensor,
                img_sin: torch.Tensor, ring: Optional[KVRing] = None, write_slot: Optional[int] = None,
                cached: Sequence[CachedChunk] = (), mark: Optional[Callable[[str], None]] = None,
                skip_text_stream: bool = False, kv_cache_write_only: bool = False,
                kv_cache_write_seq_len: Optional[int] = None, kv_cache_pre_rope: bool = True,
                joint: Optional[JointKV] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """img [1, L, E], txt [1, T, E], vec [1, E] bf16; img_cos/img_sin bf16 half tables [L, D/2].

        Writes the first ``kv_cache_write_seq_len`` (default all) video tokens' K and V into ``ring``
        slot ``write_slot`` (if given) -- K before RoPE when ``kv_cache_pre_rope``, else rotated -- and
        attends to [cached chunks | video | condition] (``dit.py:489-498``), or to [cached chunks |
        video] with ``skip_text_stream`` (``dit.py:481-487``; txt is returned unchanged).
        ``kv_cache_write_only`` returns (img, txt) unchanged right after the ring write
        (``dit.py:446-459``). ``joint`` keeps the joint K / V buffers across calls and reuses their
        cached rows while the cached chunks are unchanged (``JointKV``). ``mark(name)`` is called after
        each stage (the benchmark places timing events there). Returns the updated (img, txt).
        """
        mark = mark or (lambda name: None)
        E, H, D = self.hidden, self.heads, self.head_dim
        L, T = img.shape[1], txt.shape[1]
        n_cache = L if kv_cache_write_seq_len is None else int(kv_cache_write_seq_len)
        self.check_cache_args(L, ring, write_slot, cached, n_cache)
        if kv_cache_write_only and write_slot is None:
            raise ValueError("kv_cache_write_only needs a ring and a write_slot")
        ring_k, ring_v, slot = (ring.k, ring.v, write_slot) if write_slot is not None else (None, None, 0)
        img2, txt2 = img.reshape(L, E), txt.reshape(T, E)
        im = self.modulation(self.img, vec)

        if kv_cache_write_only:
            # only the ring is written: Q is not read, no attention operand is produced
            q8, s8 = self.norm_quant(img2, im[0], im[1], E)
            self._video_qkv(q8, s8, img_cos, img_sin, None, None, ring_k, ring_v, slot, None, n_cache,
                            kv_cache_pre_rope)
            ring.lengths[write_slot], ring.pre_rope[write_slot] = n_cache, kv_cache_pre_rope
            ring.touch(write_slot)
            mark("qkv_norm_rope")
            return img, txt

        text = not skip_text_stream
        # joint attention operands: Q = [video | condition], K, V = [cached | video | condition]
        C = sum(ring.lengths[c.slot] for c in cached) if cached else 0
        n_q = L if skip_text_stream else L + T
        q = torch.empty(1, n_q, H, D, dtype=torch.bfloat16, device=img.device)
        reuse_cached = False
        if joint is None:
            k = torch.empty(1, C + n_q, H, D, dtype=torch.bfloat16, device=img.device)
            v = torch.empty_like(k)
        else:
            if joint.k is None or tuple(joint.k.shape) != (1, C + n_q, H, D) or joint.k.device != img.device:
                joint.k = torch.empty(1, C + n_q, H, D, dtype=torch.bfloat16, device=img.device)
                joint.v = torch.empty_like(joint.k)
                joint.stamp = None
            k, v = joint.k, joint.v
            stamp = cached_rows_stamp(ring, cached)
            reuse_cached = joint.stamp == stamp
            joint.stamp = None  # set again once the cached rows are assembled
        main = torch.cuda.current_stream(img.device)
        side = self._side_stream(img.device) if text and self.overlap_streams else None

        def text_qkv():
            tm = self.modulation(self.txt, vec)
            q8, s8 = self.norm_quant(txt2, tm[0], tm[1], E)
            return tm, self.txt.qkv.gemm(q8, s8)

        def text_pack(txt_qkv):
            # condition stream: two-rounding q/k RMSNorm into the tails of Q / K / V
            tv = txt_qkv.view(1, T, 3, H, D)
            fused_text_qkv_pack(tv[:, :, 0], tv[:, :, 1], tv[:, :, 2], self.txt.q_norm, self.txt.k_norm, NORM_EPS,
                                q[:, L:], k[:, C + L:], v[:, C + L:])

        def proj_ffn(x2d, w, m, a, then=None):
            x = w.proj.gated_residual(a, x2d, m[2])            # new tensor: the caller's input stays
            if then is not None:
                then()
            q8, s8 = self.norm_quant(x, m[3], m[4], E)
            h = w.up.gemm(q8, s8)
            w.down.gated_residual(h, x, m[5], inplace=True)
            return x

        if side is not None:  # fork: the condition stream's QKV and pack beside the video stream's
            side.wait_stream(main)
            with torch.cuda.stream(side):
                tm, txt_qkv = text_qkv()
                text_pack(txt_qkv)

        # QKV projections; the video stream's q/k norm + RoPE into the joint buffers and K / V into
        # the ring (in its QKV projection when fused, after it otherwise)
        q8, s8 = self.norm_quant(img2, im[0], im[1], E)
        args = (img_cos, img_sin, q[0, :L], k[0, C:C + L], ring_k, ring_v, slot, v[0, C:C + L], n_cache,
                kv_cache_pre_rope)
        img_qkv = self._video_qkv(q8, s8, *args) if self.fuse_qkv else self.img.qkv.gemm(q8, s8)
        if text and side is None:
            tm, txt_qkv = text_qkv()
        mark("qkv")

        if not self.fuse_qkv:
            fused_qkv_norm_rope_cache(img_qkv, H, NORM_EPS, self.img.q_norm, self.img.k_norm, img_cos, img_sin,
                                      q[0, :L], k[0, C:C + L], ring_k, ring_v, slot, 0, v_out=v[0, C:C + L],
                                      cache_tokens=n_cache, cache_pre_rope=kv_cache_pre_rope)
        if write_slot is not None:
            ring.lengths[write_slot], ring.pre_rope[write_slot] = n_cache, kv_cache_pre_rope
            ring.touch(write_slot)
        mark("qkv_norm_rope")

        if not reuse_cached:
            self._cached_into(ring, cached, k, v)
        if joint is not None:
            joint.stamp = stamp
        mark("cached_kv")

        if side is not None:
            main.wait_stream(side)  # join: the condition rows of Q / K / V are written
        elif text:
            text_pack(txt_qkv)
        mark("joint_pack")
        attn = self.attention(q, k, v).flatten(2, 3)
        mark("attention")

        txt_out = []

        def fork_post():
            # fork after the video out-projection is queued: the condition stream's projection and
            # FFN then fill the CUs that the video GEMMs' last partial rounds and the memory-bound
            # quantisers leave idle (forked right after attention they compete with the video
            # out-projection's full rounds: 10.25-10.32 vs 10.23-10.29 ms per cfg-4 block, both
            # streams serial 10.39-10.43)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                txt_out.append(proj_ffn(txt2, self.txt, tm, attn[0, L:]))

        img_x = proj_ffn(img2, self.img, im, attn[0, :L], fork_post if side is not None else None)
        txt_x = txt_out[0] if txt_out else None
        if side is not None:
            main.wait_stream(side)
            txt_x.record_stream(main)  # allocated on the side stream, handed to the caller's
        elif text:
            txt_x = proj_ffn(txt2, self.txt, tm, attn[0, L:])
        mark("proj_ffn")
        txt_out = txt if skip_text_stream else txt_x.reshape(1, T, E)
        return img_x.reshape(1, L, E), txt_out
