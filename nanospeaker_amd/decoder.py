"""
The decoder around the MoE block, for the 20-layer prefill workload (reference:
src/model/nanospeaker.py:133-269 -- embedding, 20 pre-norm blocks of attention and MoE,
final norm, tied unembedding; src/model/mha.py:245-287 for the attention, ln.py:30-36
for RMSNorm, rope.py for the rotary embedding).

The FFN half of each block, x + moe(norm_ffn(x)), runs through MoEBlock.forward_residual,
which takes the RMSNorm and the residual add into the block's HIP kernels.  The attention
of a gradient-free 16-bit forward on the GPU (the prefill) runs through `attn_prefill`,
the library's HIP kernels (nsmoe_attn_prefill: QK-norm, RoPE, windowed or full causal
grouped-query flash attention) between two torch GEMMs, the fused Q/K/V projection and
W_O.  Everywhere else (CPU, fp32 / fp64, a forward that autograd differentiates, or
`kernel=False`) the attention is plain PyTorch: `F.rms_norm`, the rotation in the dtype
and `scaled_dot_product_attention` (the reference's SDPA path, `flex=False`); that path is
also the GPU kernel's reference in the tests.  The stack runs the prefill of the
benchmark's fifth workload (batch 4 x 8192 tokens, eval, bf16) with the MoE kernels in
situ, so the block's share of a real forward can be measured.

Attention follows the reference's semantics: grouped-query heads (9 query, 3 key/value,
d_head 64), a per-head RMSNorm of Q and K before the rotation, rotary embeddings with the
"rotate half" pairing over the whole head (base 500000 for this workload), causal
masking, and a sliding window of 512 keys (the query's own position counted) on every
layer but each `global_every`-th.  A windowed layer is computed in blocks of `window`
queries, each against the `2 window` keys that can reach it, with SDPA and the band
mask of that block -- the same result as one SDPA call under the full [T, T] band mask,
at 2 window / T of its work.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as nat
from .head import linear_cross_entropy
from .moe import MoEBlock


@dataclass
class DecoderConfig:
    """nanoSpeaker's decoder (nanospeaker.py:71-100) with the prefill workload's settings."""

    vocab_size: int = 32768
    d_model: int = 576
    n_layers: int = 20
    n_heads: int = 9
    n_kv_heads: int = 3
    d_head: int = 64
    n_experts: int = 76
    n_shared: int = 2
    top_k: int = 6
    d_expert: int = 128
    aux_loss_coef: float = 1e-2
    rope_base: float = 500_000.0
    window: "int | None" = 512
    global_every: "int | None" = 4
    std: float = 0.02
    norm_eps: float = 1e-6

    def layer_window(self, i: int) -> "int | None":
        """None (full causal attention) on every global_every-th layer, else the window."""
        if self.global_every and i % self.global_every == 0:
            return None
        return self.window


class RMSNorm(nn.Module):
    """x / rms(x) * gamma over the last dim (ln.py:30-36, F.rms_norm's arithmetic).  A
    gradient-free 16-bit forward of contiguous rows on the GPU runs the library's kernel
    (nsmoe_rms_norm: one HBM read and write of the rows); everything else is F.rms_norm."""

    def __init__(self, d: int, eps: float = 1e-6, kernel: bool = True):
        super().__init__()
        self.d, self.eps, self.kernel = d, eps, kernel
        self.gamma = nn.Parameter(torch.ones(d))

    def use_kernel(self, x: torch.Tensor) -> bool:
        return (self.kernel and x.is_cuda and x.dtype in _ATTN_DT
                and self.gamma.dtype == x.dtype and x.is_contiguous() and self.d % 8 == 0
                and self.d <= 1024
                and not (torch.is_grad_enabled() and (x.requires_grad or self.gamma.requires_grad)))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.use_kernel(x):
            return rms_norm(x, self.gamma, self.eps)
        return F.rms_norm(x, (self.d,), self.gamma, self.eps)


class Rotary:
    """Rotary position tables: plane j of a head turns by pos * base^(-2j / d_head); dim i
    pairs with dim i + d_head / 2.  The angles are formed in fp32 and the cos / sin
    tables cast once per compute dtype."""

    def __init__(self, d_head: int, base: float):
        self.d_head, self.base = d_head, base
        self._tables: dict = {}

    def tables(self, n: int, device, dtype):
        key = (n, str(device), dtype)
        hit = self._tables.get(key)
        if hit is None:
            half = self.d_head // 2
            inv = self.base ** (-torch.arange(half, dtype=torch.float32, device=device) * 2.0
                                / self.d_head)
            ang = torch.arange(n, dtype=torch.float32, device=device)[:, None] * inv[None, :]
            hit = self._tables[key] = (ang.cos().to(dtype), ang.sin().to(dtype))
        return hit

    def tables_f32(self, n: int, device):
        """The fp32 cos / sin tables [n, d_head / 2] (what `tables` casts)."""
        return self.tables(n, device, torch.float32)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        cos, sin = self.tables(x.shape[-2], x.device, x.dtype)
        half = self.d_head // 2
        a, b = x[..., :half], x[..., half:]
        return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


_ATTN_DT = {torch.bfloat16: nat.BF16, torch.float16: nat.F16}


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """F.rms_norm(x, (d,), w, eps) of a contiguous 16-bit GPU tensor on the library's kernel
    (nsmoe_rms_norm).  Forward only."""
    d = x.shape[-1]
    y = torch.empty_like(x)
    wc = w.detach().contiguous()
    nat.check(nat.lib().nsmoe_rms_norm(_ATTN_DT[x.dtype], x.data_ptr(), wc.data_ptr(),
                                       float(eps), x.numel() // d, d, y.data_ptr(), None,
                                       torch.cuda.current_stream().cuda_stream),
              "nsmoe_rms_norm")
    return y


def attn_prefill(qkv: torch.Tensor, B: int, T: int, n_heads: int, n_kv_heads: int,
                 q_gamma: torch.Tensor, k_gamma: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, window: "int | None", eps: float) -> torch.Tensor:
    """
    The attention of a prefill (positions 0 .. T - 1) on the library's HIP kernels
    (nsmoe_attn_prefill): qkv [B * T, (n_heads + 2 n_kv_heads) * 64] is the fused
    projection Z [W_q | W_k | W_v]; its key heads are normalised and rotated in place.
    Returns [B * T, n_heads * 64], the input of W_O.  q_gamma / k_gamma are the two
    RMSNorm gains, cos / sin the fp32 rotary tables [T, 32]; window None is full causal
    attention.  Forward only (no autograd).
    """
    if qkv.dtype not in _ATTN_DT:
        raise ValueError(f"attn_prefill: 16-bit types only, got {qkv.dtype}")
    dt = qkv.dtype
    qkv = qkv.contiguous()
    out = torch.empty((B * T, n_heads * 64), dtype=dt, device=qkv.device)
    qg = q_gamma.detach().to(dt).contiguous()
    kg = k_gamma.detach().to(dt).contiguous()
    cos, sin = cos.float().contiguous(), sin.float().contiguous()
    a = nat.AttnArgs(dtype=_ATTN_DT[dt], n_heads=n_heads, n_kv_heads=n_kv_heads,
                     head_dim=64, batch=B, seq_len=T, ld=qkv.shape[1],
                     window=0 if window is None else int(window), eps=float(eps),
                     reserved=0, qkv=qkv.data_ptr(), q_gamma=qg.data_ptr(),
                     k_gamma=kg.data_ptr(), cos=cos.data_ptr(), sin=sin.data_ptr(),
                     out=out.data_ptr())
    nat.check(nat.lib().nsmoe_attn_prefill(a, torch.cuda.current_stream().cuda_stream),
              "nsmoe_attn_prefill")
    return out


def band_attention(q, k, v, window: int) -> torch.Tensor:
    """
    Causal sliding-window attention (each query sees itself and the window - 1 keys before
    it) for q [B, Hq, T, dh] and k, v [B, Hkv, T, dh], Hq a multiple of Hkv.  Queries are
    taken in blocks of `window`; block b attends to keys [(b - 1) window, (b + 1) window)
    under its band mask, one batched SDPA call for all blocks.
    """
    B, Hq, T, dh = q.shape
    Hkv = k.shape[1]
    if Hkv != Hq:
        # Query head h reads key/value head h // (Hq / Hkv), as enable_gqa pairs them.  The
        # heads are expanded here because ROCm's SDPA takes a mask together with grouped
        # heads only on its math path (measured at the prefill shape: 3.5 ms per layer
        # against 0.71 ms on the memory-efficient kernel with expanded heads).
        k = k.repeat_interleave(Hq // Hkv, dim=1)
        v = v.repeat_interleave(Hq // Hkv, dim=1)
        Hkv = Hq
    w = window
    nb = -(-T // w)
    pad = nb * w - T
    if pad:
        q = F.pad(q, (0, 0, 0, pad))
        k = F.pad(k, (0, 0, 0, pad))
        v = F.pad(v, (0, 0, 0, pad))
    # keys of block b: the previous block (zeros before the first) and block b itself
    kb = k.view(B, Hkv, nb, w, dh)
    vb = v.view(B, Hkv, nb, w, dh)
    k2 = torch.cat((F.pad(kb, (0, 0, 0, 0, 1, 0))[:, :, :nb], kb), dim=3)
    v2 = torch.cat((F.pad(vb, (0, 0, 0, 0, 1, 0))[:, :, :nb], vb), dim=3)
    qb = q.view(B, Hq, nb, w, dh).transpose(1, 2).reshape(B * nb, Hq, w, dh)
    k2 = k2.transpose(1, 2).reshape(B * nb, Hkv, 2 * w, dh)
    v2 = v2.transpose(1, 2).reshape(B * nb, Hkv, 2 * w, dh)
    # query i of a block sits at key position w + i; key j is allowed when
    # 0 <= (w + i) - j < w, and the first block's previous-block keys do not exist
    qi = torch.arange(w, device=q.device)[:, None] + w
    kj = torch.arange(2 * w, device=q.device)[None, :]
    band = (kj <= qi) & (qi - kj < w)
    first = band & (kj >= w)
    mask = band.expand(B, nb, w, 2 * w).clone()
    mask[:, 0] = first
    mask = mask.reshape(B * nb, 1, w, 2 * w)
    out = F.scaled_dot_product_attention(qb, k2, v2, attn_mask=mask)
    out = out.view(B, nb, Hq, w, dh).transpose(1, 2).reshape(B, Hq, nb * w, dh)
    return out[:, :, :T]


class Attention(nn.Module):
    """Grouped-query self-attention with QK-norm, rotary embeddings and an optional window
    (reference: OptimizedMultiHeadAttention, mha.py:245-287, on its SDPA path)."""

    def __init__(self, cfg: DecoderConfig, rotary: Rotary, window: "int | None",
                 kernel: bool = True):
        super().__init__()
        d, h, hk, dh = cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.d_head
        self.h, self.hk, self.dh, self.window, self.rotary = h, hk, dh, window, rotary
        self.kernel = kernel
        self.W_q = nn.Parameter(torch.randn(d, h * dh) * cfg.std)
        self.W_k = nn.Parameter(torch.randn(d, hk * dh) * cfg.std)
        self.W_v = nn.Parameter(torch.randn(d, hk * dh) * cfg.std)
        # output projection damped by 1 / sqrt(2 n_layers), as the reference does
        self.W_O = nn.Parameter(torch.randn(h * dh, d) * cfg.std / math.sqrt(2 * cfg.n_layers))
        self.q_norm = RMSNorm(dh, cfg.norm_eps)
        self.k_norm = RMSNorm(dh, cfg.norm_eps)

    def use_kernel(self, z: torch.Tensor) -> bool:
        """The HIP prefill kernels take a gradient-free 16-bit forward on the GPU with
        64-wide heads and 1-4 query heads per key/value head."""
        return (self.kernel and z.is_cuda and z.dtype in _ATTN_DT and self.dh == 64
                and self.h % self.hk == 0 and self.h // self.hk <= 4
                and not (torch.is_grad_enabled() and any(
                    t.requires_grad for t in (z, self.W_q, self.W_k, self.W_v, self.W_O))))

    def _w_qkv(self, dtype) -> torch.Tensor:
        """[W_q | W_k | W_v] in `dtype`, kept while the three weights are unchanged (their
        identity, storage and autograd versions)."""
        key = tuple((t.data_ptr(), t._version) for t in (self.W_q, self.W_k, self.W_v))
        key += (dtype,)
        hit = getattr(self, "_qkv_cache", None)
        if hit is None or hit[0] != key:
            w = torch.cat((self.W_q, self.W_k, self.W_v), dim=1).to(dtype).detach()
            hit = self._qkv_cache = (key, w)
        return hit[1]

    def _w_o_t(self, dtype) -> torch.Tensor:
        """W_O in `dtype` as the transpose of a contiguous [d, h dh] copy, kept while W_O is
        unchanged: the library's GEMM of the residual update, x + o W_O, runs faster with
        that operand layout (47 against 53 us at the prefill's 32,768 x 576 x 576)."""
        key = (self.W_O.data_ptr(), self.W_O._version, dtype)
        hit = getattr(self, "_wo_cache", None)
        if hit is None or hit[0] != key:
            w = self.W_O.detach().to(dtype).t().contiguous()
            hit = self._wo_cache = (key, w)
        return hit[1].t()

    def _kernel_attention(self, z: torch.Tensor) -> torch.Tensor:
        """[B T, h dh]: the attention output before W_O, on the HIP prefill kernels."""
        B, T, _ = z.shape
        qkv = z.reshape(B * T, -1) @ self._w_qkv(z.dtype)
        cos, sin = self.rotary.tables_f32(T, z.device)
        return attn_prefill(qkv, B, T, self.h, self.hk, self.q_norm.gamma, self.k_norm.gamma,
                            cos, sin, self.window, self.q_norm.eps)

    def forward_residual(self, x: torch.Tensor, z: torch.Tensor,
                         inplace: bool = False) -> torch.Tensor:
        """x + self(z): on the kernel path the residual enters the W_O GEMM as its addend
        (one rounding of x + o W_O instead of two); elsewhere exactly x + self(z).  With
        `inplace` (a caller that owns x and needs it no more) the kernel path accumulates
        into x's own memory and returns x, which saves the library GEMM's copy of the
        addend (37.7 MB at the prefill's 32,768 x 576)."""
        if self.use_kernel(z) and x.dtype == z.dtype and not (
                torch.is_grad_enabled() and x.requires_grad):
            B, T, d = x.shape
            o = self._kernel_attention(z)
            w = self._w_o_t(z.dtype)
            if inplace and x.is_contiguous():
                x.view(B * T, d).addmm_(o, w)
                return x
            return torch.addmm(x.reshape(B * T, d), o, w).view(B, T, d)
        return x + self(z)

    def forward(self, z: torch.Tensor) -> torch.Tensor:
        B, T, _ = z.shape
        if self.use_kernel(z):
            o = self._kernel_attention(z)
            return o.view(B, T, self.h * self.dh) @ self.W_O
        q = (z @ self.W_q).view(B, T, self.h, self.dh).transpose(1, 2)
        k = (z @ self.W_k).view(B, T, self.hk, self.dh).transpose(1, 2)
        v = (z @ self.W_v).view(B, T, self.hk, self.dh).transpose(1, 2)
        q = self.rotary(self.q_norm(q))
        k = self.rotary(self.k_norm(k))
        if self.window is None or self.window >= T:
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True,
                                               enable_gqa=self.h != self.hk)
        else:
            o = band_attention(q, k, v, self.window)
        return o.transpose(1, 2).reshape(B, T, self.h * self.dh) @ self.W_O


class DecoderBlock(nn.Module):
    """Pre-norm block (nanospeaker.py:138-169): x + attn(norm(x)), then x + moe(norm(x))
    (MoEBlock.forward_residual).  Returns the new residual stream and the MoE block's
    balance loss."""

    def __init__(self, cfg: DecoderConfig, rotary: Rotary, layer: int, kernel: bool = True):
        super().__init__()
        self.norm_attn = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.attn = Attention(cfg, rotary, cfg.layer_window(layer), kernel)
        self.norm_ffn = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.ffn = MoEBlock(cfg.d_model, cfg.n_experts, 3 * cfg.d_expert // 2,
                            top_k=cfg.top_k, n_shared=cfg.n_shared, capacity_factor=None,
                            normalize_weights=True, aux_loss_coef=cfg.aux_loss_coef,
                            std=cfg.std, fused=False, kernel=kernel)

    def forward(self, x: torch.Tensor, inplace: bool = False):
        """`inplace`: the caller owns x and needs it no more (Attention.forward_residual)."""
        x = self.attn.forward_residual(x, self.norm_attn(x), inplace=inplace)
        return self.ffn.forward_residual(x, self.norm_ffn), self.ffn.aux_loss


class Decoder(nn.Module):
    """Embedding, the blocks, the final norm and the tied unembedding
    (nanospeaker.py:172-245); `forward(idx)` returns the logits [B, T, vocab]."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), kernel: bool = True):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        nn.init.normal_(self.embed.weight, std=cfg.std)
        rotary = Rotary(cfg.d_head, cfg.rope_base)
        self.blocks = nn.ModuleList(DecoderBlock(cfg, rotary, i, kernel)
                                    for i in range(cfg.n_layers))
        self.norm_out = RMSNorm(cfg.d_model, cfg.norm_eps)

    def trunk(self, idx: torch.Tensor, ffn_hook=None):
        """(final normed hidden states, summed balance loss).  ffn_hook, when given, is
        called as ffn_hook(block, x) in place of each block's FFN half and must return
        what it returns, x + moe(norm_ffn(x)) (the benchmark times those calls through
        it)."""
        x = self.embed(idx)
        aux = torch.zeros((), dtype=torch.float32, device=x.device)
        zeros16 = []
        # The residual stream is the trunk's own: the embedding's output, then each block's
        # fresh output, so the attention's residual add may accumulate in place.
        for blk in self.blocks:
            if ffn_hook is None:
                x, a = blk(x, inplace=True)
            else:
                x = blk.attn.forward_residual(x, blk.norm_attn(x), inplace=True)
                x = ffn_hook(blk, x)
                a = blk.ffn.aux_loss
            # The fp32 sum aux + a of the reference's trunk, a widened exactly (torch's
            # mixed-dtype add takes ~45 us for a 0-dim tensor on this stack).  A block
            # that computed no balance loss (eval, or a zero coefficient) returns a zero of
            # its dtype: those are summed once at the end, in one widening reduction,
            # instead of a conversion and an add per layer; a sum of zeros is zero in any
            # order.
            if not blk.ffn.router.wants_probs() and a.dtype != aux.dtype:
                zeros16.append(a)
            else:
                aux = aux + (a if a.dtype == aux.dtype else a.float())
        if zeros16:
            aux = aux + torch.stack(zeros16).sum(dtype=torch.float32)
        return self.norm_out(x), aux

    def forward(self, idx: torch.Tensor, targets: "torch.Tensor | None" = None,
                ffn_hook=None):
        """Logits [B, T, vocab] (the tied unembedding), or with `targets` [B, T] the
        next-token loss and the summed balance loss (nanospeaker.py:236-250): position t
        predicts token t + 1, through head.linear_cross_entropy (the HIP cross-entropy
        between library GEMMs on the GPU; F.cross_entropy of the materialised fp32 logits
        elsewhere), never materialising more logits than one chunk."""
        x, aux = self.trunk(idx, ffn_hook)
        if targets is None:
            return x @ self.embed.weight.t()
        h = x[:, :-1].reshape(-1, self.cfg.d_model)
        y = targets[:, 1:].reshape(-1)
        return linear_cross_entropy(h, self.embed.weight, y), aux
