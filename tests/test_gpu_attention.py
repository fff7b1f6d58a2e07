"""
GPU parity of the prefill attention kernels (nsmoe_attn_prefill, nanospeaker_amd/csrc/
attention.hip) against the reference's attention semantics (src/model/mha.py:245-287 on the
SDPA path, masks mha.py:49-66): per-head RMSNorm of Q and K, rotary embedding, causal
attention with a sliding window (the query counted) or over the whole prefix, grouped-query
heads.

The reference side is the harness's torch path (decoder.Attention with kernel=False) on
the same projection the kernel reads: F.rms_norm and the rotation in bf16 tensor ops,
exactly as the reference module computes them, followed here by attention in fp32 (scores,
mask, softmax and P V chunked over the queries, every key of the prefix materialised): the
fp32-accumulated reference the north star's bar is read against.

  * the key heads the kernel normalises and rotates in place equal the torch path's bf16
    keys up to one bf16 step of the rotation's inputs (F.rms_norm's rstd can differ in its
    last bit; the rest is the same sequence of bf16 roundings);
  * the attention output (before W_O) is within the bf16 bar of the fp32 attention on the
    torch path's bf16 q / k / v: max abs <= 2e-2 on the tensor's scale, rel-L2 <= 5e-3;
  * the module's output after W_O is within the bar of the torch path run in fp32 on the
    same bf16 projections.

Shapes: the prefill workload's heads (9 query / 3 key-value heads, head dim 64) at
T = 8192 with the 512-token window and with full causal attention, and ragged lengths,
batches, tiny windows and the other grouped-query ratios (1, 2, 4) the kernel takes.
"""

import math

import pytest
import torch

from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd.decoder import (Attention, DecoderConfig, Rotary,  # noqa: E402
                                     attn_prefill)

DEV = "cuda"


def make_attention(h, hk, window, seed=0, base=500_000.0):
    torch.manual_seed(seed)
    cfg = DecoderConfig(n_layers=20, n_heads=h, n_kv_heads=hk, rope_base=base)
    att = Attention(cfg, Rotary(64, base), window, kernel=True)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        att.q_norm.gamma.copy_(1 + 0.2 * torch.randn(64, generator=g))
        att.k_norm.gamma.copy_(1 + 0.2 * torch.randn(64, generator=g))
    return att.to(torch.bfloat16).to(DEV).eval()


def torch_qkv(att, qkv, B, T):
    """q [B, h, T, 64], k, v [B, hk, T, 64] as the torch path computes them (bf16), from
    the projection qkv [B * T, (h + 2 hk) 64] the kernel reads: the same GEMM output on
    both sides (the separate z W_q, z W_k, z W_v GEMMs of the torch path may round their
    sums in another order), so the comparison isolates the kernels."""
    h, hk = att.h, att.hk
    heads = qkv.view(B, T, h + 2 * hk, 64).transpose(1, 2)
    q, k, v = heads[:, :h], heads[:, h:h + hk], heads[:, h + hk:]
    return att.rotary(att.q_norm(q)), att.rotary(att.k_norm(k)), v.contiguous()


def ref_attention(q, k, v, window):
    """fp32 causal attention (optionally windowed, the query counted) with grouped heads,
    chunked over the queries; q [B, H, T, 64], k / v [B, Hk, T, 64] -> [B, T, H * 64]."""
    B, H, T, dh = q.shape
    G = H // k.shape[1]
    q, k, v = q.float(), k.float().repeat_interleave(G, 1), v.float().repeat_interleave(G, 1)
    kt = k.transpose(-1, -2).contiguous()
    out = torch.empty(B, H, T, dh, device=q.device)
    kj = torch.arange(T, device=q.device)[None, :]
    for s in range(0, T, 512):
        e = min(T, s + 512)
        sc = (q[:, :, s:e] @ kt) / math.sqrt(dh)
        qi = torch.arange(s, e, device=q.device)[:, None]
        allowed = kj <= qi
        if window is not None:
            allowed = allowed & (qi - kj < window)
        sc = sc.masked_fill(~allowed, float("-inf"))
        out[:, :, s:e] = torch.softmax(sc, -1) @ v
    return out.transpose(1, 2).reshape(B, T, H * dh)


def run(B, T, h, hk, window, seed=0):
    print(f"[attn] B={B} T={T} heads={h}/{hk} window={window}", flush=True)
    att = make_attention(h, hk, window, seed)
    z = (torch.randn(B, T, 576, generator=torch.Generator().manual_seed(seed + 2))
         .to(torch.bfloat16).to(DEV))
    with torch.no_grad():
        assert att.use_kernel(z)
        w = torch.cat((att.W_q, att.W_k, att.W_v), dim=1)
        qkv = z.reshape(B * T, -1) @ w
        qkv_raw = qkv.clone()
        q, k, v = torch_qkv(att, qkv_raw, B, T)
        cos, sin = att.rotary.tables_f32(T, z.device)
        o = attn_prefill(qkv, B, T, h, hk, att.q_norm.gamma, att.k_norm.gamma, cos, sin,
                         window, att.q_norm.eps)
        torch.cuda.synchronize()
        # the key heads, normalised and rotated in place: where F.rms_norm's rstd differs
        # in its last bit a normalised element moves by one bf16 step (at most 2^-7 of its
        # size), and the rotation carries that into both outputs of its plane, so the
        # bound is one step of the plane's inputs plus one of the output
        k_got = qkv[:, h * 64:(h + hk) * 64].reshape(B, T, hk, 64).transpose(1, 2)
        n = att.k_norm(qkv_raw[:, h * 64:(h + hk) * 64].reshape(B, T, hk, 64)
                       .transpose(1, 2)).float().abs()
        plane = n + torch.cat((n[..., 32:], n[..., :32]), -1)
        diff = (k_got.float() - k.float()).abs()
        bound = 2.0 ** -7 * (plane + k.float().abs()) * 1.001
        worst = float((diff / (bound + 1e-30)).max())
        print(f"  keys: {float((diff > 0).float().mean()):.2e} of elements differ from the "
              f"torch path; worst {worst:.2f} of the bound", flush=True)
        assert worst <= 1.0, "prepared keys off by more than one bf16 step of their inputs"
        ref = ref_attention(q, k, v, window)
        assert_close_bf16("attention output", o.float().cpu(), ref.reshape(B * T, -1).cpu())
        # the whole module (W_O included) against the torch path's projections in fp32
        out = att(z)
        ref_mod = ref.reshape(B, T, -1) @ att.W_O.float()
        assert_close_bf16("module output", out.float().cpu(), ref_mod.cpu())


def test_prefill_shape_window_512_T8192():
    run(1, 8192, 9, 3, 512)


def test_prefill_shape_full_causal_T8192():
    run(1, 8192, 9, 3, None)


@pytest.mark.parametrize("B,T,h,hk,window", [
    (2, 1000, 9, 3, 512),   # ragged length, two sequences
    (1, 100, 9, 3, 7),      # a tiny window
    (1, 130, 9, 3, 1),      # each query sees itself only
    (2, 65, 4, 4, None),    # plain multi-head, one key past a tile
    (1, 300, 8, 4, 64),     # two query heads per key/value head
    (1, 200, 8, 2, None),   # four query heads per key/value head
    (1, 1, 9, 3, 512),      # one token
    (3, 577, 9, 3, 600),    # the window longer than the sequence: full causal
])
def test_ragged_windows_and_head_groups(B, T, h, hk, window):
    run(B, T, h, hk, window, seed=T)


def test_module_falls_back_to_torch_when_differentiated():
    att = make_attention(9, 3, 512)
    z = torch.randn(1, 64, 576, device=DEV).to(torch.bfloat16).requires_grad_(True)
    assert not att.use_kernel(z)
    att(z).float().sum().backward()
    assert z.grad is not None


@pytest.mark.parametrize("shape,dt", [((8192, 576), torch.bfloat16), ((3, 7, 64), torch.float16),
                                      ((1, 1024), torch.bfloat16)])
def test_rms_norm_kernel_matches_the_oracle(shape, dt):
    """nsmoe_rms_norm (the attention's pre-norm and the final norm on the kernel path)
    against the oracle's restatement of F.rms_norm (pinned bit for bit to torch's CPU
    F.rms_norm): equal up to one rounding step where the fp32 rstd's last bit differs
    (summation order), and the module takes the kernel for a gradient-free 16-bit call."""
    from oracle import moe_ref as R
    from nanospeaker_amd.decoder import RMSNorm, rms_norm
    g = torch.Generator().manual_seed(shape[-1])
    x = (torch.randn(*shape, generator=g) * 3).to(dt)
    w = (1 + 0.2 * torch.randn(shape[-1], generator=g)).to(dt)
    ref, _ = R.rms_norm(x, w, 1e-6)
    got = rms_norm(x.to(DEV), w.to(DEV), 1e-6).cpu()
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dt]
    diff = (got.float() - ref.float()).abs()
    assert bool((diff <= ulp * ref.float().abs() * 1.001 + 1e-30).all())
    print(f"  rms_norm {shape}: {float((diff > 0).float().mean()):.2e} of elements one step off",
          flush=True)
    norm = RMSNorm(shape[-1], 1e-6).to(dt).to(DEV)
    with torch.no_grad():
        norm.gamma.copy_(w)
        assert norm.use_kernel(x.to(DEV))
        assert torch.equal(norm(x.to(DEV)).cpu(), got)


def test_residual_in_place_equals_the_copying_add():
    """forward_residual(inplace=True) accumulates x + o W_O into x's own memory (no copy
    of the addend) and gives the same bits as the copying form."""
    att = make_attention(9, 3, 512)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 300, 576, generator=g).to(torch.bfloat16).to(DEV)
    z = torch.randn(2, 300, 576, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        ref = att.forward_residual(x.clone(), z)
        xi = x.clone()
        got = att.forward_residual(xi, z, inplace=True)
    assert got.data_ptr() == xi.data_ptr()
    assert torch.equal(got, ref)


def test_decoder_trunk_matches_its_blocks_run_one_by_one():
    """The trunk (which lets each block's attention add its residual in place) against
    the blocks called one at a time with copying adds."""
    from nanospeaker_amd.decoder import Decoder
    torch.manual_seed(0)
    model = Decoder(DecoderConfig(n_layers=2, vocab_size=512)).to(torch.bfloat16)
    model = model.to(DEV).eval()
    idx = torch.randint(0, 512, (1, 200), device=DEV)
    with torch.no_grad():
        h, _ = model.trunk(idx)
        x = model.embed(idx)
        for blk in model.blocks:
            x, _ = blk(x)
        ref = model.norm_out(x)
    assert torch.equal(h, ref)
