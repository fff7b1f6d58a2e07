"""
GPU parity of the FFN half of the reference's pre-norm block, x + moe(norm_ffn(x))
(src/model/nanospeaker.py:169; RMSNorm ln.py:30-36), with the norm inside the router
kernel, the residual add inside the combine and the norm's backward + the residual's
gradient in one kernel (MoEBlock.forward_residual, nsmoe.h NSMOE_BLOCK_NORM):

  * the normalised input the router kernel stores: F.rms_norm's arithmetic (the oracle's
    rms_norm, pinned to torch's F.rms_norm on the CPU), equal up to one rounding step of
    the dtype where the fp32 rstd's last bit differs (summation order), and rstd to fp32
    rounding;
  * routing bit-exact and the block's output, every gradient and the balance loss to the
    bf16 bar against the oracle run on the kernel's own normalised input and logits;
  * out = x + the block output (each rounded), dx = g + the norm's backward of the
    block's input gradient, and the gain's gradient, against the oracle's closed forms
    (rms_norm_backward) to the bf16 bar;
  * the unfused path (fp32 blocks, or norm modules it does not take) is exactly
    x + block(norm(x)).

Sizes: T = 8192 train forward + backward, T = 2048 train forward, T = 32768 eval forward
(the prefill's per-layer call), T = 512 fp16, and ragged / other shapes.
"""

import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import assert_close_bf16
from tests.test_gpu_block import DEV, build

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import _native as nat  # noqa: E402
from nanospeaker_amd.decoder import RMSNorm  # noqa: E402


def make_norm(d, dtype, seed=3):
    g = torch.Generator().manual_seed(seed)
    norm = RMSNorm(d, 1e-6)
    with torch.no_grad():
        norm.gamma.copy_(1 + 0.1 * torch.randn(d, generator=g))
    return norm.to(dtype)


def run(T, train, backward, *, dtype=torch.bfloat16, scale=2.0, **cfg):
    m, p, x, g = build(T, dtype=dtype, **cfg)
    x = (x.float() * scale).to(dtype)  # a residual stream a few units wide
    d = x.shape[1]
    norm = make_norm(d, dtype)
    w = norm.gamma.detach().clone()
    m, norm = m.to(DEV).train(train), norm.to(DEV)
    xg = x.to(DEV).requires_grad_(backward)
    print(f"[norm] T={T} train={train} backward={backward} dtype={dtype} cfg={cfg}",
          flush=True)
    assert mk.norm_fusable(dtype, d, m.n_experts, m.top_k)
    out, aux, counts, idx, logits, saved, flags = mk.block_forward_state(
        xg, m.router.W, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, m.b_in, m.b_out, m.b_sh_in,
        m.b_sh_out, m.top_k, m.router.wants_probs(), m.router.normalize_weights, "silu",
        m.router.aux_loss_coef, norm_w=norm.gamma, norm_eps=1e-6)
    assert flags & nat.BLOCK_NORM
    if backward:
        torch.autograd.backward([out, aux], [g.to(DEV), torch.ones_like(aux)])
    torch.cuda.synchronize()
    h = m.W_in.shape[2] // 2
    S = 0 if m.W_sh_in is None else m.W_sh_in.shape[0]
    offs = mk.block_saved_offsets(T, m.n_experts, m.top_k, dtype, m.router.wants_probs(),
                                  bool(flags & nat.BLOCK_SAVE_ACT), d, h, S, True)
    xn = saved[offs[nat.SAVED_XN]:offs[nat.SAVED_XN] + T * d * 2].view(dtype).view(T, d).cpu()
    rstd = saved[offs[nat.SAVED_RSTD]:offs[nat.SAVED_RSTD] + T * 4].view(torch.float32).cpu()

    # the norm: the oracle's F.rms_norm arithmetic
    ref_xn, ref_rstd = R.rms_norm(x, w, 1e-6)
    # fp32 sums of d squares in two orders: a few units in the last place of rstd
    torch.testing.assert_close(rstd, ref_rstd, rtol=4e-6, atol=0)
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]  # relative, at most
    diff = (xn.float() - ref_xn.float()).abs()
    assert bool((diff <= ulp * ref_xn.float().abs() * 1.001 + 1e-30).all()), "xn off by > 1 ulp"
    print(f"  xn: {float((diff > 0).float().mean()):.2e} of elements one rounding step off "
          f"F.rms_norm's", flush=True)

    # the block on the kernel's own normalised input
    grads = {}
    if backward:
        grads = {"W": m.router.W.grad.cpu()}
        for n_ in ("W_in", "W_out", "W_sh_in", "W_sh_out", "b_in", "b_out", "b_sh_in",
                   "b_sh_out"):
            t = getattr(m, n_)
            if t is not None:
                grads[n_] = t.grad.cpu()
    ref = R.block(xn, p, m.top_k, train=train, grad_out=g if backward else None, fp32=True,
                  logits=logits.float().cpu())
    block_out = ref.out
    assert_close_bf16("out = x + block", out.detach().float().cpu(),
                      x.float() + block_out.float())
    if not backward:
        return ref
    # the block's own gradients (everything but dx) as the plain block's test holds them
    gr = ref.grads
    d_logits = gr["logits"]
    dxn = gr["x"] + d_logits @ p.W.float().t()
    assert_close_bf16("d router.W", grads.pop("W"), xn.float().t() @ d_logits)
    for name, got in grads.items():
        assert_close_bf16(f"d {name}", got, gr[name])
    # dx through the norm and the residual, and the gain's gradient
    dx_norm, dw = R.rms_norm_backward(dxn, x, w, rstd)
    assert_close_bf16("dx", xg.grad.float().cpu(), g.float() + dx_norm)
    assert_close_bf16("d gamma", norm.gamma.grad.float().cpu(), dw)
    if train:
        torch.testing.assert_close(aux.float().cpu().reshape(()),
                                   ref.aux_loss.float().reshape(()), rtol=1e-5, atol=1e-7)
    assert torch.equal(idx.cpu(), ref.topk_idx) and torch.equal(counts.cpu().long(), ref.counts)
    return ref


def test_forward_backward_T8192_train():
    run(8192, True, True)


def test_forward_T2048_train():
    run(2048, True, False)


def test_prefill_sublayer_T32768_eval():
    """The FFN sublayer exactly as the 20-layer prefill runs it in every layer (batch 4 x
    8192 = 32768 tokens, eval): the norm in the router kernel, the residual in the combine,
    196,608 routed pairs."""
    ref = run(32768, False, False)
    assert int(ref.counts.sum()) == 32768 * 6


def test_eval_forward_backward_T512_fp16():
    run(512, False, True, dtype=torch.float16)


@pytest.mark.parametrize("cfg", [dict(S=0, bias=True), dict(d=128, E=12, d_ff=96, k=4, S=1),
                                 dict(d=64, E=8, d_ff=96, k=2, S=2)])
def test_other_shapes(cfg):
    run(300, True, True, **cfg)


@pytest.mark.parametrize("waves", [8, 16])
def test_router_workgroup_shapes_with_the_norm(waves):
    """The norm inside the router kernel under both of its workgroup shapes (forced): 8
    waves, the default once the grid has more workgroups than CUs (the prefill's
    T = 32768 above), and 16."""
    from tests.helpers import lib_options

    with lib_options(router_waves=waves):
        run(300, True, True)
        run(1000, False, False)


def test_ragged_and_single_token():
    run(1, True, True)
    run(33, True, True)


def test_module_path_is_the_fused_sublayer_and_falls_back_exactly():
    """MoEBlock.forward_residual takes the fused op for a bf16 block, and for an fp32
    block is exactly x + block(norm(x))."""
    m, p, x, g = build(256)
    norm = make_norm(576, torch.bfloat16).to(DEV)
    m = m.to(DEV).train()
    xd = x.to(DEV)
    calls = nat.lib().nsmoe_launch_count()
    y = m.forward_residual(xd, norm)
    torch.cuda.synchronize()
    assert nat.lib().nsmoe_launch_count() > calls
    out, *_ = mk.block_forward(xd, m.router.W, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, None,
                               None, None, None, m.top_k, m.router.wants_probs(),
                               m.router.normalize_weights, "silu", m.router.aux_loss_coef,
                               norm_w=norm.gamma, norm_eps=1e-6)
    assert torch.equal(y, out)
    m32 = m.float()
    n32 = make_norm(576, torch.float32).to(DEV)
    x32 = xd.float()
    with torch.no_grad():
        torch.testing.assert_close(m32.forward_residual(x32, n32), x32 + m32(n32(x32)),
                                   rtol=0, atol=0)
