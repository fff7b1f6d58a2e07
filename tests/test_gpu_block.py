"""
End-to-end GPU parity of the drop-in MoEBlock at the benchmark's workloads.

The block runs on the GPU exactly as a caller runs it: one autograd node (router GEMM,
HIP route / dispatch / grouped experts / combine / balance loss, HIP backward).  The
block's router GEMM is recomputed on the GPU (the same bf16 GEMM, the same values) and
handed to the CPU oracle, so both sides route the same logits; from there:

  * routing indices, the per-expert counts and the dispatch permutation: bit-exact;
  * the output, dX, every expert weight gradient and router.W's gradient: within the
    bf16 bar against the fp32-accumulated oracle (max abs <= 2e-2 on the tensor's scale,
    rel-L2 <= 5e-3);
  * the balance loss: to fp32 rounding.

Workloads (seed 0, parameters in the reference's draw order, x ~ N(0, 1) in bf16):
  T = 2048 forward (train), T = 8192 forward + backward (train), T = 64 forward (eval),
  T = 16384 forward + backward with the skewed (Zipf 1.2) logit offset of
  tests/golden/zipf_logit_bias.npy, and a zero router (every token on the same experts).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import MoEBlock  # noqa: E402

DEV = "cuda"
ZIPF = Path(__file__).resolve().parent / "golden" / "zipf_logit_bias.npy"


def build(T, seed=0, zero_router=False):
    torch.manual_seed(seed)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(torch.bfloat16)
    if zero_router:
        with torch.no_grad():
            m.router.W.zero_()
    x = torch.randn(T, 576).to(torch.bfloat16)
    g = torch.randn(T, 576).to(torch.bfloat16)
    p = R.Params(m.router.W.data.clone(), m.W_in.data.clone(), m.W_out.data.clone(),
                 m.W_sh_in.data.clone(), m.W_sh_out.data.clone())
    return m, p, x, g


def check_against_oracle(x, p, g, logits, idx, counts, out, aux, grads, train, backward,
                         bias=None):
    """Routing bit-exact, outputs and gradients to the bf16 bar, against the oracle run on
    the GPU's own logits (the router GEMM's bf16 values)."""
    ref = R.block(x, p, 6, train=train, grad_out=g if backward else None, fp32=True,
                  logits=logits, logit_bias=bias)
    assert torch.equal(idx, ref.topk_idx), "routing indices differ"
    assert torch.equal(counts.long(), ref.counts), "counts differ"
    sids, _, offs, dcounts, _, inv = mk.moe_dispatch(idx.to(DEV), 76)
    r_sids, _, r_offs, r_counts, _, r_inv = R.dispatch_buffers(ref.topk_idx, 76, mk.ALIGN_M)
    assert torch.equal(sids.cpu(), r_sids) and torch.equal(inv.cpu(), r_inv)
    assert torch.equal(offs.cpu(), r_offs) and torch.equal(dcounts.cpu(), r_counts)
    assert_close_bf16("out", out.float(), ref.out)
    if train:
        torch.testing.assert_close(aux.float().cpu().reshape(()), ref.aux_loss.float().reshape(()),
                                   rtol=1e-5, atol=1e-7)
    else:
        assert float(aux) == 0.0
    if not backward:
        return ref
    gr = ref.grads
    d_logits = gr["logits"]
    assert_close_bf16("dx", grads["x"].float(), gr["x"] + d_logits @ p.W.float().t())
    assert_close_bf16("d router.W", grads["W"].float(), x.float().t() @ d_logits)
    for name in ("W_in", "W_out", "W_sh_in", "W_sh_out"):
        assert_close_bf16(f"d {name}", grads[name].float(), gr[name])
    return ref


def run_case(T, train, backward, zero_router=False):
    """The drop-in MoEBlock, as a caller runs it (one fused autograd node on the GPU)."""
    m, p, x, g = build(T, zero_router=zero_router)
    m = m.to(DEV).train(train)
    xg = x.to(DEV).requires_grad_(backward)
    print(f"[block] T={T} train={train} backward={backward} zero_router={zero_router}",
          flush=True)
    out = m(xg)
    assert m._use_kernel(xg.reshape(-1, 576)), "the HIP path was not taken"
    if backward:
        torch.autograd.backward([out, m.aux_loss], [g.to(DEV), torch.ones_like(m.aux_loss)])
    torch.cuda.synchronize()
    logits = (x.to(DEV) @ m.router.W.detach()).float().cpu()  # the block's own router GEMM
    grads = {}
    if backward:
        grads = {"x": xg.grad.cpu(), "W": m.router.W.grad.cpu()}
        grads.update({n: getattr(m, n).grad.cpu() for n in ("W_in", "W_out", "W_sh_in",
                                                            "W_sh_out")})
    return check_against_oracle(x, p, g, logits, m._routing.cpu(), m.expert_counts.cpu(),
                                out.detach().cpu(), m.aux_loss.detach().cpu(), grads, train,
                                backward)


def run_ops_case(T, bias):
    """The same kernels composed op by op (route -> moe_dispatch -> moe_block, balance loss
    in torch), with a harness-level per-expert offset added to the logits: the reference
    router has no bias, so the skewed workload cannot go through MoEBlock itself."""
    m, p, x, g = build(T)
    m = m.to(DEV).train(True)
    xg = x.to(DEV).requires_grad_(True)
    print(f"[ops] T={T} skewed", flush=True)
    logits = (xg @ m.router.W).float()
    w, idx, probs = mk.route(logits + bias.to(DEV), 6, True, True,
                             mk.route_dtype_code(torch.bfloat16))
    sids, _, offs, counts, _, inv = mk.moe_dispatch(idx, 76)
    out, _ = mk.moe_block(xg, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, None, None, None, None,
                          w, sids, offs, counts, inv, "silu")
    aux = m.router.balance_loss(probs, counts)
    torch.autograd.backward([out, aux], [g.to(DEV), torch.ones_like(aux)])
    torch.cuda.synchronize()
    grads = {"x": xg.grad.cpu(), "W": m.router.W.grad.cpu()}
    grads.update({n: getattr(m, n).grad.cpu() for n in ("W_in", "W_out", "W_sh_in",
                                                        "W_sh_out")})
    return check_against_oracle(x, p, g, logits.detach().cpu(), idx.cpu(), counts.cpu(),
                                out.detach().cpu(), aux.detach().cpu(), grads, True, True,
                                bias=bias)


def test_forward_T2048_train():
    run_case(2048, train=True, backward=False)


def test_forward_backward_T8192_train():
    run_case(8192, train=True, backward=True)


def test_decode_T64_eval():
    ref = run_case(64, train=False, backward=False)
    print(f"[block] T=64: {int((ref.counts == 0).sum())} empty experts", flush=True)


def test_eval_forward_backward_T512():
    """Eval branch (top-k on the logits, softmax over the k): its backward reads the bf16
    logits and writes bf16 d(logits) straight into the router GEMM's backward."""
    run_case(512, train=False, backward=True)


def test_skewed_T16384_forward_backward():
    bias = torch.from_numpy(np.load(ZIPF, allow_pickle=False))
    ref = run_ops_case(16384, bias)
    share = ref.counts.double() / ref.counts.sum()
    assert 0.12 < float(share.max()) < 1 / 6 + 1e-9   # the hot expert holds ~15 %


def test_zero_router_sends_every_token_to_the_same_experts():
    ref = run_case(2048, train=True, backward=True, zero_router=True)
    assert int((ref.counts > 0).sum()) == 6 and int(ref.counts.max()) == 2048
