"""
End-to-end GPU parity of the drop-in MoEBlock at the benchmark's workloads.

The block runs on the GPU exactly as a caller runs it (router GEMM, HIP route / dispatch /
grouped experts / combine, HIP backward, torch autograd around them).  The logits the
block's router produced are captured at the route op and handed to the CPU oracle, so
both sides route the same fp32 values; from there:

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


class RouteTap:
    """Wraps moe_kernel.route: records the logits the router produced (and adds a fixed
    per-expert offset first, for the skewed workload) and the op's outputs."""

    def __init__(self, bias=None):
        self.orig = mk.route
        self.bias = bias
        self.calls = []

    def __call__(self, logits, top_k, want_probs, normalize, w_dtype):
        src = logits if self.bias is None else logits + self.bias
        w, idx, probs = self.orig(src, top_k, want_probs, normalize, w_dtype)
        self.calls.append((logits.detach().cpu(), idx.detach().cpu()))
        return w, idx, probs


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


def run_case(monkeypatch, T, train, backward, bias=None, zero_router=False):
    m, p, x, g = build(T, zero_router=zero_router)
    tap = RouteTap(None if bias is None else bias.to(DEV))
    monkeypatch.setattr(mk, "route", tap)
    m = m.to(DEV).train(train)
    xg = x.to(DEV).requires_grad_(backward)
    print(f"[block] T={T} train={train} backward={backward} "
          f"skewed={bias is not None} zero_router={zero_router}", flush=True)
    out = m(xg)
    assert m._use_kernel(xg.reshape(-1, 576)), "the HIP path was not taken"
    if backward:
        torch.autograd.backward([out, m.aux_loss], [g.to(DEV), torch.ones_like(m.aux_loss)])
    torch.cuda.synchronize()
    assert len(tap.calls) == 1
    logits, idx = tap.calls[0]

    ref = R.block(x, p, 6, train=train, grad_out=g if backward else None, fp32=True,
                  logits=logits, logit_bias=bias)
    # routing and the permutation: bit-exact
    assert torch.equal(idx, ref.topk_idx), "routing indices differ"
    assert torch.equal(m.expert_counts.cpu().long(), ref.counts), "counts differ"
    sids, _, offs, counts, _, inv = mk.moe_dispatch(idx.to(DEV), 76)
    r_sids, _, r_offs, r_counts, _, r_inv = R.dispatch_buffers(ref.topk_idx, 76, mk.ALIGN_M)
    assert torch.equal(sids.cpu(), r_sids) and torch.equal(inv.cpu(), r_inv)
    assert torch.equal(offs.cpu(), r_offs) and torch.equal(counts.cpu(), r_counts)
    # output and balance loss
    assert_close_bf16("out", out.detach().float(), ref.out)
    if train:
        torch.testing.assert_close(m.aux_loss.detach().float().cpu(), ref.aux_loss.float(),
                                   rtol=1e-5, atol=1e-7)
    else:
        assert float(m.aux_loss) == 0.0
    if not backward:
        return ref
    gr = ref.grads
    w32 = p.W.float()
    d_logits = gr["logits"]
    assert_close_bf16("dx", xg.grad.float(), gr["x"] + d_logits @ w32.t())
    assert_close_bf16("d router.W", m.router.W.grad.float(), x.float().t() @ d_logits)
    for name, key in (("W_in", "W_in"), ("W_out", "W_out"), ("W_sh_in", "W_sh_in"),
                      ("W_sh_out", "W_sh_out")):
        assert_close_bf16(f"d {name}", getattr(m, name).grad.float(), gr[key])
    return ref


def test_forward_T2048_train(monkeypatch):
    run_case(monkeypatch, 2048, train=True, backward=False)


def test_forward_backward_T8192_train(monkeypatch):
    run_case(monkeypatch, 8192, train=True, backward=True)


def test_decode_T64_eval(monkeypatch):
    ref = run_case(monkeypatch, 64, train=False, backward=False)
    print(f"[block] T=64: {int((ref.counts == 0).sum())} empty experts", flush=True)


def test_skewed_T16384_forward_backward(monkeypatch):
    bias = torch.from_numpy(np.load(ZIPF, allow_pickle=False))
    ref = run_case(monkeypatch, 16384, train=True, backward=True, bias=bias)
    share = ref.counts.double() / ref.counts.sum()
    assert 0.12 < float(share.max()) < 1 / 6 + 1e-9   # the hot expert holds ~15 %


def test_zero_router_sends_every_token_to_the_same_experts(monkeypatch):
    ref = run_case(monkeypatch, 2048, train=True, backward=True, zero_router=True)
    assert int((ref.counts > 0).sum()) == 6 and int(ref.counts.max()) == 2048
