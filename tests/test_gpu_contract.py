"""
The drop-in contract around the kernels, on the GPU (reference: tests/test_moe_kernel.py
:224-254 and src/model/nanospeaker.py:224-227):

  * torch.library.opcheck on the ops -- schema, fake tensors, autograd registration and,
    for the ops whose every output byte is defined, AOT dispatch with dynamic shapes;
  * torch.compile(MoEBlock, fullgraph=True): forward and backward trace without a graph
    break and equal eager;
  * reentrant activation checkpointing (the trainer's use_reentrant=True) gives the
    unwrapped block's gradients bit for bit;
  * the same three for the pre-norm FFN half x + moe(norm(x)) (MoEBlock.forward_residual,
    the norm and residual inside the block's op);
  * the weight-pack cache: reused while the weights are unchanged, invalidated by an
    in-place optimizer update, with the updated block still matching the oracle.
"""

import importlib.util

import pytest
import torch
from torch.utils.checkpoint import checkpoint

from oracle import moe_ref as R
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import MoEBlock  # noqa: E402
from nanospeaker_amd import _native as nat  # noqa: E402

DEV = "cuda"


def small_block(dtype=torch.float32, **kw):
    torch.manual_seed(0)
    m = MoEBlock(**{"d_model": 32, "n_experts": 8, "d_ff": 64, "fused": False,
                    "capacity_factor": None, "n_shared": 1, **kw})
    return m.to(dtype).to(DEV)


def test_opcheck_dispatch_and_expert_ops():
    print("[contract] opcheck moe_dispatch / moe_experts / moe_block", flush=True)
    topk_idx = torch.randint(0, 4, (10, 2), device=DEV)
    torch.library.opcheck(mk.moe_dispatch, (topk_idx, 4))
    m = small_block(n_experts=4)
    x = torch.randn(10, 32, device=DEV)
    with torch.no_grad():
        topk_w, topk_idx, _ = m.router(x)
    sids, eids, offs, counts, npp, inv = mk.moe_dispatch(topk_idx, 4)
    leaf = lambda t: t.detach().clone().requires_grad_(True)
    torch.library.opcheck(mk.moe_experts, (
        leaf(x), leaf(m.W_in), leaf(m.W_out), leaf(topk_w), None, None,
        sids, eids, offs, counts, npp, inv, "silu"))
    torch.library.opcheck(mk.moe_block, (
        leaf(x), leaf(m.W_in), leaf(m.W_out), leaf(m.W_sh_in), leaf(m.W_sh_out), None, None,
        None, None, leaf(topk_w), sids, offs, counts, inv, "silu"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_opcheck_block_op(dtype):
    """nsmoe::block_fwd.  Its `saved` output carries alignment gaps the kernels never
    write, so AOT dispatch (which compares every output byte) is left to the compile test
    below, which compares what a caller sees."""
    print(f"[contract] opcheck block_fwd {dtype}", flush=True)
    m = small_block(dtype)
    x = torch.randn(13, 32, device=DEV).to(dtype)
    leaf = lambda t: t.detach().clone().requires_grad_(True)
    args = (leaf(x), leaf(m.router.W), leaf(m.W_in), leaf(m.W_out), leaf(m.W_sh_in),
            leaf(m.W_sh_out), None, None, None, None, 2, True, True, "silu", 1e-2)
    torch.library.opcheck(mk.block_fwd, args,
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))


def test_opcheck_block_op_with_norm():
    """nsmoe::block_fwd with the RMSNorm gain: x is the residual stream."""
    print("[contract] opcheck block_fwd + norm", flush=True)
    m = small_block(torch.bfloat16)
    x = torch.randn(13, 32, device=DEV).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(32, device=DEV)).to(torch.bfloat16)
    leaf = lambda t: t.detach().clone().requires_grad_(True)
    args = (leaf(x), leaf(m.router.W), leaf(m.W_in), leaf(m.W_out), leaf(m.W_sh_in),
            leaf(m.W_sh_out), None, None, None, None, 2, True, True, "silu", 1e-2, None,
            True, leaf(w), 1e-6)
    torch.library.opcheck(mk.block_fwd, args,
                          test_utils=("test_schema", "test_autograd_registration",
                                      "test_faketensor"))


class PreNormFFN(torch.nn.Module):
    """The FFN half of the reference's Block.forward (nanospeaker.py:169)."""

    def __init__(self, dtype):
        super().__init__()
        from nanospeaker_amd.decoder import RMSNorm
        self.ffn = small_block(dtype)
        self.norm = RMSNorm(32).to(dtype).to(DEV)
        with torch.no_grad():
            self.norm.gamma.copy_(1 + 0.1 * torch.randn(32, device=DEV))

    def forward(self, x):
        return self.ffn.forward_residual(x, self.norm), self.ffn.aux_loss


def test_pre_norm_ffn_compiles_fullgraph_and_checkpoints():
    """torch.compile(fullgraph) and a reentrant checkpoint of x + moe(norm(x)) give the
    eager module's output, balance loss and every gradient bit for bit."""
    print("[contract] pre-norm FFN: compile + checkpoint", flush=True)
    torch._dynamo.reset()
    torch.manual_seed(1)
    mods = [PreNormFFN(torch.bfloat16) for _ in range(3)]
    for q in mods[1:]:
        q.load_state_dict(mods[0].state_dict())
    eager, comp, ckpt = mods
    cm = torch.compile(comp, fullgraph=True, backend="aot_eager")
    x = (2 * torch.randn(2, 33, 32, device=DEV)).to(torch.bfloat16)
    g = torch.randn(2, 33, 32, device=DEV).to(torch.bfloat16)

    def grads(fn, mod):
        xg = x.clone().requires_grad_(True)
        out, aux = fn(xg)
        ((out.float() * g.float()).sum() + aux).backward()
        return out.detach(), aux.detach(), [xg.grad] + [p.grad for p in mod.parameters()]

    ref = grads(eager, eager)
    for got in (grads(cm, comp),
                grads(lambda t: checkpoint(ckpt, t, use_reentrant=True), ckpt)):
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
        for i, (a, b) in enumerate(zip(got[2], ref[2])):
            assert torch.equal(a, b), f"gradient {i}"


BACKENDS = ["aot_eager"] + (["inductor"] if importlib.util.find_spec("triton") else [])


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_compiles_fullgraph_through_forward_and_backward(backend, dtype):
    print(f"[contract] torch.compile fullgraph backend={backend} {dtype}", flush=True)
    torch._dynamo.reset()
    m = small_block(dtype)
    twin = small_block(dtype)
    cm = torch.compile(m, fullgraph=True, backend=backend)
    x = torch.randn(2, 33, 32, device=DEV).to(dtype)
    xc, xe = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    out = cm(xc)
    (out.float().square().mean() + m.aux_loss).backward()
    ref = twin(xe)
    (ref.float().square().mean() + twin.aux_loss).backward()
    assert torch.equal(out, ref)
    assert torch.equal(m.aux_loss, twin.aux_loss)
    assert torch.equal(m.expert_counts, twin.expert_counts)
    assert torch.equal(xc.grad, xe.grad)
    for (n, a), (_, b) in zip(m.named_parameters(), twin.named_parameters()):
        assert torch.equal(a.grad, b.grad), n


def test_reentrant_checkpoint_equals_unwrapped():
    """nanospeaker.py:224-227 runs each block under checkpoint(use_reentrant=True): the
    forward without autograd, then again with it during the backward."""
    print("[contract] reentrant checkpoint", flush=True)
    torch.manual_seed(0)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(torch.bfloat16).to(DEV).train()
    x = torch.randn(2048, 576, device=DEV).to(torch.bfloat16)
    g = torch.randn(2048, 576, device=DEV).to(torch.bfloat16)

    def body(t):
        return m(t), m.aux_loss

    def grads(wrap):
        m.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        out, aux = checkpoint(body, xg, use_reentrant=True) if wrap else body(xg)
        ((out.float() * g.float()).sum() + aux).backward()
        return [xg.grad] + [p.grad.clone() for p in m.parameters()], out.detach(), aux.detach()

    plain, out_p, aux_p = grads(False)
    ckpt, out_c, aux_c = grads(True)
    assert torch.equal(out_p, out_c) and torch.equal(aux_p, aux_c)
    for i, (a, b) in enumerate(zip(plain, ckpt)):
        assert torch.equal(a, b), f"gradient {i}"


def test_pack_cache_reuse_and_invalidation():
    print("[contract] pack cache", flush=True)
    torch.manual_seed(0)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(torch.bfloat16).to(DEV).eval()
    x = torch.randn(512, 576).to(torch.bfloat16)
    xd = x.to(DEV)
    mk.PACKS.clear()
    h0, m0 = mk.PACKS.hits, mk.PACKS.misses

    def packed_by(call):
        # the library's named stages that packed: the pack launch, or the place launch
        # that packs beside its placement workgroups
        nat.timing_enable(256)
        try:
            out = call()
            torch.cuda.synchronize()
            return out, sum(nat.timing_read(k)[1] for k in ("pack", "place_pack"))
        finally:
            nat.timing_enable(0)

    with torch.no_grad():
        out1, packs1 = packed_by(lambda: m(xd))
        out2, packs2 = packed_by(lambda: m(xd))
    assert (mk.PACKS.misses - m0, mk.PACKS.hits - h0) == (1, 1)
    assert packs1 == 1 and packs2 == 0, f"pack stages per call: {packs1}, then {packs2}"
    assert torch.equal(out1, out2)
    # an optimizer step updates the weights in place: the next call packs again
    opt = torch.optim.SGD(m.parameters(), lr=1.0)
    for p in m.parameters():
        p.grad = torch.randn_like(p) * 0.01
    opt.step()
    with torch.no_grad():
        out3 = m(xd)
    assert mk.PACKS.misses - m0 == 2
    fields = ("W_in", "W_out", "W_sh_in", "W_sh_out")
    p = R.Params(m.router.W.detach().cpu(), *(getattr(m, f).detach().cpu() for f in fields))
    logits = m._logits.float().cpu()
    ref = R.block(x, p, 6, train=False, fp32=True, logits=logits)
    assert torch.equal(m._routing.cpu(), ref.topk_idx)
    assert_close_bf16("out after the update", out3.float().cpu(), ref.out)
    assert not torch.equal(out3, out1)


def test_pack_cache_hits_for_cast_parameters():
    """fp32 parameters with bf16 activations (an autocast-style caller): every call hands
    the op fresh bf16 casts, and the cache, keyed on the parameters, packs once -- the
    second call and the reentrant checkpoint's forward and recompute all hit -- while
    the output still matches the oracle run on the cast weights."""
    print("[contract] pack cache with cast parameters", flush=True)
    torch.manual_seed(0)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, capacity_factor=None, fused=False)
    m = m.to(DEV).eval()  # fp32 parameters
    x = torch.randn(512, 576).to(torch.bfloat16)
    xd = x.to(DEV)
    mk.PACKS.clear()
    h0, m0 = mk.PACKS.hits, mk.PACKS.misses
    with torch.no_grad():
        out1 = m(xd)
        out2 = m(xd)
    assert (mk.PACKS.misses - m0, mk.PACKS.hits - h0) == (1, 1)
    assert torch.equal(out1, out2)
    fields = ("W_in", "W_out", "W_sh_in", "W_sh_out")
    p = R.Params(m.router.W.detach().cpu().to(torch.bfloat16),
                 *(getattr(m, f).detach().cpu().to(torch.bfloat16) for f in fields))
    ref = R.block(x, p, 6, train=False, fp32=True, logits=m._logits.float().cpu())
    assert torch.equal(m._routing.cpu(), ref.topk_idx)
    assert_close_bf16("out, cast parameters", out1.float().cpu(), ref.out)
    m.train()
    xg = xd.clone().requires_grad_(True)
    out, aux = checkpoint(lambda t: (m(t), m.aux_loss), xg, use_reentrant=True)
    ((out.float() ** 2).mean() + aux).backward()
    torch.cuda.synchronize()
    assert (mk.PACKS.misses - m0, mk.PACKS.hits - h0) == (1, 3), \
        (mk.PACKS.misses - m0, mk.PACKS.hits - h0)
    assert all(t.grad is not None and t.grad.dtype == torch.float32 for t in m.parameters())
