"""
End-to-end GPU parity of the drop-in MoEBlock.

The block runs on the GPU exactly as a caller runs it: one op per direction (router GEMM,
HIP route / dispatch / grouped experts / combine / balance loss, HIP backward).  The
block's router GEMM is recomputed on the GPU (the same GEMM, the same values) and handed
to the CPU oracle, so both sides route the same logits; from there:

  * routing indices, the per-expert counts and the dispatch permutation: bit-exact;
  * the output, dX, every expert weight and bias gradient and router.W's gradient: within
    the bf16 bar against the fp32-accumulated oracle (max abs <= 2e-2 on the tensor's
    scale, rel-L2 <= 5e-3) for 16-bit blocks, and within fp32 rounding for fp32 blocks;
  * the balance loss: to fp32 rounding.

Workloads (seed 0, parameters in the reference's draw order, x ~ N(0, 1)): the benchmark's
configurations -- T = 2048 forward (train), T = 8192 forward + backward (train), T = 64
forward (eval), T = 16384 forward + backward with the skewed (Zipf 1.2) logit offset of
tests/golden/zipf_logit_bias.npy, and T = 32768 forward (eval), the per-layer shape of the
20-layer prefill -- a zero router (every token on the same experts), and a matrix of
dtypes, biases, shared-expert counts and shapes that take the block's other code paths
(the router backward in torch, the slow dx combine for k > 8 or more than two shared
experts).
"""

import math
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
NS = dict(d=576, E=76, d_ff=192, k=6, S=2)
# Largest share of tokens whose routing may differ between the block's logits and the CPU
# bf16 GEMM's (check_router_gemm; one token is always allowed).
FLIP_BOUND = 2e-3


def build(T, *, d=576, E=76, d_ff=192, k=6, S=2, bias=False, dtype=torch.bfloat16, seed=0,
          zero_router=False):
    torch.manual_seed(seed)
    m = MoEBlock(d, E, d_ff=d_ff, top_k=k, n_shared=S, bias=bias, capacity_factor=None,
                 fused=False)
    if bias:
        g_b = torch.Generator().manual_seed(seed + 11)
        with torch.no_grad():
            for name in ("b_in", "b_out", "b_sh_in", "b_sh_out"):
                t = getattr(m, name)
                if t is not None:
                    t.copy_(torch.randn(t.shape, generator=g_b) * 0.1)
    m = m.to(dtype)
    if zero_router:
        with torch.no_grad():
            m.router.W.zero_()
    x = torch.randn(T, d).to(dtype)
    g = torch.randn(T, d).to(dtype)
    fields = ("W_in", "W_out", "W_sh_in", "W_sh_out", "b_in", "b_out", "b_sh_in", "b_sh_out")
    p = R.Params(m.router.W.data.clone(), *(None if getattr(m, f) is None
                                             else getattr(m, f).data.clone() for f in fields))
    return m, p, x, g


def close(name, got, ref, dtype):
    """16-bit blocks: the bf16 bar.  fp32 blocks: fp32 rounding (max abs <= 1e-4 on the
    tensor's scale, rel-L2 <= 1e-5)."""
    if dtype == torch.float32:
        assert_close_bf16(name, got.float(), ref, max_abs=1e-4, rel_l2=1e-5)
    else:
        assert_close_bf16(name, got.float(), ref)


def check_router_gemm(x, W, logits, logit_bias, dt):
    """The block's logits are x W (+ the offset) accumulated in fp32 and rounded to the
    block's dtype: within one rounding step of the fp32 product.  Also reports how many
    tokens the CPU's own bf16 GEMM would route differently (accumulation order)."""
    ref = x.double() @ W.double()
    if logit_bias is not None:
        ref = ref + logit_bias.double()
    if dt == torch.float32:
        torch.testing.assert_close(logits.double(), ref, rtol=1e-5, atol=1e-5)
        return
    step = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dt]
    bound = step * ref.abs() * 1.01 + 1e-5
    err = (logits.double() - ref).abs()
    assert bool((err <= bound).all()), f"router GEMM off by {float((err / bound).max()):.2f} steps"
    if logit_bias is None:
        cpu = (x @ W).float()  # the CPU's own bf16 GEMM, as the reference computes it
    else:
        # the harness offset has no counterpart in the reference: its defined value is
        # the fp32 product plus the offset, rounded once (what the kernel computes)
        cpu = (x.float() @ W.float() + logit_bias.float()).to(dt).float()
    k = 6 if W.shape[1] >= 6 else 1
    flips = (R.route_from_logits(cpu, k, False, True, dt)[1]
             != R.route_from_logits(logits, k, False, True, dt)[1]).any(1).float().mean()
    differ = float((logits != cpu).float().mean())
    print(f"  router GEMM: {differ:.4f} of logits differ from the CPU bf16 GEMM; routing "
          f"flips on {float(flips):.4%} of tokens", flush=True)
    # Both GEMMs sum in fp32 and round once; they differ only in summation order, which
    # moves about 1e-4 of the logits by one rounding step.  A token's routing can flip
    # only where such a logit sits at its top-k boundary (one of the ~k + 1 contenders):
    # about 76 * 1e-4 * 7 / 76 = 7e-4 of the tokens at most.
    n_flip, n_tok = round(float(flips) * x.shape[0]), x.shape[0]
    assert n_flip <= max(1, FLIP_BOUND * n_tok), f"routing flips on {n_flip} of {n_tok} tokens"


def check_against_oracle(x, p, g, logits, idx, counts, out, aux, grads, train, backward,
                         k=6):
    """Routing bit-exact, outputs and gradients to the dtype's bar, against the oracle run
    on the GPU's own logits (the router GEMM's values, offset included)."""
    dt = x.dtype
    E = p.W_in.shape[0]
    ref = R.block(x, p, k, train=train, grad_out=g if backward else None, fp32=True,
                  logits=logits)
    assert torch.equal(idx, ref.topk_idx), "routing indices differ"
    assert torch.equal(counts.long(), ref.counts), "counts differ"
    sids, _, offs, dcounts, _, inv = mk.moe_dispatch(idx.to(DEV), E)
    r_sids, _, r_offs, r_counts, _, r_inv = R.dispatch_buffers(ref.topk_idx, E, mk.ALIGN_M)
    assert torch.equal(sids.cpu(), r_sids) and torch.equal(inv.cpu(), r_inv)
    assert torch.equal(offs.cpu(), r_offs) and torch.equal(dcounts.cpu(), r_counts)
    close("out", out, ref.out, dt)
    if train:
        torch.testing.assert_close(aux.float().cpu().reshape(()), ref.aux_loss.float().reshape(()),
                                   rtol=1e-5, atol=1e-7)
    else:
        assert float(aux) == 0.0
    if not backward:
        return ref
    gr = ref.grads
    d_logits = gr["logits"]
    close("dx", grads["x"], gr["x"] + d_logits @ p.W.float().t(), dt)
    close("d router.W", grads["W"], x.float().t() @ d_logits, dt)
    for name in grads:
        if name not in ("x", "W"):
            close(f"d {name}", grads[name], gr[name], dt)
    return ref


def run_case(T, train, backward, *, logit_bias=None, collect=None, **cfg):
    """The drop-in MoEBlock, as a caller runs it (one op per direction on the GPU).  The
    GPU's output and gradients also go into `collect` when a dict is given."""
    m, p, x, g = build(T, **cfg)
    dt = x.dtype
    m = m.to(DEV).train(train)
    xg = x.to(DEV).requires_grad_(backward)
    print(f"[block] T={T} train={train} backward={backward} cfg={cfg} "
          f"skewed={logit_bias is not None}", flush=True)
    if logit_bias is None:
        out = m(xg)
        aux = m.aux_loss
        idx, counts, kl = m._routing, m.expert_counts, m._logits
        assert m._use_kernel(xg.reshape(-1, x.shape[1])), "the HIP path was not taken"
    else:
        # The reference router has no bias: the offset goes in through the op's hook.
        out, aux, counts, idx, kl = mk.block_forward(
            xg, m.router.W, m.W_in, m.W_out, m.W_sh_in, m.W_sh_out, m.b_in, m.b_out,
            m.b_sh_in, m.b_sh_out, m.top_k, m.router.wants_probs(),
            m.router.normalize_weights, "silu", m.router.aux_loss_coef,
            logit_bias=logit_bias.to(DEV))
    if backward:
        torch.autograd.backward([out, aux], [g.to(DEV), torch.ones_like(aux)])
    torch.cuda.synchronize()
    # The oracle routes the block's own router GEMM output (the values its routing ran
    # on); that output is checked against an fp32 GEMM of the same operands.
    logits = kl.float().cpu()
    check_router_gemm(x, p.W, logits, logit_bias, dt)
    grads = {}
    if backward:
        grads = {"x": xg.grad.cpu(), "W": m.router.W.grad.cpu()}
        for n in ("W_in", "W_out", "W_sh_in", "W_sh_out", "b_in", "b_out", "b_sh_in",
                  "b_sh_out"):
            t = getattr(m, n)
            if t is not None:
                grads[n] = t.grad.cpu()
    if collect is not None:
        collect.update(grads, out=out.detach().cpu())
    return check_against_oracle(x, p, g, logits, idx.cpu(), counts.cpu(),
                                out.detach().cpu(), aux.detach().cpu(), grads, train,
                                backward, k=m.top_k)


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


def test_skewed_T16384_forward_backward_block_path():
    """Config 4 through the block path itself: the fused router backward (combine_dx with
    d(logits) W^T, router_dw's split-K), the in-launch balance loss and the dW split-K
    under a hot expert holding ~15 % of the pairs."""
    bias = torch.from_numpy(np.load(ZIPF, allow_pickle=False)).float()
    ref = run_case(16384, train=True, backward=True, logit_bias=bias)
    share = ref.counts.double() / ref.counts.sum()
    assert 0.12 < float(share.max()) < 1 / 6 + 1e-9   # the hot expert holds ~15 %


def test_skewed_T8192_forward_backward_block_path():
    """The headline shape under the Zipf offset: T k = 49,152 pairs sit below E x 691, so
    the dW split-K reduce inside combine_dx's launch takes the routed groups in its one
    looping row, and with ~15 % of the pairs on the hot expert several routed groups span
    more than one 768-row chunk and are reduced there one after another."""
    bias = torch.from_numpy(np.load(ZIPF, allow_pickle=False)).float()
    ref = run_case(8192, train=True, backward=True, logit_bias=bias)
    assert int((ref.counts > 768).sum()) >= 2


def test_prefill_layer_T32768_eval():
    """One MoE call of the 20-layer prefill (batch 4 x 8192): T = 32768, 196,608 pairs,
    about 262 k grouped-GEMM rows and 302 MB of expert output rows."""
    ref = run_case(32768, train=False, backward=False)
    assert int(ref.counts.sum()) == 32768 * 6


@pytest.mark.parametrize("T", [300, 1024])
def test_glu_backward_96_row_tiles_forced(T):
    """The GLU backward's 96-row tiles (taken by default only once 64-row tiles overflow
    three workgroups per CU, T = 8192 here) forced at small T: their epilogue stages the
    tile in two passes of 48 rows, and the ragged last tiles of the groups leave the
    second pass partly or wholly empty.  Checked against the oracle through dx and every
    gradient, with the forward's saved pre-activations (the block's default)."""
    from tests.helpers import lib_options

    assert mk.SAVE_ACT
    with lib_options(bwd_rows=96):
        run_case(T, train=True, backward=True)


def test_zero_router_sends_every_token_to_the_same_experts():
    ref = run_case(2048, train=True, backward=True, zero_router=True)
    assert int((ref.counts > 0).sum()) == 6 and int(ref.counts.max()) == 2048


@pytest.mark.parametrize("cfg", [dict(S=2), dict(S=0, bias=True, dtype=torch.float16),
                                 dict(d=128, E=12, d_ff=96, k=4, S=1)])
def test_saved_pre_activations_and_recompute_agree(monkeypatch, cfg):
    """The default backward reads the forward's saved pre-activations x W_in + b_in
    (rounded to the block's dtype, as the reference's backward rounds its recomputed
    ones); the alternative recomputes them in fp32.  Both meet the bar against the oracle
    and agree with each other to the same bar; the saved ones make `saved` larger."""
    runs = {}
    for save in (True, False):
        monkeypatch.setattr(mk, "SAVE_ACT", save)
        runs[save] = {}
        run_case(1024, train=True, backward=True, collect=runs[save], **cfg)
    dt = cfg.get("dtype", torch.bfloat16)
    for name, ref in runs[False].items():
        close(f"saved vs recomputed: {name}", runs[True][name], ref.float(), dt)
    d, h = cfg.get("d", 576), cfg.get("d_ff", 192) * 2 // 3
    assert mk.save_act_supported(dt, d, h)
    e, k, S = cfg.get("E", 76), cfg.get("k", 6), cfg.get("S", 2)
    assert (mk.block_saved_bytes(1024, e, k, dt, True, True, d, h, S)
            > mk.block_saved_bytes(1024, e, k, dt, True, False, d, h, S))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("S", [0, 2])
def test_block_dtype_bias_shared_matrix(dtype, bias, S):
    """The block node at nanoSpeaker's shape in every dtype it takes, with and without
    biases and shared experts (fp32 finishes the router GEMM's backward in torch)."""
    run_case(300, train=True, backward=True, dtype=dtype, bias=bias, S=S)


@pytest.mark.parametrize("cfg", [
    dict(d=72, E=10, d_ff=96, k=3, S=1),    # d % 16 != 0, E % 4 != 0: router bwd in torch
    dict(d=64, E=16, d_ff=96, k=10, S=2),   # k > 8: the general dx combine
    dict(d=64, E=8, d_ff=96, k=2, S=3),     # more than two shared experts
    dict(d=128, E=12, d_ff=192, k=4, S=0, bias=True),
    dict(d=96, E=12, d_ff=96, k=3, S=1),    # d % 64 != 0: combine_dx's last column tile
    dict(d=80, E=8, d_ff=96, k=2, S=1),     # ragged in halves; d % 32 != 0: router fwd in torch
])
@pytest.mark.parametrize("train", [True, False])
def test_block_other_shapes(cfg, train):
    run_case(257, train=train, backward=True, **cfg)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_eval_loss_is_a_zero_the_library_writes(dtype):
    """In eval the block's loss is a zero of its dtype (moe.py's eval branch); the library's
    dispatch launch writes it into memory the op leaves uninitialised.  Each call below
    takes its small buffers from blocks just freed from NaN-filled tensors of the same
    size class, so a zero that was not written would show."""
    m, _, x, _ = build(256, dtype=dtype)
    m = m.to(DEV).eval()
    x = x.to(DEV)
    with torch.no_grad():
        for _ in range(3):
            junk = [torch.full((128,), float("nan"), device=DEV) for _ in range(16)]
            del junk
            m(x)
            aux = m.aux_loss
            assert aux.dtype == dtype and aux.shape == ()
            assert float(aux) == 0.0 and not math.copysign(1.0, float(aux)) < 0


@pytest.mark.parametrize("cfg", [dict(), dict(dtype=torch.float16), dict(S=0, bias=True)])
def test_weight_pack_in_the_router_launch_matches_the_place_launch(cfg):
    """In training at T = 8192 the expert-weight pack runs inside the router's launch (the
    last 4 waves of each 16-wave workgroup, beside the selection and the exact pass); the
    "pack_in_place" option moves it back into the dispatch's place launch.  Every output
    and gradient agrees bit for bit (bf16, fp16, and without shared experts), and the
    library's launch timers show where the pack ran.  (test_forward_backward_T8192_train
    checks the default against the oracle.)"""
    from nanospeaker_amd import _native as nat
    from tests.helpers import lib_options

    m, _, x, g = build(8192, **cfg)
    m = m.to(DEV).train()
    xd, gd = x.to(DEV), g.to(DEV)
    params = list(m.parameters())

    def step(**opts):
        with lib_options(**opts):
            nat.timing_enable(256)
            try:
                mk.PACKS.clear()
                xr = xd.detach().requires_grad_(True)
                out = m(xr)
                gs = torch.autograd.grad([out, m.aux_loss], [xr] + params,
                                         [gd, torch.ones_like(m.aux_loss)])
                torch.cuda.synchronize()
                launches = (nat.timing_read("place_pack")[1], nat.timing_read("dispatch")[1])
            finally:
                nat.timing_enable(0)
        return [out.detach().cpu()] + [t.cpu() for t in gs], launches

    in_router, n_router = step()
    in_place, n_place = step(pack_in_place=1)
    assert n_router == (0, 1) and n_place == (1, 0), (n_router, n_place)
    for i, (a, b) in enumerate(zip(in_router, in_place)):
        assert torch.equal(a, b), i
