"""
The fused router (router.hip: x W_r, softmax, top-k, gates, histograms, tie pass) through
the block op, against the oracle fed the kernel's own logits: routing indices, counts and
every dispatch buffer bit-exact, gates and probs-derived balance loss within tolerance.

Inputs stress what the selection must get right: router weights with duplicated columns
(every token's experts tie in pairs, so every token goes through the exact pass), all-zero
tokens (all experts tie), NaN tokens, -inf offsets, and token counts around the
64-token workgroup boundary; E from 4 to 128, top_k from 1 to 16, both router branches
with and without renormalisation.
"""

import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")

DEV = "cuda"


def run(T, E, k, train, normalize, dtype=torch.bfloat16, d=64, mode="rand", bias=None, seed=0,
        with_logits=False):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(d, E, generator=g) * 0.3).to(dtype)
    if mode == "pairs":
        W[:, 1::2] = W[:, 0::2]
    x = torch.randn(T, d, generator=g).to(dtype)
    if mode == "zeros":
        x[::3] = 0
    if mode == "nan":
        x[::5, 3] = float("nan")
    H = 32
    w_in = (torch.randn(E, d, 2 * H, generator=g) * 0.05).to(dtype).to(DEV)
    w_out = (torch.randn(E, H, d, generator=g) * 0.05).to(dtype).to(DEV)
    print(f"[router] T={T} E={E} k={k} train={train} normalize={normalize} mode={mode}",
          flush=True)
    with torch.no_grad():
        out, aux, counts, idx, logits = mk.block_forward(
            x.to(DEV), W.to(DEV), w_in, w_out, None, None, None, None, None, None, k, train,
            normalize, "silu", 1e-2, logit_bias=None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    lg = logits.float().cpu()
    ref_w, ref_idx, ref_probs = R.route_from_logits(lg, k, train, normalize, dtype)
    assert torch.equal(idx.cpu(), ref_idx), "routing indices differ"
    gw = _gates(x, W, w_in, w_out, k, train, normalize, bias).float().cpu()
    ok = ~torch.isnan(ref_w.float()).any(1)  # NaN tokens: NaN gates on both sides
    assert torch.isnan(gw[~ok]).all(1).all() if (~ok).any() else True
    assert_close_bf16("gates", gw[ok], ref_w.float()[ok])
    _, _, _, rc = R.plan(ref_idx, E)
    assert torch.equal(counts.cpu().long(), rc)
    sids, eids, offs, dc, npp, inv = mk.moe_dispatch(idx, E)
    r = R.dispatch_buffers(ref_idx, E, mk.ALIGN_M)
    for name, a_, b_ in zip(("sorted_ids", "expert_ids", "pad_offsets", "counts", "n_post_pad",
                             "inv"), (sids, eids, offs, dc, npp, inv), r):
        assert torch.equal(a_.cpu(), torch.as_tensor(b_, dtype=a_.dtype).reshape(a_.shape)), name
    if train and not torch.isnan(ref_probs).any():
        ref_aux = R.balance_loss(ref_probs, rc, 1e-2, E)
        torch.testing.assert_close(aux.float().cpu(), ref_aux.float(), rtol=1e-5, atol=1e-7)
    return (ref_idx, logits.cpu()) if with_logits else ref_idx


def _gates(x, W, w_in, w_out, k, train, normalize, bias):
    """The block's gate weights, read back through the op's saved gates."""
    with torch.no_grad():
        res = mk.block_fwd(x.to(DEV), W.to(DEV), w_in, w_out, None, None, None, None, None,
                           None, k, train, normalize, "silu", 1e-2,
                           None if bias is None else bias.to(DEV))
    saved = res[5]
    T = x.shape[0]
    return saved[: T * k * 2].view(torch.bfloat16 if x.dtype == torch.bfloat16
                                   else torch.float16).view(T, k)


@pytest.mark.parametrize("mode", ["rand", "pairs", "zeros", "nan"])
@pytest.mark.parametrize("train,normalize", [(True, True), (False, True), (False, False),
                                             (True, False)])
def test_fused_router_ties_and_branches(mode, train, normalize):
    run(300, 76, 6, train, normalize, mode=mode, seed=len(mode))


@pytest.mark.parametrize("T", [1, 63, 64, 65, 1000])
@pytest.mark.parametrize("E,k", [(4, 1), (8, 2), (76, 6), (80, 16), (128, 16), (64, 8), (12, 12)])
def test_fused_router_shapes(T, E, k):
    run(T, E, k, True, True, mode="pairs" if T % 2 else "rand", seed=T + E)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_router_dtypes_and_width(dtype):
    run(777, 76, 6, True, True, dtype=dtype, d=576, seed=3)
    run(777, 76, 6, False, True, dtype=dtype, d=576, mode="pairs", seed=4)


def test_fused_router_offsets_including_minus_inf():
    bias = torch.zeros(76)
    bias[::7] = float("-inf")
    bias[3] = 2.0
    idx = run(500, 76, 6, True, True, bias=bias, seed=5)
    assert not torch.isin(idx, torch.arange(0, 76, 7)).any()


@pytest.mark.parametrize("T,E,k,d,mode,dtype", [
    (300, 76, 6, 576, "pairs", torch.bfloat16), (1000, 76, 6, 224, "rand", torch.bfloat16),
    (65, 80, 16, 576, "zeros", torch.bfloat16), (777, 12, 12, 160, "nan", torch.bfloat16),
    (40, 76, 6, 64, "pairs", torch.bfloat16), (513, 76, 6, 576, "rand", torch.float16)])
def test_fused_router_both_workgroup_shapes(T, E, k, d, mode, dtype):
    """Both workgroup shapes of the router kernel, forced: 16 waves with W_r whole in LDS,
    and 8 waves (two workgroups per CU, the default past one workgroup per CU) with W_r
    in parts of 6 k-steps double-buffered through LDS -- d = 576 takes three parts, 224
    two (the second partial), 160 and 64 one.  Each shape's routing is bit-exact against
    the oracle on its own logits, and the two shapes' logits are bit-identical (every
    logit is the same MFMA chain over the same k-steps in the same order)."""
    from tests.helpers import lib_options

    got = {}
    for waves in (16, 8):
        with lib_options(router_waves=waves):
            for train in (True, False):
                got[waves, train] = run(T, E, k, train, True, dtype=dtype, d=d, mode=mode,
                                        seed=T + d, with_logits=True)
    for train in (True, False):
        (i16, l16), (i8, l8) = got[16, train], got[8, train]
        assert torch.equal(l8.view(torch.int16), l16.view(torch.int16)), "logits differ"
        assert torch.equal(i8, i16)
