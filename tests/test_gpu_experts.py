"""
GPU parity of the grouped experts (forward and backward) against the CPU oracle.

Routing is fixed on the CPU (oracle router on CPU logits) and handed to both sides, so
the comparison isolates the expert math.  fp32 kernels are held to 1e-5 (the reference's
own kernel-vs-eager tolerance, test_moe_kernel.py:101-130); bf16/fp16 to the north-star
bar against the fp32-accumulated reference: max abs err <= 2e-2, rel-L2 <= 5e-3.
"""

import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import F32_ATOL, assert_close_bf16, lib_options

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")

DEV = "cuda"
GRAD_NAMES = ("W_in", "W_out", "W_sh_in", "W_sh_out", "b_in", "b_out", "b_sh_in", "b_sh_out")


def make_case(d, E, d_ff, k, S, bias, T, dtype, seed=0, train=True):
    p = R.make_params(seed, d, E, d_ff, n_shared=S, bias=bias)
    if bias:
        g = torch.Generator().manual_seed(seed + 7)
        for n in ("b_in", "b_out", "b_sh_in", "b_sh_out"):
            t = getattr(p, n)
            if t is not None:
                setattr(p, n, torch.randn(t.shape, generator=g) * 0.1)
    p = p.to(dtype=dtype)
    x = torch.randn(T, d).to(dtype)
    gout = torch.randn(T, d).to(dtype)
    logits = R.router_logits(x, p.W)
    topk_w, topk_idx, _ = R.route_from_logits(logits, k, train, True, dtype)
    return p, x, gout, topk_w, topk_idx


def oracle_fwd_bwd(p, x, gout, topk_w, topk_idx, act, with_grad=True):
    """fp32 eager forward with routing fixed; grads of (out * gout).sum()."""
    leaves = {"x": x.float().clone().requires_grad_(with_grad),
              "topk_w": topk_w.float().clone().requires_grad_(with_grad)}
    named = {k: v.float().clone().requires_grad_(with_grad) for k, v in p.named().items()
             if k != "W"}
    pl = R.Params(**{f: named.get(f) for f in R.Params.__dataclass_fields__})
    out = R.eager_forward(leaves["x"], pl, leaves["topk_w"], topk_idx, act)
    grads = {}
    if with_grad:
        (out * gout.float()).sum().backward()
        grads = {k: v.grad for k, v in {**leaves, **named}.items()}
    return out.detach(), grads


def gpu_fwd_bwd(p, x, gout, topk_w, topk_idx, act, with_grad=True):
    dev = lambda t: None if t is None else t.to(DEV).clone().requires_grad_(with_grad)
    xg, twg = dev(x), dev(topk_w)
    P = {n: dev(getattr(p, n)) for n in ("W_in", "W_out") + GRAD_NAMES[2:]}
    sids, eids, offs, counts, npp, inv = mk.moe_dispatch(topk_idx.to(DEV), p.W_in.shape[0])
    out, _ = mk.moe_block(xg, P["W_in"], P["W_out"], P["W_sh_in"], P["W_sh_out"], P["b_in"],
                          P["b_out"], P["b_sh_in"], P["b_sh_out"], twg, sids, offs, counts, inv,
                          act)
    grads = {}
    if with_grad:
        (out.float() * gout.to(DEV).float()).sum().backward()
        grads = {"x": xg.grad, "topk_w": twg.grad}
        grads.update({n: t.grad for n, t in P.items() if t is not None})
    return out.detach().cpu(), {k: v.cpu() for k, v in grads.items()}


def check(name, got, ref, dtype):
    if dtype == torch.float32:
        torch.testing.assert_close(got.float(), ref.float(), atol=F32_ATOL, rtol=1e-4,
                                   msg=lambda m: f"{name}: {m}")
    else:
        assert_close_bf16(name, got.float(), ref.float())


SHAPES = {  # d, E, d_ff (H = 2 * d_ff // 3)
    "tiny_h42": (32, 8, 64),
    "mid_h64": (64, 8, 96),
    "wide_h64": (256, 8, 96),    # one 64-column hidden block per wave; last pass 64 wide
    "wide_h96": (256, 8, 144),   # hidden blocks past H inside the 128-wide tile
    "ns_h128": (576, 76, 192),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("k,S,bias", [(2, 0, False), (1, 1, True), (6, 2, False)])
@pytest.mark.parametrize("T", [1, 37, 300])
def test_experts_forward_backward(dtype, shape, k, S, bias, T):
    d, E, d_ff = SHAPES[shape]
    if k > E:
        pytest.skip("top_k > E")
    p, x, gout, tw, ti = make_case(d, E, d_ff, k, S, bias, T, dtype, seed=T + k)
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, "silu")
    out, g = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    check("out", out, ref_out, dtype)
    for n in ref_g:
        check(f"grad {n}", g[n], ref_g[n], dtype)


@pytest.mark.parametrize("dist", ["2", "3", "6"])
@pytest.mark.parametrize("mb", ["2", "4", "6"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", ["wide_h64", "wide_h96", "ns_h128"])
@pytest.mark.parametrize("T", [37, 300, 1000])
def test_forward_tile_heights(dist, mb, dtype, shape, T):
    """Every forward tile height (32-, 64- and 96-row tiles, forced) and weight prefetch
    distance (2, 3 and, for 32-row tiles, 6 steps; each only where the step counts
    divide, else the library's own) against the oracle, with ragged last tiles and the
    shared experts' full-T groups."""
    if dist == "6" and mb != "2":
        pytest.skip("distance 6 is for 32-row tiles")
    d, E, d_ff = SHAPES[shape]
    p, x, gout, tw, ti = make_case(d, E, d_ff, 6, 2, T % 2 == 0, T, dtype, seed=T + int(mb))
    ref_out, _ = oracle_fwd_bwd(p, x, gout, tw, ti, "silu", with_grad=False)
    with lib_options(fwd_rows=16 * int(mb), fwd_dist=int(dist)):
        out, _ = gpu_fwd_bwd(p, x, gout, tw, ti, "silu", with_grad=False)
    check("out", out, ref_out, dtype)


@pytest.mark.parametrize("mb,dist,bwd_dist,bwd_mb",
                         [("4", "2", "2", "4"), ("6", "2", "3", "4"), ("4", "4", "3", "3"),
                          ("6", "3", "2", "3"), ("4", "2", "2", "5")])
@pytest.mark.parametrize("shape", ["wide_h64", "ns_h128"])
@pytest.mark.parametrize("T", [37, 1000])
def test_backward_tile_heights_and_prefetch(mb, dist, bwd_dist, bwd_mb, shape, T):
    """The dX-row kernel at both tile heights and several weight prefetch distances, and
    the GLU-backward kernel at 48-, 64- and 80-row tiles and both of its prefetch distances
    (all forced), checked through dx and every weight gradient."""
    d, E, d_ff = SHAPES[shape]
    p, x, gout, tw, ti = make_case(d, E, d_ff, 6, 2, T % 2 == 1, T, torch.bfloat16,
                                   seed=T + int(mb))
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, "silu")
    with lib_options(dx_rows=16 * int(mb), dx_dist=int(dist), bwd_dist=int(bwd_dist),
                     bwd_rows=16 * int(bwd_mb)):
        out, g = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    check("out", out, ref_out, torch.bfloat16)
    for n in ref_g:
        check(f"grad {n}", g[n], ref_g[n], torch.bfloat16)


def test_dw_reduce_skewed_routing():
    """Routed experts average far fewer rows than a dW chunk (768), so the dW reduce takes
    them in its one looping row; experts 0, 1 and 2 still get 900+ rows (two chunks each)
    and are summed there one after another, beside the shared experts.  Three groups in
    turn exercise the reduce's reuse of its shared base between groups."""
    d, E, d_ff = SHAPES["ns_h128"]
    T = 2000
    p, x, gout, tw, _ = make_case(d, E, d_ff, 2, 2, False, T, torch.bfloat16, seed=11)
    t = torch.arange(T)
    first = torch.where(t < 900, torch.zeros_like(t),
                        torch.where(t < 1800, torch.ones_like(t), 3 + t % (E - 3)))
    second = torch.where(t < 900, torch.full_like(t, 2), 3 + (t * 7 + 3) % (E - 3))
    second = torch.where(second == first, 3 + (second - 2) % (E - 3), second)
    ti = torch.stack([first, second], 1).to(torch.int64)
    counts = torch.bincount(ti.flatten(), minlength=E)
    assert (ti[:, 0] != ti[:, 1]).all()
    assert (counts[:3] > 768).all() and (counts[3:] <= 768).all()
    assert T * 2 < E * 691  # the reduce's single looping row for routed groups
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, "silu")
    out, g = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    check("out", out, ref_out, torch.bfloat16)
    for n in ref_g:
        check(f"grad {n}", g[n], ref_g[n], torch.bfloat16)


@pytest.mark.parametrize("act", ["silu", "gelu", "relu", "sigmoid", "tanh"])
@pytest.mark.parametrize("shape", ["tiny_h42", "ns_h128"])
def test_every_activation(act, shape):
    d, E, d_ff = SHAPES[shape]
    dtype = torch.float32 if shape == "tiny_h42" else torch.bfloat16
    p, x, gout, tw, ti = make_case(d, E, d_ff, 2, 1, True, 90, dtype, seed=3)
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, act)
    out, g = gpu_fwd_bwd(p, x, gout, tw, ti, act)
    check("out", out, ref_out, dtype)
    for n in ref_g:
        check(f"grad {n}", g[n], ref_g[n], dtype)


def test_reference_schema_equals_block_op_without_shared():
    """moe_experts (reference schema) and moe_block (S = 0) share kernels: same bits."""
    d, E, d_ff = SHAPES["ns_h128"]
    p, x, gout, tw, ti = make_case(d, E, d_ff, 6, 0, False, 257, torch.bfloat16, seed=5)
    out1, g1 = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    xg = x.to(DEV).requires_grad_(True)
    W_in = p.W_in.to(DEV).requires_grad_(True)
    W_out = p.W_out.to(DEV).requires_grad_(True)
    twg = tw.to(DEV).requires_grad_(True)
    sids, eids, offs, counts, npp, inv = mk.moe_dispatch(ti.to(DEV), E)
    out2 = mk.moe_experts(xg, W_in, W_out, twg, None, None, sids, eids, offs, counts, npp, inv,
                          "silu")
    (out2.float() * gout.to(DEV).float()).sum().backward()
    assert torch.equal(out1, out2.detach().cpu())
    for n, t in (("x", xg), ("W_in", W_in), ("W_out", W_out), ("topk_w", twg)):
        assert torch.equal(g1[n], t.grad.cpu()), n


def test_collapsed_routing_ragged_tail():
    """Everything on one expert (empty runs elsewhere, one long ragged run); zero dW elsewhere."""
    d, E, d_ff = SHAPES["ns_h128"]
    p, x, gout, _, _ = make_case(d, E, d_ff, 1, 0, False, 3000, torch.bfloat16, seed=9)
    ti = torch.zeros(3000, 1, dtype=torch.long)
    tw = torch.ones(3000, 1, dtype=torch.bfloat16)
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, "silu")
    out, g = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    check("out", out, ref_out, torch.bfloat16)
    for n in ("x", "W_in", "W_out", "topk_w"):
        check(f"grad {n}", g[n], ref_g[n], torch.bfloat16)
    assert float(g["W_in"][1:].abs().sum()) == 0.0 and float(g["W_out"][1:].abs().sum()) == 0.0


def test_reference_schema_ops():
    """fused_moe_forward / moe_experts / moe_experts_bwd keep the reference contract."""
    d, E, d_ff = SHAPES["mid_h64"]
    p, x, gout, tw, ti = make_case(d, E, d_ff, 2, 0, True, 111, torch.float32, seed=4)
    ref_out, ref_g = oracle_fwd_bwd(p, x, gout, tw, ti, "silu")
    xg = x.to(DEV).requires_grad_(True)
    W_in = p.W_in.to(DEV).requires_grad_(True)
    W_out = p.W_out.to(DEV).requires_grad_(True)
    b_in = p.b_in.to(DEV).requires_grad_(True)
    b_out = p.b_out.to(DEV).requires_grad_(True)
    twg = tw.to(DEV).requires_grad_(True)
    out, counts = mk.fused_moe_forward(xg, W_in, W_out, twg, ti.to(DEV), b_in, b_out, "silu")
    assert counts.dtype == torch.int32
    assert torch.equal(counts.cpu().long(), torch.bincount(ti.reshape(-1), minlength=E))
    (out * gout.to(DEV)).sum().backward()
    check("out", out.detach().cpu(), ref_out, torch.float32)
    for n, t in (("x", xg), ("W_in", W_in), ("W_out", W_out), ("b_in", b_in),
                 ("b_out", b_out), ("topk_w", twg)):
        check(f"grad {n}", t.grad.cpu(), ref_g[n], torch.float32)


def test_forward_is_deterministic():
    d, E, d_ff = SHAPES["ns_h128"]
    p, x, gout, tw, ti = make_case(d, E, d_ff, 6, 2, False, 2048, torch.bfloat16, seed=1)
    a, ga = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    b, gb = gpu_fwd_bwd(p, x, gout, tw, ti, "silu")
    assert torch.equal(a, b)
    for n in ga:
        assert torch.equal(ga[n], gb[n]), n
