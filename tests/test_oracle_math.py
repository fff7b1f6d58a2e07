"""
Pins the oracle by mathematics, independently of the golden fixtures: each check below
would fail on a plausible mistake (a dropped term, a wrong index, a transposed operand).

  * dense_forward (every expert on every token, einsum mix; moe.py:459-474) equals the
    ragged eager loop in fp64 -- two different formulas for the same sum;
  * the dispatch buffers equal a counting sort done with numpy's stable argsort;
  * gradients of the fp64 block equal finite differences (torch.autograd.gradcheck);
  * router closed forms: gates sum to 1, train and eval branches agree, the balance loss
    KATs of the reference suite (test_moe.py:56-88).
"""

import numpy as np
import pytest
import torch

from oracle import moe_ref as R

ALIGN = 16


def _case(seed, d=32, E=8, d_ff=64, k=2, S=0, bias=False, T=51, dtype=torch.float64):
    p = R.make_params(seed, d, E, d_ff, n_shared=S, bias=bias)
    if bias:
        g = torch.Generator().manual_seed(seed)
        for n in ("b_in", "b_out", "b_sh_in", "b_sh_out"):
            t = getattr(p, n)
            if t is not None:
                setattr(p, n, torch.randn(t.shape, generator=g) * 0.1)
    p = p.to(dtype=dtype)
    x = torch.randn(T, d, dtype=dtype)
    tw, ti, _ = R.route_from_logits(R.router_logits(x, p.W), k, True, True, dtype)
    return p, x, tw, ti


@pytest.mark.parametrize("k", [1, 2, 8])
@pytest.mark.parametrize("S,bias", [(0, False), (2, True)])
@pytest.mark.parametrize("act", ["silu", "gelu", "relu", "sigmoid", "tanh"])
def test_eager_equals_dense_in_fp64(k, S, bias, act):
    p, x, tw, ti = _case(k + S, k=k, S=S, bias=bias)
    a = R.eager_forward(x, p, tw, ti, act)
    b = R.dense_forward(x, p, tw, ti, act)
    assert torch.allclose(a, b, atol=1e-12)


def test_one_expert_is_a_plain_glu():
    """test_moe.py:220-228: a 1-expert top-1 MoE is the GLU FFN."""
    p, x, _, _ = _case(3, E=1, k=1)
    ti = torch.zeros(x.shape[0], 1, dtype=torch.long)
    tw = torch.ones(x.shape[0], 1, dtype=x.dtype)
    gate, up = (x @ p.W_in[0]).chunk(2, dim=-1)
    want = (torch.nn.functional.silu(gate) * up) @ p.W_out[0]
    assert torch.allclose(R.eager_forward(x, p, tw, ti), want, atol=1e-12)


def test_shared_expert_is_a_plain_glu_over_every_token():
    """test_moe.py:243-252."""
    p, x, tw, ti = _case(4, S=1)
    p.W_out = torch.zeros_like(p.W_out)
    gate, up = (x @ p.W_sh_in[0]).chunk(2, dim=-1)
    want = (torch.nn.functional.silu(gate) * up) @ p.W_sh_out[0]
    assert torch.allclose(R.eager_forward(x, p, tw, ti), want, atol=1e-12)


def _numpy_dispatch(flat: np.ndarray, E: int):
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    padded = -(-counts // ALIGN) * ALIGN
    offs = np.concatenate([[0], np.cumsum(padded)])
    return order, counts, offs


@pytest.mark.parametrize("T,E,k", [(1, 8, 1), (50, 8, 2), (64, 76, 6), (2000, 76, 6),
                                   (100, 1000, 3), (16, 8, 8)])
def test_dispatch_buffers_equal_a_numpy_counting_sort(T, E, k):
    g = torch.Generator().manual_seed(T)
    ti = torch.rand(T, E, generator=g).topk(k, dim=-1).indices
    sids, eids, offs, counts, npp, inv = R.dispatch_buffers(ti, E, ALIGN)
    flat = ti.reshape(-1).numpy()
    order, c_np, o_np = _numpy_dispatch(flat, E)
    M = flat.size
    assert np.array_equal(counts.numpy(), c_np)
    assert np.array_equal(offs.numpy(), o_np)
    assert npp == o_np[-1]
    start = np.concatenate([[0], np.cumsum(c_np)])
    for e in range(E):
        run = sids[o_np[e]: o_np[e] + c_np[e]].numpy()
        assert np.array_equal(run, order[start[e]: start[e + 1]])
        assert (sids[o_np[e] + c_np[e]: o_np[e + 1]].numpy() == M).all()
    assert np.array_equal(sids.numpy()[inv.numpy()], np.arange(M))
    for b in range(npp // ALIGN):      # block owner: the run containing slot b * ALIGN
        e = int(eids[b])
        assert o_np[e] <= b * ALIGN < o_np[e + 1]


def test_plan_on_a_tiny_case_by_hand():
    ti = torch.tensor([[2, 0], [0, 1], [2, 1]])
    experts, order, token, counts = R.plan(ti, 3)
    assert order.tolist() == [1, 2, 3, 5, 0, 4]
    assert token.tolist() == [0, 1, 1, 2, 0, 2]
    assert counts.tolist() == [2, 2, 2]


@pytest.mark.parametrize("train", [True, False])
def test_block_gradients_match_finite_differences(train):
    """gradcheck of the whole fp64 block with routing held fixed (tiny shape)."""
    p, x, tw, ti = _case(5, d=8, E=4, d_ff=12, k=2, S=1, bias=True, T=6)

    def f(x_, w_in, w_out, w_sh_in, tw_):
        q = R.Params(p.W, w_in, w_out, w_sh_in, p.W_sh_out, p.b_in, p.b_out, p.b_sh_in,
                     p.b_sh_out)
        return R.eager_forward(x_, q, tw_, ti, "silu")

    args = [t.clone().requires_grad_(True) for t in (x, p.W_in, p.W_out, p.W_sh_in, tw)]
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-8)


def test_router_gradient_matches_finite_differences():
    logits = torch.randn(5, 8, dtype=torch.float64)
    for want_probs, normalize in ((True, True), (True, False), (False, True), (False, False)):
        f = lambda l: R.route_from_logits(l, 3, want_probs, normalize, torch.float64)[0]
        assert torch.autograd.gradcheck(f, [logits.clone().requires_grad_(True)])


def test_router_gate_sums_and_branch_agreement():
    """test_moe.py:56-66 and 422-439."""
    logits = torch.randn(64, 8, dtype=torch.float64)
    w_tr, i_tr, probs = R.route_from_logits(logits, 3, True, True, torch.float64)
    w_ev, i_ev, none = R.route_from_logits(logits, 3, False, True, torch.float64)
    assert none is None and torch.equal(i_tr, i_ev)
    assert torch.allclose(w_tr.sum(-1), torch.ones(64, dtype=torch.float64))
    assert torch.allclose(w_tr, w_ev, atol=1e-12)
    w_un, i_un, p_un = R.route_from_logits(logits, 3, True, False, torch.float64)
    assert torch.allclose(w_un, p_un.gather(1, i_un))


def test_balance_loss_kats():
    """test_moe.py:69-88."""
    uniform = R.balance_loss(torch.full((16, 4), 0.25), torch.tensor([4, 4, 4, 4]), 1e-2, 4)
    collapsed = R.balance_loss(torch.tensor([[0.7, 0.1, 0.1, 0.1]]).expand(16, 4),
                               torch.tensor([16, 0, 0, 0]), 1e-2, 4)
    assert collapsed > uniform
    probs = torch.full((16, 4), 0.25)
    a = R.balance_loss(probs, torch.tensor([4, 4, 4, 4]), 1e-2, 4)
    b = R.balance_loss(probs, torch.tensor([16, 0, 0, 0]), 1e-2, 4)
    assert float(a) == pytest.approx(float(b))
    assert float(a) == pytest.approx(1e-2)   # coef * E * sum_e (1/4)(1/4) = coef


def test_flops_per_token_matches_the_survey():
    """3,626,496 forward FLOPs per token at nanoSpeaker's shape: 8 pairs x (2*d*2H + 2*H*d) + 2*d*E."""
    c = R.nanospeaker_config()
    assert R.flops_per_token(c["d"], 128, c["top_k"], c["n_shared"], c["E"]) == 3_626_496


# ---- the RMSNorm in front of the block (ln.py:30-36) ------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,d", [(257, 576), (64, 64), (33, 1024)])
def test_rms_norm_equals_torch_rms_norm(dtype, T, d):
    """The oracle's written-out norm is torch's F.rms_norm (a library routine) bit for bit
    on the CPU: same fp32 rstd, same (x rstd) w order, one rounding."""
    g = torch.Generator().manual_seed(T + d)
    x = (torch.randn(T, d, generator=g) * 3).to(dtype)
    w = (1 + 0.2 * torch.randn(d, generator=g)).to(dtype)
    xn, rstd = R.rms_norm(x, w, 1e-6)
    assert torch.equal(xn, torch.nn.functional.rms_norm(x, (d,), w, 1e-6))
    ref = torch.rsqrt(x.double().pow(2).mean(-1) + 1e-6)
    torch.testing.assert_close(rstd.double(), ref, rtol=1e-6, atol=0)


def test_rms_norm_backward_equals_autograd():
    """dx and dw of the oracle's closed form equal autograd through F.rms_norm in fp64."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(40, 96, generator=g, dtype=torch.float64, requires_grad=True)
    w = (1 + 0.3 * torch.randn(96, generator=g, dtype=torch.float64)).requires_grad_()
    dy = torch.randn(40, 96, generator=g, dtype=torch.float64)
    y = torch.nn.functional.rms_norm(x, (96,), w, 1e-6)
    ax, aw = torch.autograd.grad(y, [x, w], dy)
    rstd = torch.rsqrt(x.detach().pow(2).mean(-1) + 1e-6)  # fp64, as autograd has it
    dx, dw = R.rms_norm_backward(dy, x.detach(), w.detach(), rstd)
    # rms_norm_backward works in fp32: compare at fp32 precision
    torch.testing.assert_close(dx.double(), ax, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(dw.double(), aw, rtol=1e-5, atol=1e-4)


def test_rms_norm_backward_rejects_a_dropped_term():
    """A planted mistake in the oracle (the mean term of dx dropped, or dw taken without
    rstd) fails the autograd check above."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(16, 64, generator=g, dtype=torch.float64, requires_grad=True)
    w = (1 + 0.3 * torch.randn(64, generator=g, dtype=torch.float64)).requires_grad_()
    dy = torch.randn(16, 64, generator=g, dtype=torch.float64)
    ax, aw = torch.autograd.grad(torch.nn.functional.rms_norm(x, (64,), w, 1e-6), [x, w], dy)
    rstd = torch.rsqrt(x.detach().pow(2).mean(-1, keepdim=True) + 1e-6)
    xh = x.detach() * rstd
    no_mean = dy * w.detach() * rstd
    assert not torch.allclose(no_mean, ax, rtol=1e-3, atol=1e-3)
    no_rstd_dw = (dy * x.detach()).sum(0)
    assert not torch.allclose(no_rstd_dw, aw, rtol=1e-3, atol=1e-3)
    assert torch.allclose((dy * xh).sum(0), aw)
