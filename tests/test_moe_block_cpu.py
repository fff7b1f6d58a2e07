"""
Host-side behaviour of the drop-in MoEBlock / TopKRouter, on CPU (no kernels run here):
constructor validation, parameter layout and RNG order, side-effect attributes, the
dispatch policy (capacity "auto", the kernel gate) and the reference's non-kernel modes.
Semantics follow the reference suite tests/test_moe.py; the code is this build's own.
"""

import pytest
import torch

from nanospeaker_amd import ACTIVATIONS, GLUFeedForward, MoEBlock, TopKRouter, glu_hidden_dim
from nanospeaker_amd import moe_kernel as mk
from oracle import moe_ref as R


def make(**kw):
    return MoEBlock(**{"d_model": 32, "n_experts": 8, "d_ff": 64, "fused": False, **kw})


# --- parameters -----------------------------------------------------------------------------

def test_parameter_layout_and_draw_order_match_the_reference():
    """Same seed -> the same tensors as the reference's MoEBlock (moe.py:131-168)."""
    torch.manual_seed(3)
    m = MoEBlock(576, 76, d_ff=192, top_k=6, n_shared=2, fused=False)
    p = R.make_params(3, 576, 76, 192, n_shared=2)
    assert m.W_in.shape == (76, 576, 256) and m.W_out.shape == (76, 128, 576)
    assert m.W_sh_in.shape == (2, 576, 256) and m.router.W.shape == (576, 76)
    for name, ref in (("W_in", p.W_in), ("W_out", p.W_out), ("W_sh_in", p.W_sh_in),
                      ("W_sh_out", p.W_sh_out)):
        assert torch.equal(getattr(m, name).data, ref), name
    assert torch.equal(m.router.W.data, p.W)


def test_state_dict_keys_are_the_references():
    m = make(n_shared=1, bias=True)
    assert set(m.state_dict()) == {"router.W", "W_in", "W_out", "b_in", "b_out", "W_sh_in",
                                   "W_sh_out", "b_sh_in", "b_sh_out"}


def test_glu_width_is_two_thirds_of_d_ff():
    assert glu_hidden_dim(192) == 128 and make().d_hidden == 42


# --- configuration ----------------------------------------------------------------------------

@pytest.mark.parametrize("kw", [{"top_k": 9}, {"top_k": 0}, {"n_experts": 0}, {"d_model": 0},
                                {"d_ff": 0}, {"d_ff": 1}, {"n_shared": -1},
                                {"capacity_factor": 0}, {"capacity_factor": -1.0}])
def test_impossible_configs_raise(kw):
    with pytest.raises(ValueError):
        make(**kw)


@pytest.mark.parametrize("bad", ["swiglu", "SiLU ", "", None, 7])
def test_unknown_activation_raises(bad):
    with pytest.raises(ValueError):
        make(activation=bad)


def test_activation_names_are_case_insensitive_and_callables_pass_through():
    assert make(activation="GELU").activation == "gelu"
    custom = make(activation=lambda t: t * torch.sigmoid(t))
    assert custom._kernel_act is None


def test_a_name_shadowed_by_a_callable_never_reaches_the_kernel():
    def silu(t):
        return t * torch.sigmoid(t)
    assert make(activation=silu)._kernel_act is None


def test_kernel_activations_match_the_reference_ids():
    assert mk.KERNEL_ACTIVATIONS == {"silu": 0, "swish": 0, "gelu": 1, "relu": 2,
                                     "sigmoid": 3, "tanh": 4}
    assert set(mk.KERNEL_ACTIVATIONS) == set(ACTIVATIONS)


# --- dispatch policy ---------------------------------------------------------------------------

def test_auto_capacity_pads_where_the_kernel_cannot_run():
    m = make()
    assert m._capacity_setting == "auto" and m.capacity_factor == 1.25
    assert not m._kernel_ready()


def test_auto_capacity_follows_the_kernel_gate(monkeypatch):
    m = make()
    monkeypatch.setattr(type(m), "_kernel_ready", lambda self: True)
    assert m.capacity_factor is None
    monkeypatch.setattr(type(m), "_kernel_ready", lambda self: False)
    assert m.capacity_factor == 1.25


def test_explicit_capacity_overrides_auto():
    assert make(capacity_factor=None).capacity_factor is None
    assert make(capacity_factor=4.0).capacity_factor == 4.0


def test_kernel_opt_out_and_fp64_fall_back_to_padding():
    assert make(kernel=False).capacity_factor == 1.25
    assert make().double().capacity_factor == 1.25


def test_kernel_predicate_is_device_and_dtype():
    assert not mk.kernel_supported(torch.zeros(1))
    assert not make(capacity_factor=None)._use_kernel(torch.zeros(1, 32))


def test_shape_limits():
    assert mk.shape_supported(76, 2, 128, torch.bfloat16)
    assert mk.shape_supported(76, 2, 256, torch.bfloat16)
    assert not mk.shape_supported(76, 2, 256, torch.float32)
    assert not mk.shape_supported(2000, 0, 64, torch.bfloat16)


# --- forward semantics (non-kernel modes on CPU) ------------------------------------------------

@pytest.mark.parametrize("shape", [(32,), (5, 32), (2, 7, 32), (2, 3, 5, 32)])
def test_leading_dims_are_preserved(shape):
    assert make()(torch.randn(*shape)).shape == shape


def test_empty_input_returns_empty_and_keeps_the_graph():
    x = torch.zeros(0, 32, requires_grad=True)
    y = make()(x)
    assert y.shape == (0, 32)
    y.sum().backward()


def test_wrong_width_raises():
    with pytest.raises(ValueError):
        make()(torch.randn(3, 31))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_dtype_is_preserved_and_finite(dtype):
    m = make().to(dtype)
    y = m(torch.randn(2, 8, 32, dtype=dtype))
    assert y.dtype == dtype and torch.isfinite(y).all()


@pytest.mark.parametrize("k", [1, 2, 8])
@pytest.mark.parametrize("bias", [False, True])
def test_ragged_dispatch_matches_dense_in_fp64(k, bias):
    m = make(top_k=k, bias=bias, capacity_factor=None, n_shared=1).double()
    x = torch.randn(3, 17, 32, dtype=torch.double)
    assert torch.allclose(m(x), m.dense_forward(x), atol=1e-12)


def test_ragged_cpu_path_equals_the_oracle_bit_for_bit():
    torch.manual_seed(0)
    m = MoEBlock(32, 8, d_ff=64, top_k=2, n_shared=1, capacity_factor=None,
                 fused=False).to(torch.bfloat16)
    x = torch.randn(40, 32).to(torch.bfloat16)
    p = R.Params(m.router.W.data, m.W_in.data, m.W_out.data, m.W_sh_in.data, m.W_sh_out.data)
    ref = R.block(x, p, 2)
    assert torch.equal(m(x), ref.out)
    assert torch.equal(m.expert_counts, ref.counts)


def test_counts_and_aux_loss_side_effects():
    m = make(top_k=3)
    m(torch.randn(4, 25, 32))
    assert int(m.expert_counts.sum()) == 4 * 25 * 3
    assert float(m.aux_loss.detach()) > 0
    m.eval()
    m(torch.randn(4, 32))
    assert float(m.aux_loss) == 0.0
    z = make(aux_loss_coef=0.0)
    z(torch.randn(4, 32))
    assert float(z.aux_loss) == 0.0


def test_capacity_drops_the_later_tokens():
    """test_moe.py:316-331, restated."""
    m = make(top_k=1)
    with torch.no_grad():
        m.router.W.zero_()
    out = m(torch.randn(64, 32))
    assert int(m.dropped) == 54
    assert (out[:10].abs().sum(1) > 0).all() and torch.allclose(out[10:], torch.zeros(54, 32))
    out = m(torch.randn(20, 32))
    assert (out.abs().sum(1) > 0).nonzero().flatten().tolist() == [0, 1, 2, 3]


def test_padded_and_ragged_agree_when_nothing_overflows():
    torch.manual_seed(0)
    padded = make(top_k=2, capacity_factor=100.0).double()
    torch.manual_seed(0)
    ragged = make(top_k=2, capacity_factor=None).double()
    x = torch.randn(4, 16, 32, dtype=torch.double)
    assert torch.allclose(padded(x), ragged(x), atol=1e-12)


def test_one_expert_moe_is_the_dense_glu():
    m = make(n_experts=1, top_k=1, normalize_weights=False).double()
    g = GLUFeedForward(32, d_ff=64, fused=False).double()
    g.W_in.data, g.W_out.data = m.W_in[0].data, m.W_out[0].data
    x = torch.randn(6, 32, dtype=torch.double)
    assert torch.allclose(m(x), g(x), atol=1e-12)


# --- router -----------------------------------------------------------------------------------

def test_router_outputs_and_short_circuit():
    r = TopKRouter(32, 8, top_k=3)
    w, idx, probs = r(torch.randn(20, 32))
    assert torch.allclose(w.sum(-1), torch.ones(20), atol=1e-6) and probs is not None
    assert r.eval()(torch.randn(4, 32))[2] is None


def test_router_noise_only_in_training():
    r = TopKRouter(32, 8, top_k=1, noise_std=5.0)
    x = torch.randn(64, 32)
    r.train()
    picks = {tuple(r(x)[1].flatten().tolist()) for _ in range(5)}
    assert len(picks) > 1
    r.eval()
    assert torch.equal(r(x)[1], r(x)[1])


def test_balance_loss_is_the_references():
    r = TopKRouter(32, 4, top_k=1)
    probs = torch.rand(16, 4).softmax(-1)
    counts = torch.tensor([5, 3, 8, 0])
    assert torch.equal(r.balance_loss(probs, counts), R.balance_loss(probs, counts, 1e-2, 4))
