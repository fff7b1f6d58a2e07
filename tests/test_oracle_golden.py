"""
Pins the oracle's restatement of the reference eager path (oracle/moe_ref.py) against
vectors the reference itself produced (tests/golden/make_golden.py): RNG draw order,
routing indices and gates, the stable permutation, counts, the bf16/fp32 outputs, the
balance loss and every gradient -- bit for bit.
"""

import hashlib

import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import from_np, golden, golden_inputs

META, ARRAYS = golden()


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _check(name, key, t):
    spec = META[name]["arrays"][key]
    assert list(t.shape) == spec["shape"], f"{name}/{key} shape"
    digest = hashlib.sha256(_np(t).tobytes()).hexdigest()
    if spec["full"]:
        want = ARRAYS[f"{name}/{key}"]
        assert np.array_equal(_np(t), want), f"{name}/{key} differs from the reference"
    assert digest == spec["sha256"], f"{name}/{key} digest differs from the reference"


def _compare_with_fixture(name):
    info = META[name]
    p, x, g = golden_inputs(info)
    res = R.block(x, p, info["top_k"], train=info["train"], normalize=info["normalize"],
                  activation=info["activation"], grad_out=g)
    _, order, _, counts = R.plan(res.topk_idx, info["E"])
    _check(name, "topk_idx", res.topk_idx)
    _check(name, "topk_w", res.topk_w)
    _check(name, "order", order)
    _check(name, "counts", counts)
    _check(name, "out", res.out)
    _check(name, "aux_loss", res.aux_loss.reshape(1))
    _check(name, "grad_x", res.grads["x"])
    rename = {"router_W": "W"}
    for key in info["arrays"]:
        if key.startswith("grad_") and key != "grad_x":
            pname = rename.get(key[5:], key[5:])
            _check(name, key, res.grads[pname])


@pytest.mark.parametrize("name", sorted(META))
def test_oracle_reproduces_the_reference(name):
    _compare_with_fixture(name)


# Planted mistakes: each is a plausible slip in a restatement of the reference, and the
# fixtures above must reject every one of them (otherwise they would pin nothing).
def _glu_swapped(act, gate, up):
    return act(up) * gate


def _expert_without_b_out(x, W_in, W_out, b_in, b_out, act):
    return _ORIG_EXPERT(x, W_in, W_out, b_in, None, act)


def _plan_unstable(topk_idx, E):
    flat = topk_idx.reshape(-1)
    n = flat.numel()
    key = flat * n + (n - 1 - torch.arange(n))       # reversed order inside each expert
    order = key.argsort()
    experts = flat[order]
    counts = torch.searchsorted(experts, torch.arange(E + 1)).diff()
    return experts, order, order // topk_idx.shape[-1], counts


def _route_without_renorm(logits, top_k, want_probs, normalize, dtype):
    return _ORIG_ROUTE(logits, top_k, want_probs, False, dtype)


def _balance_without_E(probs, counts, coef, E):
    return _ORIG_BALANCE(probs, counts, coef, 1)


_ORIG_EXPERT, _ORIG_ROUTE, _ORIG_BALANCE = R._expert, R.route_from_logits, R.balance_loss

MUTANTS = [
    ("_glu", _glu_swapped, "small_bf16"),
    ("_expert", _expert_without_b_out, "small_k8_bias"),
    ("plan", _plan_unstable, "small_k2"),
    ("route_from_logits", _route_without_renorm, "small_k2"),
    ("balance_loss", _balance_without_E, "small_k1"),
]


@pytest.mark.parametrize("attr,mutant,case", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_fixtures_reject_a_planted_mistake(monkeypatch, attr, mutant, case):
    monkeypatch.setattr(R, attr, mutant)
    with pytest.raises(AssertionError):
        _compare_with_fixture(case)


def test_fixture_inputs_follow_the_baseline_recipe():
    """The nanoSpeaker cases use the benchmark's shapes (d 576, 76 + 2 experts, k 6, H 128)."""
    info = META["ns_t64_train"]
    assert (info["d"], info["E"], info["n_shared"], info["top_k"]) == (576, 76, 2, 6)
    assert R.glu_hidden_dim(info["d_ff"]) == 128
