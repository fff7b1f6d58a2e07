"""
GPU parity of the router tail and the dispatch against the CPU oracle.

Routing indices, counts and the whole permutation must be bit-exact: the oracle is
CPU torch.topk (the call the reference makes, router.py:81/87) and the stable sort of
MoEBlock._plan (moe.py:220-222).  Gates and probabilities are floating point and are
held to fp32 / bf16 rounding.
"""

import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests.helpers import nanospeaker_inputs, tie_heavy

pytestmark = pytest.mark.gpu

mk = pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd import _native as nat  # noqa: E402

DEV = "cuda"


def _gpu_route(logits, k, want_probs, normalize, dtype):
    w, idx, probs = mk.route(logits.to(DEV), k, want_probs, normalize, mk.route_dtype_code(dtype))
    return w.cpu(), idx.cpu(), probs.cpu() if want_probs else None


@pytest.mark.parametrize("E,k", [(76, 6), (8, 2), (8, 8), (76, 1), (128, 2), (8, 1), (3, 2)])
@pytest.mark.parametrize("train", [True, False])
@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("levels", [2, 5, 40, 0])
def test_route_indices_bit_exact_with_ties(E, k, train, normalize, levels):
    """Tie-heavy and realistic logit rows: indices equal CPU torch.topk's, ties included."""
    T = 700
    if levels:
        logits = tie_heavy(T, E, levels, seed=E * 100 + k * 7 + levels)
    else:  # bf16-rounded realistic logits, as (x @ W).float() produces them
        logits = (torch.randn(T, E) * 0.48).bfloat16().float()
    w_ref, idx_ref, p_ref = R.route_from_logits(logits, k, train, normalize, torch.float32)
    w, idx, p = _gpu_route(logits, k, train, normalize, torch.float32)
    assert torch.equal(idx, idx_ref)
    torch.testing.assert_close(w, w_ref, rtol=2e-6, atol=2e-7)
    if train:
        torch.testing.assert_close(p, p_ref, rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("train", [True, False])
def test_route_rows_with_and_without_ties_in_one_launch(train):
    """The kernel takes a fast arg-max path on rows whose top k is unique and the exact
    introselect on rows with ties; rows of both kinds, interleaved, plus signed zeros,
    infinities and NaN rows, must all equal CPU torch.topk."""
    E, k, T = 76, 6, 1024
    g = torch.Generator().manual_seed(11)
    logits = (torch.randn(T, E, generator=g) * 0.48).bfloat16().float()
    ties = tie_heavy(T, E, 3, seed=12)
    logits[1::3] = ties[1::3]                                  # every third row tie-heavy
    logits[5, :] = 0.0
    logits[5, 10] = -0.0                                       # -0 and +0 compare equal
    logits[7, :6] = torch.tensor([3.0, 2.0, 1.0, 0.5, -0.0, 0.0])
    logits[8, :] = -float("inf")
    logits[8, 3] = 1.0                                         # one finite value, rest -inf
    logits[9, 2] = float("inf")
    logits[10, 40] = float("nan")
    logits[11, :8] = torch.arange(8.0)                         # tie exactly at the boundary
    logits[11, 8:] = 1.0
    w_ref, idx_ref, _ = R.route_from_logits(logits, k, train, True, torch.float32)
    w, idx, _ = _gpu_route(logits, k, train, True, torch.float32)
    assert torch.equal(idx, idx_ref)
    ok = torch.isfinite(w_ref).all(dim=1)
    torch.testing.assert_close(w[ok], w_ref[ok], rtol=2e-6, atol=2e-7)


def test_route_bf16_gates_and_probs():
    """nanoSpeaker router shape, bf16 gates: at most one bf16 ulp from the CPU cast."""
    p, x, _ = nanospeaker_inputs(4096)
    logits = R.router_logits(x, p.W)
    w_ref, idx_ref, p_ref = R.route_from_logits(logits, 6, True, True, torch.bfloat16)
    w, idx, pr = _gpu_route(logits, 6, True, True, torch.bfloat16)
    assert torch.equal(idx, idx_ref)
    torch.testing.assert_close(w.float(), w_ref.float(), rtol=8e-3, atol=0)
    torch.testing.assert_close(pr, p_ref, rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("train,normalize,k", [(True, True, 6), (True, False, 6),
                                               (False, True, 6), (False, False, 3),
                                               (True, True, 1)])
def test_route_backward_matches_autograd(train, normalize, k):
    E, T = 76, 500
    logits = torch.randn(T, E) * 0.6
    gw = torch.randn(T, k)
    gp = torch.randn(T, E) * 1e-3
    lr = logits.clone().requires_grad_(True)
    w_ref, _, p_ref = R.route_from_logits(lr, k, train, normalize, torch.float32)
    loss = (w_ref * gw).sum() + ((p_ref * gp).sum() if train else 0.0)
    loss.backward()
    lg = logits.to(DEV).requires_grad_(True)
    w, _, pr = mk.route(lg, k, train, normalize, mk.route_dtype_code(torch.float32))
    loss_g = (w * gw.to(DEV)).sum() + ((pr * gp.to(DEV)).sum() if train else 0.0)
    loss_g.backward()
    torch.testing.assert_close(lg.grad.cpu(), lr.grad, rtol=1e-4, atol=1e-6)


def _dispatch_check(topk_idx, E):
    got = [t.cpu() for t in mk.moe_dispatch(topk_idx.to(DEV), E)]
    ref = R.dispatch_buffers(topk_idx, E, mk.ALIGN_M)
    sids, eids, offs, counts, npp, inv = got
    assert torch.equal(sids, ref[0]), "sorted ids differ"
    assert torch.equal(eids, ref[1]), "block owners differ"
    assert torch.equal(offs, ref[2]), "run offsets differ"
    assert torch.equal(counts, ref[3]), "counts differ"
    assert int(npp) == ref[4]
    assert torch.equal(inv, ref[5]), "inverse differs"
    return got


@pytest.mark.parametrize("T,E,k", [(1, 8, 1), (1, 8, 2), (3, 8, 8), (15, 8, 2), (16, 8, 2),
                                   (17, 8, 2), (64, 76, 6), (2048, 76, 6), (8192, 76, 6),
                                   (333, 1000, 4)])
def test_dispatch_bit_exact(T, E, k):
    g = torch.Generator().manual_seed(T + E)
    scores = torch.rand(T, E, generator=g)
    topk_idx = scores.topk(k, dim=-1).indices
    _dispatch_check(topk_idx, E)


def test_dispatch_collapsed_and_skewed():
    """One expert takes everything; then a Zipf-skewed load."""
    _dispatch_check(torch.zeros(300, 1, dtype=torch.long), 8)
    E, T, k = 76, 16384, 6
    w = 1.0 / torch.arange(1, E + 1).double() ** 1.2
    g = torch.Generator().manual_seed(3)
    idx = torch.multinomial(w.expand(T, E), k, replacement=False, generator=g)
    sids, _, _, counts, _, _ = _dispatch_check(idx, E)
    assert int(counts.max()) > 0.1 * T


def test_dispatch_reference_invariants():
    """test_moe_kernel.py:197-216, restated: dense prefixes, sentinels, block owners."""
    topk_idx = torch.randint(0, 8, (50, 2))
    sids, eids, offs, counts, npp, inv = [t.cpu() for t in mk.moe_dispatch(topk_idx.to(DEV), 8)]
    m = topk_idx.numel()
    assert torch.equal(sids[inv.long()], torch.arange(m, dtype=torch.int32))
    assert torch.equal(counts.long(), torch.bincount(topk_idx.reshape(-1), minlength=8))
    assert int(npp) == int((torch.ceil(counts.float() / mk.ALIGN_M) * mk.ALIGN_M).sum())
    flat = topk_idx.reshape(-1)
    for e in range(8):
        run = sids[int(offs[e]): int(offs[e]) + int(counts[e])].long()
        assert (flat[run] == e).all()
        assert torch.equal(run, run.sort().values)       # stable: increasing pair id
        pad = sids[int(offs[e]) + int(counts[e]): int(offs[e + 1])]
        assert (pad == m).all()
    blocks = torch.arange(int(npp) // mk.ALIGN_M) * mk.ALIGN_M
    assert (offs[eids[: len(blocks)].long()] <= blocks).all()


def test_dispatch_handles_no_pairs():
    sids, eids, offs, counts, npp, inv = mk.moe_dispatch(
        torch.zeros(0, 2, dtype=torch.long, device=DEV), 8)
    assert sids.numel() == 0 and int(npp) == 0 and int(counts.sum()) == 0 and inv.numel() == 0


def test_dispatch_is_deterministic():
    idx = torch.randint(0, 76, (8192, 6))
    a = [t.cpu() for t in mk.moe_dispatch(idx.to(DEV), 76)]
    b = [t.cpu() for t in mk.moe_dispatch(idx.to(DEV), 76)]
    assert all(torch.equal(u, v) for u, v in zip(a, b))


def test_native_library_ran():
    before = nat.launch_count()
    mk.moe_dispatch(torch.randint(0, 8, (10, 2), device=DEV), 8)
    torch.cuda.synchronize()
    assert nat.launch_count() > before
