"""
GPU parity of the tied head's cross-entropy (nsmoe_cross_entropy_rows,
nanospeaker_amd/csrc/ce.hip, inside head.linear_cross_entropy) against the reference's
expression, F.cross_entropy((h @ W.T).float(), y) (src/model/nanospeaker.py:241-250):

  * per row, on the same bf16 logits: the loss to fp32 rounding of F.cross_entropy's
    (reduction='none'), and the gradient written in place, (softmax - onehot) / n, within
    one bf16 rounding step (plus 1e-9 absolute) of torch's fp32 gradient of the mean loss;
  * end to end, the mean loss to fp32 rounding of F.cross_entropy on the same bf16 logits
    (and within 1 % of the loss on fp32 logits), and dh, dW within the bf16 bar of the
    reference's gradient accumulated in fp32 (its bf16 logits, d(loss)/d(logits) in
    fp32, the GEMM backward in fp32), with ignored targets, with the rows split over
    several chunks, and at the long-context shape (8191 next-token rows, 32768-token
    vocabulary, d 576);
  * a target past the vocabulary gives a NaN loss instead of a read outside the row; every
    target ignored gives NaN, as F.cross_entropy's mean does.
"""

import pytest
import torch
import torch.nn.functional as F

from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

pytest.importorskip("nanospeaker_amd.moe_kernel")
from nanospeaker_amd.head import cross_entropy_rows, linear_cross_entropy  # noqa: E402

DEV = "cuda"


def make(n, V, d, seed=0, ignore_every=0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, d, generator=g) * 0.05).to(torch.bfloat16)
    y = torch.randint(0, V, (n,), generator=g)
    if ignore_every:
        y[::ignore_every] = -100
    return h.to(DEV), W.to(DEV), y.to(DEV)


@pytest.mark.parametrize("n,V", [(300, 32768), (17, 1000), (64, 8), (5, 65536)])
def test_rows_loss_and_gradient(n, V):
    print(f"[head] rows n={n} V={V}", flush=True)
    g = torch.Generator().manual_seed(V)
    logits = (torch.randn(n, V, generator=g) * 3).to(torch.bfloat16).to(DEV)
    y = torch.randint(0, V, (n,), generator=g).to(DEV)
    y[1::7] = -100
    ref = F.cross_entropy(logits.float(), y, reduction="none")
    n_valid = (y != -100).sum()
    got = cross_entropy_rows(logits.clone(), y, -100, n_valid, grad=False)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)
    lf = logits.float().requires_grad_(True)
    F.cross_entropy(lf, y).backward()
    work = logits.clone()
    cross_entropy_rows(work, y, -100, n_valid, grad=True)
    step = 2.0 ** -8 * lf.grad.abs() + 1e-9
    err = (work.float() - lf.grad).abs()
    assert bool((err <= step * 1.01).all()), f"gradient off by {float((err / step).max()):.2f} steps"


@pytest.mark.parametrize("n,V,d,ignore_every,chunk_bytes", [
    (500, 4096, 64, 0, 4 << 30),
    (500, 4096, 64, 5, 4 << 30),        # ignored targets excluded from the mean
    (500, 4096, 64, 3, 100 * 4096 * 2),  # five chunks, dW accumulated in fp32
])
def test_linear_cross_entropy_small(n, V, d, ignore_every, chunk_bytes):
    run(n, V, d, ignore_every, chunk_bytes)


def test_linear_cross_entropy_long_context_shape():
    """One 8192-token sequence: 8191 next-token rows against the 32768-token vocabulary."""
    run(8191, 32768, 576, 0, 4 << 30)


def run(n, V, d, ignore_every, chunk_bytes):
    print(f"[head] n={n} V={V} d={d} ignore_every={ignore_every} chunk={chunk_bytes}",
          flush=True)
    h, W, y = make(n, V, d, seed=n + V, ignore_every=ignore_every)
    hg, Wg = h.clone().requires_grad_(True), W.clone().requires_grad_(True)
    loss = linear_cross_entropy(hg, Wg, y, chunk_bytes=chunk_bytes)
    loss.backward()
    with torch.no_grad():
        ref_same_logits = F.cross_entropy((h @ W.t()).float(), y)
    torch.testing.assert_close(loss, ref_same_logits, rtol=1e-5, atol=1e-6)
    # The reference's own gradient, accumulated in fp32: its logits are the bf16 GEMM's
    # output (`(h @ W.T).float()`), d(loss)/d(logits) is formed in fp32, and the GEMM's
    # backward contracts it with W and h (the reference's autograd rounds it to bf16 on
    # the way back through `.float()`; here it stays fp32).
    with torch.no_grad():
        lg = (h @ W.t()).float()
    lf = lg.requires_grad_(True)
    F.cross_entropy(lf, y).backward()
    dh_ref = lf.grad @ W.float()
    dW_ref = lf.grad.t() @ h.float()
    with torch.no_grad():
        fp32_logits = F.cross_entropy(h.float() @ W.float().t(), y)
    print(f"  loss {float(loss):.6f} (fp32 logits: {float(fp32_logits):.6f})", flush=True)
    assert abs(float(loss) - float(fp32_logits)) <= 1e-2 * max(1.0, abs(float(fp32_logits)))
    assert_close_bf16("dh", hg.grad.float().cpu(), dh_ref.cpu())
    assert_close_bf16("dW", Wg.grad.float().cpu(), dW_ref.cpu())


def test_bad_target_and_all_ignored():
    logits = torch.randn(4, 64, device=DEV).to(torch.bfloat16)
    y = torch.tensor([3, 64, -5, -100], device=DEV)
    got = cross_entropy_rows(logits, y, -100)
    assert torch.isfinite(got[0]) and torch.isnan(got[1]) and torch.isnan(got[2])
    assert float(got[3]) == 0.0
    h, W, _ = make(8, 64, 32)
    y = torch.full((8,), -100, device=DEV)
    assert torch.isnan(linear_cross_entropy(h, W, y))
