"""
Writes tests/golden/zipf_logit_bias.npy: the per-expert logit offset b[76] of the skewed
routing workload (T = 16384, fwd + bwd).

The reference router has no bias parameter (src/model/router.py:50), so the skew is a
harness-level offset added to the fp32 logits before the softmax / top-k.  b is fitted
on the CPU so that the realised share of top-6 assignments per expert follows
Zipf(s = 1.2) over the 76 experts.  One expert can hold at most 1/6 of the assignments
(a token picks 6 distinct experts), so the Zipf head (28.6 % uncapped) is capped at 15 %
and the excess is spread over the other experts in proportion to their Zipf weight.

Run from the repository root:  python -m tests.golden.make_zipf_bias
Inputs: seed 0, the benchmark's parameter recipe, x ~ N(0, 1) in bf16 at T = 16384.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from oracle import moe_ref as R

OUT = Path(__file__).resolve().parent / "zipf_logit_bias.npy"
T, S_ZIPF, CAP = 16384, 1.2, 0.15


def zipf_target(E: int) -> torch.Tensor:
    w = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** S_ZIPF
    t = w / w.sum()
    for _ in range(50):                      # cap the head, renormalise the rest
        over = t > CAP
        if not over.any():
            break
        excess = float((t[over] - CAP).sum())
        t[over] = CAP
        free = ~over & (t < CAP)
        t[free] += excess * t[free] / t[free].sum()
    return t


def realised(logits: torch.Tensor, b: torch.Tensor, k: int) -> torch.Tensor:
    probs = torch.softmax(logits + b, dim=-1)
    idx = probs.topk(k, dim=-1).indices
    return torch.bincount(idx.reshape(-1), minlength=logits.shape[1]).double() / idx.numel()


def main() -> None:
    c = R.nanospeaker_config()
    p = R.make_params(0, c["d"], c["E"], c["d_ff"], n_shared=c["n_shared"]).to(
        dtype=torch.bfloat16)
    x = torch.randn(T, c["d"]).to(torch.bfloat16)
    logits = R.router_logits(x, p.W)
    target = zipf_target(c["E"])
    b = torch.zeros(c["E"], dtype=torch.float32)
    for _ in range(600):                     # damped multiplicative fit of the shares
        share = realised(logits, b, c["top_k"])
        step = (target.log() - (share + 1e-4).log()).clamp(-0.5, 0.5)
        b += 0.3 * step.float()
        b -= b.mean()
    share = realised(logits, b, c["top_k"])
    np.save(OUT, b.numpy().astype(np.float32), allow_pickle=False)
    print(f"wrote {OUT}: head share {float(share.max()):.4f}, "
          f"max |share - target| {float((share - target).abs().max()):.4f}, "
          f"empty experts {int((share == 0).sum())}")


if __name__ == "__main__":
    main()
