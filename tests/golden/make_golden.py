"""
Writes tests/golden/moe_golden.npz + moe_golden.json: input/output vectors of the
reference's own MoE block (src/model/moe.py, router.py), run on CPU in THIS container.

Why: the CPU restatement in oracle/moe_ref.py claims to reproduce the reference's eager
path bit for bit -- its RNG draw order, its routing (torch.topk tie order included), its
stable-sort permutation and its bf16 rounding points.  Nothing but the reference itself
can pin that, so this script imports it once and records what it computes; the fixtures
then travel, the reference does not.  Inputs are not stored: every case is regenerated
from (seed, shape) by the same recipe the tests use (oracle.moe_ref.make_params, then
x and the upstream gradient drawn from the same generator).

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent

CASES = [
    # name, d, E, d_ff, top_k, n_shared, bias, activation, dtype, train, n_tokens, seed, normalize
    ("small_k2", 32, 8, 64, 2, 0, False, "silu", "float32", True, 51, 0, True),
    ("small_k1", 32, 8, 64, 1, 0, False, "silu", "float32", True, 51, 1, True),
    ("small_k8_bias", 32, 8, 64, 8, 0, True, "silu", "float32", True, 51, 2, True),
    ("small_shared2_bias", 32, 8, 64, 2, 2, True, "silu", "float32", True, 51, 3, True),
    ("small_gelu", 32, 8, 64, 2, 1, False, "gelu", "float32", True, 42, 4, True),
    ("small_relu", 32, 8, 64, 2, 0, False, "relu", "float32", True, 42, 5, True),
    ("small_sigmoid", 32, 8, 64, 2, 0, False, "sigmoid", "float32", True, 42, 6, True),
    ("small_tanh", 32, 8, 64, 2, 0, False, "tanh", "float32", True, 42, 7, True),
    ("small_eval", 32, 8, 64, 3, 1, False, "silu", "float32", False, 40, 8, True),
    ("small_unnorm", 32, 8, 64, 3, 0, False, "silu", "float32", True, 40, 9, False),
    ("small_eval_unnorm", 32, 8, 64, 3, 0, False, "silu", "float32", False, 40, 10, False),
    ("small_bf16", 32, 8, 64, 2, 1, False, "silu", "bfloat16", True, 65, 11, True),
    ("ns_t64_train", 576, 76, 192, 6, 2, False, "silu", "bfloat16", True, 64, 0, True),
    ("ns_t64_eval", 576, 76, 192, 6, 2, False, "silu", "bfloat16", False, 64, 0, True),
    ("ns_t256_train", 576, 76, 192, 6, 2, False, "silu", "bfloat16", True, 256, 1, True),
]

# Arrays larger than this are stored as a digest + moments + a leading slice.
FULL_LIMIT = 1 << 16


def as_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(as_np(t).tobytes()).hexdigest()


def main() -> None:
    sys.path.insert(0, str(REF))
    from src.model.moe import MoEBlock  # noqa: E402  (the reference, CPU eager path)

    arrays: dict[str, np.ndarray] = {}
    meta: dict[str, dict] = {}
    for (name, d, E, d_ff, k, S, bias, act, dtype, train, T, seed, norm) in CASES:
        dt = getattr(torch, dtype)
        torch.manual_seed(seed)
        m = MoEBlock(d, E, d_ff=d_ff, top_k=k, n_shared=S, capacity_factor=None,
                     activation=act, bias=bias, normalize_weights=norm, fused=False,
                     kernel=False)
        if bias:  # non-zero biases so their gradients and forward terms are exercised
            g_b = torch.Generator().manual_seed(seed + 1000)
            with torch.no_grad():
                for p in (m.b_in, m.b_out, m.b_sh_in, m.b_sh_out):
                    if p is not None:
                        p.copy_(torch.randn(p.shape, generator=g_b) * 0.1)
        m = m.to(dt).train(train)
        x = torch.randn(T, d).to(dt).requires_grad_(True)
        g = torch.randn(T, d).to(dt)
        topk_w, topk_idx, probs = m.router(x.detach())
        _, order, _, counts = m._plan(topk_idx)
        out = m(x)
        loss = (out.float() * g.float()).sum() + m.aux_loss.float()
        loss.backward()
        rec = {
            "topk_idx": topk_idx, "topk_w": topk_w, "order": order, "counts": counts,
            "out": out, "aux_loss": m.aux_loss.detach().reshape(1),
            "grad_x": x.grad,
        }
        for pname, p in m.named_parameters():
            if p.grad is not None:
                rec["grad_" + pname.replace(".", "_")] = p.grad
        info = {"d": d, "E": E, "d_ff": d_ff, "top_k": k, "n_shared": S, "bias": bias,
                "activation": act, "dtype": dtype, "train": train, "n_tokens": T,
                "seed": seed, "normalize": norm, "arrays": {}}
        for key, t in rec.items():
            full = t.numel() <= FULL_LIMIT
            info["arrays"][key] = {
                "shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", ""),
                "sha256": digest(t), "full": full,
                "sum": float(t.double().sum()), "sumsq": float(t.double().square().sum()),
            }
            arr = as_np(t) if full else as_np(t.reshape(-1)[:4096])
            arrays[f"{name}/{key}"] = arr
        meta[name] = info
        print(name, "done", flush=True)

    np.savez_compressed(OUT / "moe_golden.npz", **arrays)
    (OUT / "moe_golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print("wrote", OUT / "moe_golden.npz")


if __name__ == "__main__":
    main()
