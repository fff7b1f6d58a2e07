"""Shared test plumbing: golden fixtures, input recipes, tolerances, oracle build."""

from __future__ import annotations

import ctypes
import json
import subprocess
from contextlib import contextmanager
from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

from oracle import moe_ref as R

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"

# bf16 tolerance of the north star: max abs err <= 2e-2 and rel-L2 <= 5e-3 against the
# fp32-accumulated reference.  The absolute bound is read on the tensor's own scale,
# max|err| <= 2e-2 * max(1, max|ref|): a bf16 value of magnitude 10 is itself only
# stored to +-0.03, so an unscaled bound would fail the reference's own bf16 path on
# large gradients (the shared experts' dW reach |10| at T = 2048).
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 5e-3
# fp32 kernels against the fp32 reference (the reference's own kernel tests use 1e-5).
F32_ATOL = 1e-5


@lru_cache(maxsize=1)
def golden():
    meta = json.loads((GOLDEN / "moe_golden.json").read_text())
    arrays = np.load(GOLDEN / "moe_golden.npz", allow_pickle=False)
    return meta, {k: arrays[k] for k in arrays.files}


def from_np(a: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "bfloat16":
        return torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(np.array(a))


def golden_inputs(info: dict):
    """Regenerate a golden case's params, x and upstream grad (make_golden.py's recipe)."""
    dt = getattr(torch, info["dtype"])
    p = R.make_params(info["seed"], info["d"], info["E"], info["d_ff"],
                      n_shared=info["n_shared"], bias=info["bias"])
    if info["bias"]:
        g_b = torch.Generator().manual_seed(info["seed"] + 1000)
        for name in ("b_in", "b_out", "b_sh_in", "b_sh_out"):
            t = getattr(p, name)
            if t is not None:
                setattr(p, name, torch.randn(t.shape, generator=g_b) * 0.1)
    p = p.to(dtype=dt)
    x = torch.randn(info["n_tokens"], info["d"]).to(dt)
    g = torch.randn(info["n_tokens"], info["d"]).to(dt)
    return p, x, g


def nanospeaker_inputs(T: int, seed: int = 0, dtype=torch.bfloat16):
    """Benchmark recipe: seed, params in the reference's order (x0.02, bf16), x, g."""
    c = R.nanospeaker_config()
    p = R.make_params(seed, c["d"], c["E"], c["d_ff"], n_shared=c["n_shared"]).to(dtype=dtype)
    x = torch.randn(T, c["d"]).to(dtype)
    g = torch.randn(T, c["d"]).to(dtype)
    return p, x, g


@lru_cache(maxsize=1)
def oracle_topk_lib():
    """Builds (if needed) and loads the C restatement of CPU topk (oracle/topk_select.c)."""
    src = ROOT / "oracle" / "topk_select.c"
    so = ROOT / "oracle" / "liboracle_topk.so"
    if not so.exists() or so.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["gcc", "-O2", "-fPIC", "-shared", str(src), "-o", str(so), "-lm"],
                       check=True)
    lib = ctypes.CDLL(str(so))
    lib.oracle_topk_rows.restype = ctypes.c_int
    lib.oracle_topk_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p]
    return lib


def oracle_topk(vals: np.ndarray, k: int) -> np.ndarray:
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    rows, n = vals.shape
    idx = np.zeros((rows, k), np.int64)
    scratch = np.zeros(2 * max(n, 1), np.float64)
    rc = oracle_topk_lib().oracle_topk_rows(
        vals.ctypes.data, rows, n, k, idx.ctypes.data, None, scratch.ctypes.data)
    assert rc == 0
    return idx


def tie_heavy(rows: int, n: int, levels: int, seed: int) -> torch.Tensor:
    """fp32 rows drawn from `levels` distinct values: many exact ties."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, levels, (rows, n), generator=g).float() * 0.25 - 0.5


def assert_close_bf16(name, got, ref, max_abs=BF16_MAX_ABS, rel_l2=BF16_REL_L2):
    """The bf16 bar; prints the unscaled max-abs error and rel-L2 beside the bound."""
    ref = ref.cpu()
    scale = max(1.0, float(ref.abs().max())) if ref.numel() else 1.0
    ok, err, rl2 = R.is_close(got.cpu(), ref, max_abs * scale, rel_l2)
    print(f"  {name}: max abs {err:.3e} (bound {max_abs * scale:.3e} = {max_abs} x "
          f"{scale:.3g}), rel-L2 {rl2:.3e} (bound {rel_l2})")
    assert ok, (f"{name}: max abs {err:.3e} (<= {max_abs} x {scale:.3g}), "
                f"rel-L2 {rl2:.3e} (<= {rel_l2})")


@contextmanager
def lib_options(**values):
    """Sets libnsmoe tuning options (nsmoe_set_option) for the body, then restores 0."""
    from nanospeaker_amd import _native as nat
    try:
        for name, v in values.items():
            nat.set_option(name, v)
        yield
    finally:
        for name in values:
            nat.set_option(name, 0)
