"""
ORACLE -- test infrastructure only.

Nothing in nanospeaker_amd/ imports this module.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may use it, and only as the checker (or, for the CPU
baseline, as the thing timed on the host): the product path never routes through it.

CPU restatement, op for op in torch, of the reference's eager dropless MoE path:

  router         src/model/router.py:56-111    (TopKRouter.forward / balance_loss)
  plan           src/model/moe.py:208-223      (stable sort -> order, token, counts)
  expert         src/model/moe.py:285-308      (x@W_in -> chunk -> glu -> @W_out -> *w)
  shared         src/model/moe.py:310-329
  eager forward  src/model/moe.py:345-418      (index_add_ in expert order 0..E-1)
  dense forward  src/model/moe.py:420-474      (every expert on every token)
  glu            src/model/glu.py:44-45        (act(gate) * up)
  rms norm       src/model/ln.py:30-36         (F.rms_norm: fp32 rstd, (x rstd) w, one
                                                rounding; its backward)
  ffn sublayer   src/model/nanospeaker.py:169  (x + ffn(norm_ffn(x)))

`eager_forward` keeps the reference's rounding points in the module dtype, so in bf16 it
reproduces the reference's own CPU numbers bit for bit (pinned against fixtures the
reference wrote, tests/golden).  `fp32_forward` runs the same routing with fp32
arithmetic on the same (bf16-valued) inputs: the "fp32-accumulated reference" the HIP
kernels are held to within bf16 tolerance.  Backward references are torch autograd
through these functions.

Parameter generation follows the reference's RNG order (router.W, W_in, W_out, W_sh_in,
W_sh_out; moe.py:131-165, router.py:50) so a seed means the same weights everywhere.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch
import torch.nn.functional as F

ACTS = {
    "silu": F.silu, "swish": F.silu, "gelu": F.gelu, "relu": F.relu,
    "sigmoid": torch.sigmoid, "tanh": torch.tanh,
}


@dataclass
class Params:
    W: torch.Tensor            # router [d, E]
    W_in: torch.Tensor         # [E, d, 2H]
    W_out: torch.Tensor        # [E, H, d]
    W_sh_in: Optional[torch.Tensor] = None
    W_sh_out: Optional[torch.Tensor] = None
    b_in: Optional[torch.Tensor] = None
    b_out: Optional[torch.Tensor] = None
    b_sh_in: Optional[torch.Tensor] = None
    b_sh_out: Optional[torch.Tensor] = None

    def to(self, dtype=None, device=None) -> "Params":
        conv = lambda t: None if t is None else t.to(device=device, dtype=dtype)
        return Params(*(conv(getattr(self, f)) for f in self.__dataclass_fields__))

    def named(self):
        return {f: getattr(self, f) for f in self.__dataclass_fields__
                if getattr(self, f) is not None}


def glu_hidden_dim(d_ff: int) -> int:
    """glu.py:16-29."""
    return 2 * d_ff // 3


def make_params(seed: int, d: int, E: int, d_ff: int, n_shared: int = 0, bias: bool = False,
                std: float = 0.02, dtype=torch.float32) -> Params:
    """The reference's parameter draws, in its order (MoEBlock.__init__, moe.py:131-168)."""
    torch.manual_seed(seed)
    H = glu_hidden_dim(d_ff)
    W = torch.randn(d, E) * std
    W_in = torch.randn(E, d, 2 * H) * std
    W_out = torch.randn(E, H, d) * std
    b_in = torch.zeros(E, 2 * H) if bias else None
    b_out = torch.zeros(E, d) if bias else None
    W_sh_in = W_sh_out = b_sh_in = b_sh_out = None
    if n_shared:
        W_sh_in = torch.randn(n_shared, d, 2 * H) * std
        W_sh_out = torch.randn(n_shared, H, d) * std
        if bias:
            b_sh_in = torch.zeros(n_shared, 2 * H)
            b_sh_out = torch.zeros(n_shared, d)
    p = Params(W, W_in, W_out, W_sh_in, W_sh_out, b_in, b_out, b_sh_in, b_sh_out)
    return p.to(dtype=dtype)


# ---- router (router.py:56-111) -------------------------------------------------------------

def router_logits(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """router.py:69: the GEMM in x's dtype, then lifted to fp32."""
    return (x @ W).float()


def route_from_logits(logits: torch.Tensor, top_k: int, want_probs: bool, normalize: bool,
                      out_dtype: torch.dtype):
    """router.py:79-98 on given fp32 logits -> (topk_w, topk_idx, probs or None)."""
    if want_probs:
        probs = F.softmax(logits, dim=-1)
        topk_w, topk_idx = probs.topk(top_k, dim=-1)
    else:
        probs = None
        topk_logits, topk_idx = logits.topk(top_k, dim=-1)
        topk_w = (F.softmax(topk_logits, dim=-1) if normalize
                  else F.softmax(logits, dim=-1).gather(1, topk_idx))
    if normalize and top_k > 1 and probs is not None:
        topk_w = topk_w / topk_w.sum(dim=-1, keepdim=True)
    return topk_w.to(out_dtype), topk_idx, probs


def balance_loss(probs: torch.Tensor, counts: torch.Tensor, coef: float, E: int) -> torch.Tensor:
    """router.py:100-111."""
    f = counts.float() / counts.sum().clamp(min=1)
    return coef * E * (f * probs.mean(0)).sum()


# ---- plan / dispatch (moe.py:208-223) -------------------------------------------------------

def plan(topk_idx: torch.Tensor, E: int):
    """(experts, order, token_idx, counts) of the stable sort (moe.py:220-222)."""
    k = topk_idx.shape[-1]
    experts, order = topk_idx.reshape(-1).sort(stable=True)
    token_idx = order.div(k, rounding_mode="floor")
    counts = torch.searchsorted(experts, torch.arange(E + 1, dtype=torch.long)).diff()
    return experts, order, token_idx, counts


def dispatch_buffers(topk_idx: torch.Tensor, E: int, align: int):
    """
    The dispatch buffers of moe_dispatch (moe_kernel.py:180-209), filled with the stable
    permutation of `plan`: (sorted_ids [l_cap], expert_ids [l_cap/align], offs [E+1],
    counts [E], n_post_pad, inv [M]).  Pure index arithmetic on the plan's output.
    """
    flat = topk_idx.reshape(-1)
    M = flat.numel()
    if M == 0:
        return (torch.zeros(0, dtype=torch.int32), torch.zeros(0, dtype=torch.int32),
                torch.zeros(E + 1, dtype=torch.int32), torch.zeros(E, dtype=torch.int32), 0,
                torch.zeros(0, dtype=torch.int32))
    _, order, _, counts = plan(topk_idx, E)
    padded = (counts + align - 1) // align * align
    offs = torch.zeros(E + 1, dtype=torch.long)
    offs[1:] = padded.cumsum(0)
    npp = int(offs[-1])
    l_cap = -(-(M + min(E, M) * (align - 1)) // align) * align
    sids = torch.full((l_cap,), M, dtype=torch.long)
    inv = torch.empty(M, dtype=torch.long)
    start = torch.cumsum(counts, 0) - counts
    for e in range(E):
        c = int(counts[e])
        if c:
            run = order[int(start[e]): int(start[e]) + c]
            sids[int(offs[e]): int(offs[e]) + c] = run
            inv[run] = torch.arange(int(offs[e]), int(offs[e]) + c)
    eids = torch.zeros(l_cap // align, dtype=torch.long)
    for b in range(npp // align):
        eids[b] = int((offs[:E] <= b * align).sum()) - 1
    return (sids.int(), eids.int(), offs.int(), counts.int(), npp, inv.int())


# ---- experts (moe.py:285-329, 394-418) ------------------------------------------------------

def _glu(act, gate, up):
    return act(gate) * up


def _expert(x, W_in, W_out, b_in, b_out, act):
    h = x @ W_in
    if b_in is not None:
        h = h + b_in
    gate, up = h.chunk(2, dim=-1)
    y = _glu(act, gate, up) @ W_out
    if b_out is not None:
        y = y + b_out
    return y


def shared(x: torch.Tensor, p: Params, act) -> Optional[torch.Tensor]:
    """moe.py:310-329: sum of the always-on experts (None when there are none)."""
    if p.W_sh_in is None:
        return None
    out = None
    for s in range(p.W_sh_in.shape[0]):
        y = _expert(x, p.W_sh_in[s], p.W_sh_out[s],
                    None if p.b_sh_in is None else p.b_sh_in[s],
                    None if p.b_sh_out is None else p.b_sh_out[s], act)
        out = y if out is None else out + y
    return out


def eager_forward(x: torch.Tensor, p: Params, topk_w: torch.Tensor, topk_idx: torch.Tensor,
                  activation: str = "silu") -> torch.Tensor:
    """
    The reference's ragged eager loop (moe.py:394-418) in x's dtype, given the routing:
    per-expert GEMMs, y * w, index_add_ in expert order, then + shared experts.
    """
    act = ACTS[activation]
    E = p.W_in.shape[0]
    _, order, token_idx, counts = plan(topk_idx, E)
    sizes = counts.tolist()
    xs = x.index_select(0, token_idx).split(sizes)
    ws = topk_w.reshape(-1).index_select(0, order).split(sizes)
    idx = token_idx.split(sizes)
    W_in, W_out = p.W_in.unbind(0), p.W_out.unbind(0)
    b_in = p.b_in.unbind(0) if p.b_in is not None else None
    b_out = p.b_out.unbind(0) if p.b_out is not None else None
    out = torch.zeros_like(x)
    for e, (x_e, i_e, w_e) in enumerate(zip(xs, idx, ws)):
        if x_e.shape[0] == 0:
            continue
        y = _expert(x_e, W_in[e], W_out[e], None if b_in is None else b_in[e],
                    None if b_out is None else b_out[e], act)
        out.index_add_(0, i_e, y * w_e[:, None])
    sh = shared(x, p, act)
    return out if sh is None else out + sh


def fp32_forward(x: torch.Tensor, p: Params, topk_w: torch.Tensor, topk_idx: torch.Tensor,
                 activation: str = "silu") -> torch.Tensor:
    """eager_forward with every operand lifted to fp32 (the tolerance reference)."""
    p32 = p.to(dtype=torch.float32)
    return eager_forward(x.float(), p32, topk_w.float(), topk_idx, activation)


def dense_forward(x: torch.Tensor, p: Params, topk_w: torch.Tensor, topk_idx: torch.Tensor,
                  activation: str = "silu") -> torch.Tensor:
    """moe.py:459-474: all experts on all tokens, mixed by a dense [N, E] gate matrix."""
    act = ACTS[activation]
    E = p.W_in.shape[0]
    gates = torch.zeros(x.shape[0], E, dtype=x.dtype)
    gates.scatter_(1, topk_idx, topk_w.to(x.dtype))
    h = x @ p.W_in
    h = h if p.b_in is None else h + p.b_in[:, None, :]
    gate, up = h.chunk(2, dim=-1)
    y = _glu(act, gate, up) @ p.W_out
    y = y if p.b_out is None else y + p.b_out[:, None, :]
    out = torch.einsum("enf,ne->nf", y, gates)
    sh = shared(x, p, act)
    return out if sh is None else out + sh


# ---- the whole block, forward + backward -----------------------------------------------------

@dataclass
class BlockResult:
    out: torch.Tensor
    topk_w: torch.Tensor
    topk_idx: torch.Tensor
    probs: Optional[torch.Tensor]
    counts: torch.Tensor
    aux_loss: torch.Tensor
    grads: dict = field(default_factory=dict)


def block(x: torch.Tensor, p: Params, top_k: int, *, train: bool = True,
          normalize: bool = True, aux_coef: float = 1e-2, activation: str = "silu",
          grad_out: Optional[torch.Tensor] = None, fp32: bool = False,
          logit_bias: Optional[torch.Tensor] = None,
          logits: Optional[torch.Tensor] = None) -> BlockResult:
    """
    MoEBlock.forward (moe.py:345-418) on CPU, optionally with the backward of
    (out * grad_out).sum() + aux_loss.

    fp32=False: the reference's own arithmetic in x's dtype (bf16 rounding points).
    fp32=True:  the same routing -- logits from the module-dtype GEMM, gates rounded to
    the module dtype exactly as router.py:98 does -- but every expert GEMM, the combine
    and every gradient in fp32 on the same (bf16-valued) inputs.  The router GEMM's
    gradient is taken in fp32 too (straight-through on the bf16 logit values).
    `logits` overrides the router GEMM's value; `logit_bias` is a harness-level
    per-expert offset (skewed routing).
    """
    E = p.W_in.shape[0]
    dt = x.dtype
    want_grad = grad_out is not None
    leaves = {}
    lift = (lambda t: t.detach().clone().float()) if fp32 else (lambda t: t.detach().clone())
    xl = lift(x)
    named = {k: lift(v) for k, v in p.named().items()}
    if want_grad:
        xl.requires_grad_(True)
        leaves["x"] = xl
        for k, v in named.items():
            v.requires_grad_(True)
            leaves[k] = v
    pl = Params(**{f: named.get(f) for f in Params.__dataclass_fields__})

    if logits is not None:
        lg = logits.detach().clone().float()
        if want_grad:
            lg.requires_grad_(True)
            leaves["logits"] = lg
    elif fp32:
        val = (x.detach() @ p.W.detach()).float()          # router.py:69 in the module dtype
        g = xl @ pl.W
        lg = val + (g - g.detach())
    else:
        lg = router_logits(xl, pl.W)
    if logit_bias is not None:
        lg = lg + logit_bias
    want_probs = train and aux_coef != 0.0
    topk_w, topk_idx, probs = route_from_logits(lg, top_k, want_probs, normalize, dt)
    _, _, _, counts = plan(topk_idx, E)
    aux = (balance_loss(probs, counts, aux_coef, E) if probs is not None
           else torch.zeros((), dtype=dt))
    if fp32:
        out = eager_forward(xl, pl, topk_w.float(), topk_idx, activation)
    else:
        out = eager_forward(xl, pl, topk_w, topk_idx, activation)
    res = BlockResult(out.detach(), topk_w.detach(), topk_idx, None if probs is None
                      else probs.detach(), counts, aux.detach())
    if want_grad:
        loss = (out.float() * grad_out.float()).sum() + aux.float()
        loss.backward()
        res.grads = {k: v.grad for k, v in leaves.items()}
    return res


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float):
    """(xn, rstd): F.rms_norm's arithmetic (ln.py:30-36) written out -- fp32 rstd =
    1 / sqrt(mean(x^2) + eps), xn = (x rstd) w in fp32, rounded once to x's dtype."""
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * rstd * w.float()).to(x.dtype), rstd.squeeze(-1)


def rms_norm_backward(g: torch.Tensor, x: torch.Tensor, w: torch.Tensor, rstd: torch.Tensor):
    """(dx, dw) of rms_norm for the output gradient g, in fp32: with xh = x rstd and
    gxh = g w, dx = (gxh - xh mean(xh gxh)) rstd and dw = sum over tokens of g xh."""
    gf, xf, wf = g.float(), x.float(), w.float()
    r = rstd.float().unsqueeze(-1)
    xh = xf * r
    gxh = gf * wf
    dx = (gxh - xh * (xh * gxh).mean(-1, keepdim=True)) * r
    return dx, (gf * xh).sum(0)


def flops_per_token(d: int, H: int, k: int, n_shared: int, E: int) -> int:
    """Forward FLOPs per token: routed + shared expert GEMMs and the router GEMM."""
    per_pair = 2 * d * 2 * H + 2 * H * d
    return (k + n_shared) * per_pair + 2 * d * E


def nanospeaker_config() -> dict:
    """nanoSpeaker's MoE block (nanospeaker.py:133-136; glu.py:26): d 576, E 76 + 2, k 6, H 128."""
    return dict(d=576, E=76, d_ff=192, n_shared=2, top_k=6)


def is_close(a: torch.Tensor, b: torch.Tensor, max_abs: float, rel_l2: float):
    """(ok, max abs err, rel-L2 err) of a against b in fp64."""
    a, b = a.double(), b.double()
    err = (a - b).abs().max().item() if a.numel() else 0.0
    denom = b.norm().item()
    rl2 = (a - b).norm().item() / denom if denom > 0 else (a - b).norm().item()
    return (err <= max_abs and rl2 <= rel_l2), err, rl2


__all__ = [name for name in dir() if not name.startswith("_")] + ["math"]
