"""Mixture-of-Experts block (reference: src/model/moe.py), with the dropless path on HIP."""

import math

import torch
from torch import nn

from . import moe_kernel
from .glu import glu_hidden_dim, make_glu
from .moe_kernel import KERNEL_ACTIVATIONS, fused_moe_block_forward, kernel_supported
from .router import TopKRouter
from .utils import ACTIVATIONS, Activation, resolve_activation

# Capacity "auto" resolves to this where the fused kernels do not run.
AUTO_CAPACITY = 1.25


class MoEBlock(nn.Module):
    """
    Sparse MoE feed-forward with GLU experts; a drop-in for the reference MoEBlock --
    same constructor, parameters (W_in [E, d, 2H] gate|up, W_out [E, H, d], W_sh_in,
    W_sh_out, optional biases, router.W), RNG draw order, forward signature and side
    effects (`aux_loss`, `expert_counts`, `dropped`).

    The dropless path (capacity_factor None) runs wherever the reference would run its
    Triton kernels: a GPU tensor in bf16/fp16/fp32 with a named activation.  Routing,
    dispatch, the routed and shared experts and the combine are then HIP kernels, with
    the shared experts folded into the same grouped launch, and the backward is HIP too.
    There is no fallback for such tensors: a missing native library raises.

    The reference's other modes keep their semantics as plain torch code: the padded
    capacity path (capacity_factor set) and the eager ragged loop for what the kernels
    do not take (CPU tensors, fp64, custom callables, kernel=False).
    """

    def __init__(self, d_model: int, n_experts: int, d_ff: "int | None" = None,
                 top_k: int = 2, n_shared: int = 0,
                 capacity_factor: "float | None | str" = "auto",
                 activation: "str | Activation" = "silu", bias: bool = False,
                 normalize_weights: bool = True, aux_loss_coef: float = 1e-2,
                 noise_std: float = 0.0, fused: bool = True, kernel: bool = True,
                 std: float = 0.02):
        super().__init__()
        d_ff = d_ff if d_ff is not None else 4 * d_model
        self.d_model, self.n_experts, self.d_ff = d_model, n_experts, d_ff
        self.d_hidden = glu_hidden_dim(d_ff)
        self.top_k = top_k
        if n_shared < 0:
            raise ValueError(f"n_shared ({n_shared}) cannot be negative.")
        self.n_shared = n_shared
        if capacity_factor != "auto" and capacity_factor is not None and capacity_factor <= 0:
            raise ValueError(
                f"capacity_factor ({capacity_factor}) must be > 0, None, or \"auto\"."
            )
        self._capacity_setting = capacity_factor

        # Parameter creation order is the reference's (router.W, W_in, W_out, W_sh_in,
        # W_sh_out), so one seed gives both implementations the same weights.
        self.router = TopKRouter(d_model, n_experts, top_k, normalize_weights,
                                 aux_loss_coef, noise_std, std)
        self.activation, act = resolve_activation(activation)
        self.glu = make_glu(act, fused)

        # A name shadowed by a custom callable must not reach the kernel's epilogue.
        self.kernel = kernel
        self._kernel_act = (
            self.activation
            if ACTIVATIONS.get(self.activation) is act and self.activation in KERNEL_ACTIVATIONS
            else None
        )

        H = self.d_hidden
        self.W_in = nn.Parameter(torch.randn(n_experts, d_model, 2 * H) * std)
        self.W_out = nn.Parameter(torch.randn(n_experts, H, d_model) * std)
        self.b_in = nn.Parameter(torch.zeros(n_experts, 2 * H)) if bias else None
        self.b_out = nn.Parameter(torch.zeros(n_experts, d_model)) if bias else None
        self.W_sh_in = self.W_sh_out = self.b_sh_in = self.b_sh_out = None
        if n_shared:
            self.W_sh_in = nn.Parameter(torch.randn(n_shared, d_model, 2 * H) * std)
            self.W_sh_out = nn.Parameter(torch.randn(n_shared, H, d_model) * std)
            if bias:
                self.b_sh_in = nn.Parameter(torch.zeros(n_shared, 2 * H))
                self.b_sh_out = nn.Parameter(torch.zeros(n_shared, d_model))

        self.aux_loss = torch.zeros(())
        self.expert_counts = torch.zeros(n_experts)
        self.dropped = torch.zeros((), dtype=torch.long)
        self.register_buffer(
            "edges", torch.arange(n_experts + 1, dtype=torch.long), persistent=False
        )

    # ---- dispatch policy (reference: moe.py:181-206, 331-343) ----------------------------

    def _kernel_ready(self) -> bool:
        """Whether the fused path would take this block's own weights, as they sit now."""
        return (
            self.kernel
            and self._kernel_act is not None
            and kernel_supported(self.W_in)
            and moe_kernel.shape_supported(self.n_experts, self.n_shared, self.d_hidden,
                                           self.W_in.dtype)
        )

    @property
    def capacity_factor(self):
        """Effective capacity: "auto" is None where the kernels run, AUTO_CAPACITY elsewhere."""
        if self._capacity_setting != "auto":
            return self._capacity_setting
        return None if self._kernel_ready() else AUTO_CAPACITY

    def _use_kernel(self, x: torch.Tensor) -> bool:
        return (
            self.kernel and self._kernel_act is not None
            and self.capacity_factor is None and kernel_supported(x)
            and moe_kernel.shape_supported(self.n_experts, self.n_shared, self.d_hidden,
                                           x.dtype)
        )

    # ---- helpers shared with the reference's non-kernel modes -----------------------------

    def _plan(self, topk_idx: torch.Tensor):
        """Stable sort of the pairs by expert: (experts, order, token_idx, counts) (moe.py:208-223)."""
        experts, order = topk_idx.reshape(-1).sort(stable=True)
        token_idx = order.div(self.top_k, rounding_mode="floor")
        counts = torch.searchsorted(experts, self.edges).diff()
        return experts, order, token_idx, counts

    def _capacity(self, n_tokens: int) -> int:
        fair_share = n_tokens * self.top_k / self.n_experts
        return max(1, min(math.ceil(self.capacity_factor * fair_share), n_tokens * self.top_k))

    def _slots(self, experts, counts, cap: int):
        starts = counts.cumsum(0) - counts
        rank = torch.arange(experts.numel(), device=experts.device) - starts[experts]
        keep = rank < cap
        return torch.where(keep, experts * cap + rank, self.n_experts * cap), keep

    def _glu_expert(self, x, W_in, W_out, b_in, b_out):
        h = x @ W_in
        if b_in is not None:
            h = h + b_in
        gate, up = h.chunk(2, dim=-1)
        y = self.glu(gate, up) @ W_out
        if b_out is not None:
            y = y + b_out
        return y

    def _shared(self, x: torch.Tensor) -> torch.Tensor:
        out = None
        for s in range(self.n_shared):
            y = self._glu_expert(
                x, self.W_sh_in[s], self.W_sh_out[s],
                None if self.b_sh_in is None else self.b_sh_in[s],
                None if self.b_sh_out is None else self.b_sh_out[s])
            out = y if out is None else out + y
        return out

    def _forward_padded(self, x, experts, order, token_idx, counts, topk_w, shape):
        """Fixed-capacity dispatch (reference: moe.py:244-283)."""
        cap = self._capacity(x.shape[0])
        slot, keep = self._slots(experts, counts, cap)
        self.dropped = (~keep).sum().detach()
        xb = x.new_zeros(self.n_experts * cap + 1, self.d_model)
        xb.index_copy_(0, slot, x.index_select(0, token_idx))
        xb = xb[: self.n_experts * cap].view(self.n_experts, cap, self.d_model)
        h = xb @ self.W_in
        if self.b_in is not None:
            h = h + self.b_in[:, None, :]
        gate, up = h.chunk(2, dim=-1)
        y = self.glu(gate, up) @ self.W_out
        if self.b_out is not None:
            y = y + self.b_out[:, None, :]
        y = torch.cat((y.reshape(-1, self.d_model), y.new_zeros(1, self.d_model)))
        w = topk_w.reshape(-1).index_select(0, order)
        out = torch.zeros_like(x)
        out.index_add_(0, token_idx, y.index_select(0, slot) * w[:, None])
        if self.n_shared:
            out = out + self._shared(x)
        return out.view(shape)

    def _forward_eager(self, x, order, token_idx, counts, topk_w, shape):
        """Ragged per-expert loop (reference: moe.py:394-418)."""
        sizes = counts.tolist()
        xs = x.index_select(0, token_idx).split(sizes)
        ws = topk_w.reshape(-1).index_select(0, order).split(sizes)
        idx = token_idx.split(sizes)
        W_in, W_out = self.W_in.unbind(0), self.W_out.unbind(0)
        b_in = self.b_in.unbind(0) if self.b_in is not None else None
        b_out = self.b_out.unbind(0) if self.b_out is not None else None
        out = torch.zeros_like(x)
        for e, (x_e, i_e, w_e) in enumerate(zip(xs, idx, ws)):
            if x_e.shape[0] == 0:
                continue
            y = self._glu_expert(x_e, W_in[e], W_out[e],
                                 None if b_in is None else b_in[e],
                                 None if b_out is None else b_out[e])
            out.index_add_(0, i_e, y * w_e[:, None])
        if self.n_shared:
            out = out + self._shared(x)
        return out.view(shape)

    # ---- forward -------------------------------------------------------------------------

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.d_model:
            raise ValueError(f"expected last dim {self.d_model}, got {tuple(x.shape)}.")
        shape = x.shape
        x = x.reshape(-1, self.d_model)
        if x.shape[0] == 0:
            return x.clone().view(shape)
        if self._use_kernel(x) and self.router._on_kernel(x) and not (
                self.training and self.router.noise_std):
            # The whole block as one autograd node (router GEMM + HIP router tail,
            # dispatch, experts, combine, balance loss; HIP backward).
            out, aux, counts, topk_idx, logits = moe_kernel.block_forward(
                x, self.router.W, self.W_in, self.W_out, self.W_sh_in, self.W_sh_out,
                self.b_in, self.b_out, self.b_sh_in, self.b_sh_out, self.top_k,
                self.router.wants_probs(), self.router.normalize_weights, self._kernel_act,
                self.router.aux_loss_coef)
            self.expert_counts = counts.detach()
            self._routing = topk_idx  # the last call's expert ids and router logits,
            self._logits = logits     # for inspection
            self.aux_loss = aux
            return out.view(shape)

        topk_w, topk_idx, probs = self.router(x)

        if self._use_kernel(x):
            out, counts = fused_moe_block_forward(
                x, self.W_in, self.W_out, topk_w, topk_idx, self.b_in, self.b_out,
                self.W_sh_in, self.W_sh_out, self.b_sh_in, self.b_sh_out, self._kernel_act)
            self.expert_counts = counts.detach()
            self.aux_loss = (
                self.router.balance_loss(probs, counts) if probs is not None
                else torch.zeros((), device=x.device, dtype=x.dtype)
            )
            return out.view(shape)

        experts, order, token_idx, counts = self._plan(topk_idx)
        self.expert_counts = counts.detach()
        self.aux_loss = (
            self.router.balance_loss(probs, counts) if probs is not None
            else torch.zeros((), device=x.device, dtype=x.dtype)
        )
        if self.capacity_factor is not None:
            return self._forward_padded(x, experts, order, token_idx, counts, topk_w, shape)
        return self._forward_eager(x, order, token_idx, counts, topk_w, shape)

    def forward_residual(self, x: torch.Tensor, norm: nn.Module) -> torch.Tensor:
        """
        x + self(norm(x)): the FFN half of the reference's pre-norm Block.forward
        (src/model/nanospeaker.py:169), with `norm` an RMSNorm (ln.py:30-36: a `gamma`
        of shape [d_model] and `epsilon` or `eps`; F.rms_norm arithmetic).  On the kernel
        path, for 16-bit blocks in the fused router's shapes, the norm runs inside the
        router kernel and the residual add inside the combine, and the backward's norm
        gradient and residual add in one more kernel (nsmoe.h NSMOE_BLOCK_NORM); the
        side effects are those of forward().  Anything else is exactly those three ops.
        """
        gamma = getattr(norm, "gamma", None)
        eps = getattr(norm, "epsilon", getattr(norm, "eps", None))
        shape = x.shape
        x2 = x.reshape(-1, self.d_model)
        if (gamma is not None and eps is not None and getattr(norm, "fused", True)
                and tuple(gamma.shape) == (self.d_model,) and x2.shape[0]
                and self._use_kernel(x2) and self.router._on_kernel(x2)
                and not (self.training and self.router.noise_std)
                and moe_kernel.norm_fusable(x2.dtype, self.d_model, self.n_experts,
                                            self.top_k)):
            out, aux, counts, topk_idx, logits = moe_kernel.block_forward(
                x2, self.router.W, self.W_in, self.W_out, self.W_sh_in, self.W_sh_out,
                self.b_in, self.b_out, self.b_sh_in, self.b_sh_out, self.top_k,
                self.router.wants_probs(), self.router.normalize_weights, self._kernel_act,
                self.router.aux_loss_coef, norm_w=gamma, norm_eps=float(eps))
            self.expert_counts = counts.detach()
            self._routing = topk_idx
            self._logits = logits
            self.aux_loss = aux
            return out.view(shape)
        return x + self(norm(x))

    def dense_forward(self, x: torch.Tensor) -> torch.Tensor:
        """Every expert on every token, masked by the gates (reference: moe.py:420-474)."""
        if x.shape[-1] != self.d_model:
            raise ValueError(f"expected last dim {self.d_model}, got {tuple(x.shape)}.")
        shape = x.shape
        x = x.reshape(-1, self.d_model)
        topk_w, topk_idx, probs = self.router(x)
        experts, order, _, counts = self._plan(topk_idx)
        self.expert_counts = counts.detach()
        self.aux_loss = (
            self.router.balance_loss(probs, counts) if probs is not None
            else torch.zeros((), device=x.device, dtype=x.dtype)
        )
        if self.capacity_factor is not None and x.shape[0]:
            _, keep = self._slots(experts, counts, self._capacity(x.shape[0]))
            unsorted = torch.empty_like(keep).index_copy_(0, order, keep)
            self.dropped = (~keep).sum().detach()
            topk_w = topk_w * unsorted.view_as(topk_w)
        gates = torch.zeros(x.shape[0], self.n_experts, dtype=x.dtype, device=x.device)
        gates.scatter_(1, topk_idx, topk_w)
        h = x @ self.W_in
        h = h if self.b_in is None else h + self.b_in[:, None, :]
        gate, up = h.chunk(2, dim=-1)
        y = self.glu(gate, up) @ self.W_out
        y = y if self.b_out is None else y + self.b_out[:, None, :]
        out = (y * gates.t()[:, :, None]).sum(0)
        if self.n_shared:
            out = out + self._shared(x)
        return out.view(shape)
