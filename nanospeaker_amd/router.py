"""Token-choice top-k router (reference: src/model/router.py)."""

import torch
import torch.nn.functional as F
from torch import nn

from . import moe_kernel


class TopKRouter(nn.Module):
    """
    Softmax router sending each token to its top_k experts; same constructor, parameter
    (`W` [d_model, n_experts]) and outputs as the reference TopKRouter.

    MoEBlock's kernel path does not call this forward: there the logits GEMM x @ W, the
    softmax, top-k with CPU torch.topk's tie order, renormalisation, the cast and the
    dispatch histograms are one HIP kernel (`router_fwd_kernel`, through
    `moe_kernel.block_forward`), and the GEMM's backward runs in the block's backward
    kernels.  Called on its own (the reference's standalone router), the logits GEMM
    `(x @ W).float()` and the optional exploration noise run in torch, and on a GPU the
    tail is one HIP kernel (`moe_kernel.route`), its backward another.
    """

    def __init__(self, d_model: int, n_experts: int, top_k: int = 2,
                 normalize_weights: bool = True, aux_loss_coef: float = 1e-2,
                 noise_std: float = 0.0, std: float = 0.02):
        super().__init__()
        if min(d_model, n_experts, top_k) < 1:
            raise ValueError(
                f"d_model ({d_model}), n_experts ({n_experts}) and top_k ({top_k}) "
                f"must all be >= 1."
            )
        if top_k > n_experts:
            raise ValueError(f"top_k ({top_k}) cannot exceed n_experts ({n_experts}).")
        self.n_experts, self.top_k = n_experts, top_k
        self.normalize_weights = normalize_weights
        self.aux_loss_coef = aux_loss_coef
        self.noise_std = noise_std
        self.W = nn.Parameter(torch.randn(d_model, n_experts) * std)

    def wants_probs(self) -> bool:
        """Whether the full [N, E] softmax is consumed this step (the balance loss)."""
        return self.training and self.aux_loss_coef != 0.0

    def _on_kernel(self, x: torch.Tensor) -> bool:
        return (x.is_cuda and x.dtype in moe_kernel.KERNEL_DTYPES
                and self.n_experts <= moe_kernel.ROUTE_MAX_EXPERTS
                and moe_kernel.kernel_supported(x))

    def forward(self, x: torch.Tensor):
        """[N, d_model] -> (top-k weights [N, k] in x.dtype, expert ids [N, k], probs [N, E] or None)."""
        # Matmul in x's dtype; only the selection and the softmax are lifted to fp32
        # (reference: router.py:65-69).
        logits = (x @ self.W).float()
        if self.training and self.noise_std:
            logits = logits + torch.randn_like(logits) * self.noise_std

        want = self.wants_probs()
        if self._on_kernel(x):
            w, idx, probs = moe_kernel.route(
                logits, self.top_k, want, self.normalize_weights,
                moe_kernel.route_dtype_code(x.dtype))
            return w, idx, (probs if want else None)

        # Tensors the kernels do not take (CPU, fp64): the same arithmetic in torch ops.
        if want:
            probs = F.softmax(logits, dim=-1)
            topk_w, topk_idx = probs.topk(self.top_k, dim=-1)
        else:
            probs = None
            topk_logits, topk_idx = logits.topk(self.top_k, dim=-1)
            topk_w = (F.softmax(topk_logits, dim=-1) if self.normalize_weights
                      else F.softmax(logits, dim=-1).gather(1, topk_idx))
        if self.normalize_weights and self.top_k > 1 and probs is not None:
            topk_w = topk_w / topk_w.sum(dim=-1, keepdim=True)
        return topk_w.to(x.dtype), topk_idx, probs

    def balance_loss(self, probs: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
        """Switch-style balance loss coef * E * sum_e f_e * mean_t(probs[:, e]) (router.py:100-111)."""
        f = counts.float() / counts.sum().clamp(min=1)
        return self.aux_loss_coef * self.n_experts * (f * probs.mean(0)).sum()
