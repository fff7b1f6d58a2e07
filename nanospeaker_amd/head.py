"""
The tied head with the next-token cross-entropy (reference: src/model/nanospeaker.py:236-250,
NanoSpeaker.forward with targets): loss = F.cross_entropy((h @ W.T).float(), y), the mean
over the targets that are not ignore_index, W the embedding matrix [V, d].

`linear_cross_entropy` is the drop-in for the reference's fused path
(LigerFusedLinearCrossEntropyLoss): the logits are formed in chunks of rows by a library
GEMM in the model's dtype (the values the reference's `h @ W.T` rounds to), the library's
HIP kernel (nsmoe_cross_entropy_rows) reduces each row once -- loss and, when a gradient is
needed, (softmax - onehot) / n written over the logits in place -- and two more library
GEMMs turn that into dh and dW during the forward, so the backward is a scale by the
upstream gradient.  A chunk is as many rows as `chunk_bytes` of logits hold: with 288 GB of
HBM the default 4 GiB takes the whole 4 x 8191-token batch of the reference's long-context
phase in one chunk (one GEMM each way, dW rounded once).  With several chunks dW is
accumulated in fp32 and rounded once at the end.

Off the GPU, or in fp32 / fp64, the same loss is the reference's own expression in torch.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _native as nat

_DT = {torch.bfloat16: nat.BF16, torch.float16: nat.F16}
CHUNK_BYTES = 4 << 30


def kernel_supported(h: Tensor, W: Tensor) -> bool:
    """The HIP loss takes 16-bit GPU tensors with a vocabulary that is a multiple of 8 and
    at most 65536."""
    V = W.shape[0]
    return (h.is_cuda and h.dtype in _DT and W.dtype == h.dtype and V % 8 == 0
            and V <= 65536)


def cross_entropy_rows(logits: Tensor, target: Tensor, ignore_index: int = -100,
                       n_valid: "Tensor | None" = None, grad: bool = False) -> Tensor:
    """Per-row losses [n] fp32 of 16-bit logits [n, V] (nsmoe_cross_entropy_rows); with
    `grad` the logits are overwritten by (softmax - onehot) / n_valid (n_valid: an int64
    device scalar)."""
    n, V = logits.shape
    assert logits.stride(1) == 1
    loss = torch.empty(n, dtype=torch.float32, device=logits.device)
    if grad and n_valid is None:
        raise ValueError("cross_entropy_rows: the gradient needs n_valid")
    tgt = target.to(torch.int64).contiguous()
    nat.check(nat.lib().nsmoe_cross_entropy_rows(
        _DT[logits.dtype], logits.data_ptr(), logits.stride(0), n, V, tgt.data_ptr(),
        int(ignore_index), None if n_valid is None else n_valid.data_ptr(), loss.data_ptr(),
        logits.data_ptr() if grad else None, torch.cuda.current_stream().cuda_stream),
        "nsmoe_cross_entropy_rows")
    return loss


class _LinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, W, y, ignore_index, chunk_rows):
        n, d = h.shape
        V = W.shape[0]
        need_h, need_W = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need = need_h or need_W
        n_valid = (y != ignore_index).sum()
        loss_rows = torch.empty(n, dtype=torch.float32, device=h.device)
        dh = torch.empty_like(h) if need_h else None
        dW32 = None
        dW = None
        nchunks = max(1, -(-n // chunk_rows))
        for c in range(nchunks):
            s, e = c * chunk_rows, min(n, (c + 1) * chunk_rows)
            if s >= e:
                break
            hc = h[s:e]
            logits = hc @ W.t()
            loss_rows[s:e] = cross_entropy_rows(logits, y[s:e], ignore_index, n_valid, need)
            if need_h:
                torch.mm(logits, W, out=dh[s:e])
            if need_W:
                part = logits.t() @ hc
                if nchunks == 1:
                    dW = part
                else:
                    dW32 = part.float() if dW32 is None else dW32.add_(part.float())
        if dW32 is not None:
            dW = dW32.to(W.dtype)
        ctx.save_for_backward(*(t for t in (dh, dW) if t is not None))
        ctx.has = (need_h, need_W)
        # every target ignored: 0 / 0, NaN, as F.cross_entropy's mean gives
        return loss_rows.sum() / n_valid.to(torch.float32)

    @staticmethod
    def backward(ctx, g):
        it = iter(ctx.saved_tensors)
        need_h, need_W = ctx.has
        dh = next(it) if need_h else None
        dW = next(it) if need_W else None
        if dh is not None:
            dh = dh * g.to(dh.dtype)
        if dW is not None:
            dW = dW * g.to(dW.dtype)
        return dh, dW, None, None, None


def linear_cross_entropy(h: Tensor, W: Tensor, y: Tensor, ignore_index: int = -100,
                         chunk_bytes: int = CHUNK_BYTES) -> Tensor:
    """mean cross-entropy of the logits h @ W.T [n, V] against y [n] (F.cross_entropy's
    semantics, ignore_index rows excluded from the mean); h [n, d], W [V, d]."""
    if not kernel_supported(h, W):
        return F.cross_entropy((h @ W.t()).float(), y, ignore_index=ignore_index)
    V = W.shape[0]
    chunk_rows = max(1, chunk_bytes // (V * h.element_size()))
    return _LinearCE.apply(h.contiguous(), W.contiguous(), y.contiguous(), ignore_index,
                           chunk_rows)
