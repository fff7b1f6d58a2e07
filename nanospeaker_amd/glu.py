"""GLU expert body (reference: src/model/glu.py)."""

import torch
from torch import nn

from .utils import Activation, resolve_activation


def glu_hidden_dim(d_ff: int) -> int:
    """
    GLU hidden width for a d_ff-wide FFN budget: 2 * d_ff // 3, so the GLU's three
    matrices hold what the replaced FFN's two did (reference: glu.py:16-29).
    """
    d_hidden = 2 * d_ff // 3
    if d_hidden < 1:
        raise ValueError(f"d_ff ({d_ff}) is too small: 2/3 * d_ff rounds down to {d_hidden}.")
    return d_hidden


def make_glu(act: Activation, fused: bool = True, dynamic: "bool | None" = True):
    """(gate, up) -> act(gate) * up, torch.compile'd when `fused` (reference: glu.py:32-47)."""

    def glu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
        return act(gate) * up

    return torch.compile(glu, dynamic=dynamic) if fused else glu


class GLUFeedForward(nn.Module):
    """
    Dense GLU feed-forward: h = act(x @ W_gate) * (x @ W_up); y = h @ W_down, with gate
    and up packed side by side in W_in [d_model, 2 * d_hidden] (reference: glu.py:50-102).
    """

    def __init__(self, d_model: int, d_ff: "int | None" = None,
                 activation: "str | Activation" = "silu", bias: bool = False,
                 fused: bool = True, std: float = 0.02):
        super().__init__()
        d_ff = d_ff if d_ff is not None else 4 * d_model
        self.d_model = d_model
        self.d_hidden = glu_hidden_dim(d_ff)
        self.activation, act = resolve_activation(activation)
        self.glu = make_glu(act, fused, dynamic=None)
        self.W_in = nn.Parameter(torch.randn(d_model, 2 * self.d_hidden) * std)
        self.W_out = nn.Parameter(torch.randn(self.d_hidden, d_model) * std)
        self.b_in = nn.Parameter(torch.zeros(2 * self.d_hidden)) if bias else None
        self.b_out = nn.Parameter(torch.zeros(d_model)) if bias else None

    @staticmethod
    def _affine(x, W, b):
        if b is None:
            return x @ W
        return torch.addmm(b, x, W) if x.dim() == 2 else x @ W + b

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.d_model:
            raise ValueError(f"expected last dim {self.d_model}, got {tuple(x.shape)}.")
        gate, up = self._affine(x, self.W_in, self.b_in).chunk(2, dim=-1)
        return self._affine(self.glu(gate, up), self.W_out, self.b_out)
