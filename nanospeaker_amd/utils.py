"""Gate activations by name (reference: src/model/utils.py:10-40)."""

from typing import Callable

import torch

Activation = Callable[[torch.Tensor], torch.Tensor]

# In a GLU these name the variants: silu/swish -> SwiGLU, gelu -> GEGLU, relu -> ReGLU,
# sigmoid -> the original GLU.
ACTIVATIONS: "dict[str, Activation]" = {
    "silu": torch.nn.functional.silu,
    "swish": torch.nn.functional.silu,
    "gelu": torch.nn.functional.gelu,
    "relu": torch.nn.functional.relu,
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
}


def resolve_activation(activation: "str | Activation") -> "tuple[str, Activation]":
    """
    (name, fn) for an activation name or callable.  Names are case-insensitive; an
    unknown name raises ValueError rather than falling back to a default.
    """
    if callable(activation):
        return getattr(activation, "__name__", "custom"), activation
    if isinstance(activation, str) and activation.lower() in ACTIVATIONS:
        key = activation.lower()
        return key, ACTIVATIONS[key]
    raise ValueError(
        f"Unknown activation {activation!r}. Use a callable or one of: "
        f"{', '.join(sorted(ACTIVATIONS))}."
    )
