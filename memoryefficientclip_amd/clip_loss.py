"""Drop-in CLIP loss: same classes, signatures and return values as the
reference's ``clip_loss.py`` (b0nce/MemoryEfficientCLIP), computed by the
gfx950 HIP kernels of ``libmec.so``.

    from memoryefficientclip_amd.clip_loss import MemoryEfficientCLIPLoss
    loss = MemoryEfficientCLIPLoss(temperature=0.07)(image_features, text_features)

Loss:  0.5 * (CE(S/T, arange N) + CE(S^T/T, arange N)),  S = norm(image) norm(text)^T.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _function as _f
from ._lib import MODE_CLIP


class MemoryEfficientCLIPLossNormed(torch.autograd.Function):
    """CLIP loss on already-normalised features (clip_loss.py:159-256).

    ``apply(x_normalized, y_normalized, temperature=0.07)`` returns a 0-d fp32
    loss; ``backward`` returns ``(dX, dY, None)`` with
    dX = (P_row + P_col)/(2NT) Y - Y/(NT) and dY likewise (clip_loss.py:115-156,
    :235-236).
    """

    @staticmethod
    def forward(ctx, x_normalized, y_normalized, temperature=0.07):
        return _f.forward(ctx, x_normalized, y_normalized, temperature, MODE_CLIP, False, False)

    @staticmethod
    def backward(ctx, grad_output):
        dx, dy = _f.backward(ctx, grad_output, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return dx, dy, None


class MemoryEfficientCLIPLoss(nn.Module):
    """clip_loss.py:259-273.  ``forward(image_features, text_features)``.

    With ``normalized_inputs=False`` the L2 normalisation (``F.normalize(dim=1)``
    in the reference) is fused into the kernels' load and store paths.
    """

    def __init__(self, temperature=0.07, normalized_inputs=False):
        super().__init__()
        self.temperature = temperature
        self.normalized_inputs = normalized_inputs

    def forward(self, image_features, text_features):
        if self.normalized_inputs:
            return MemoryEfficientCLIPLossNormed.apply(image_features, text_features, self.temperature)
        return _f.ContrastiveLossFn.apply(image_features, text_features, self.temperature, MODE_CLIP, True, False)


class StableMemoryEfficientCLIPLossNormed(torch.autograd.Function):
    """clip_loss.py:276-373: the same loss; gradients scaled by sqrt(N T)
    (the kernels use sqrt(N/T) in place of 1/T, clip_loss.py:299)."""

    @staticmethod
    def forward(ctx, x_normalized, y_normalized, temperature=0.07):
        return _f.forward(ctx, x_normalized, y_normalized, temperature, MODE_CLIP, False, True)

    @staticmethod
    def backward(ctx, grad_output):
        dx, dy = _f.backward(ctx, grad_output, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return dx, dy, None


class StableMemoryEfficientCLIPLoss(nn.Module):
    """clip_loss.py:376-401.

    Gradients come out sqrt(batch * temperature) times those of the standard
    loss (1/(N T) underflows in fp32 for very large batches); to mimic the
    standard CLIP update, scale the learning rate by 1/sqrt(batch * T).
    """

    def __init__(self, temperature=0.07, normalized_inputs=False):
        super().__init__()
        self.temperature = temperature
        self.normalized_inputs = normalized_inputs

    def forward(self, image_features, text_features):
        if self.normalized_inputs:
            return StableMemoryEfficientCLIPLossNormed.apply(image_features, text_features, self.temperature)
        return _f.ContrastiveLossFn.apply(image_features, text_features, self.temperature, MODE_CLIP, True, True)


__all__ = [
    "MemoryEfficientCLIPLossNormed",
    "MemoryEfficientCLIPLoss",
    "StableMemoryEfficientCLIPLossNormed",
    "StableMemoryEfficientCLIPLoss",
]
