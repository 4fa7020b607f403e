"""Drop-in LiT loss: same classes, signatures and return values as the
reference's ``lit_loss.py`` (b0nce/MemoryEfficientCLIP), computed by the
gfx950 HIP kernels of ``libmec.so``.

    from memoryefficientclip_amd.lit_loss import MemoryEfficientLiTLoss
    loss = MemoryEfficientLiTLoss(temperature=0.07)(text_features, image_features)

Loss: CE(S/T, arange N) with S = norm(text) norm(image)^T (text rows); only
the text features receive a gradient (lit_loss.py:247).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _function as _f
from ._lib import MODE_LIT


class MemoryEfficientLiTLossNormed(torch.autograd.Function):
    """LiT loss on already-normalised features (lit_loss.py:151-247).

    ``apply(x_normalized=text, y_normalized=image, temperature=0.07)``;
    ``backward`` returns ``(dX, None, None)``.
    """

    @staticmethod
    def forward(ctx, x_normalized, y_normalized, temperature=0.07):
        return _f.forward(ctx, x_normalized, y_normalized, temperature, MODE_LIT, False, False)

    @staticmethod
    def backward(ctx, grad_output):
        dx, _ = _f.backward(ctx, grad_output, ctx.needs_input_grad[0], False)
        return dx, None, None


class MemoryEfficientLiTLoss(nn.Module):
    """lit_loss.py:250-263.  ``forward(text_features, image_features)``
    (text first); the normalisation is fused when ``normalized_inputs=False``."""

    def __init__(self, temperature=0.07, normalized_inputs=False):
        super().__init__()
        self.temperature = temperature
        self.normalized_inputs = normalized_inputs

    def forward(self, text_features, image_features):
        if self.normalized_inputs:
            return MemoryEfficientLiTLossNormed.apply(text_features, image_features, self.temperature)
        return _f.ContrastiveLossFn.apply(text_features, image_features, self.temperature, MODE_LIT, True, False)


class StableMemoryEfficientLiTLossNormed(torch.autograd.Function):
    """lit_loss.py:266-362: same loss, text gradient scaled by sqrt(N T)."""

    @staticmethod
    def forward(ctx, x_normalized, y_normalized, temperature=0.07):
        return _f.forward(ctx, x_normalized, y_normalized, temperature, MODE_LIT, False, True)

    @staticmethod
    def backward(ctx, grad_output):
        dx, _ = _f.backward(ctx, grad_output, ctx.needs_input_grad[0], False)
        return dx, None, None


class StableMemoryEfficientLiTLoss(nn.Module):
    """lit_loss.py:365-389.  The reference's forward calls
    ``StableMemoryEfficientLiTLoss.apply`` (lit_loss.py:387), i.e.
    ``nn.Module.apply``, and fails; this module runs the Stable LiT Function it
    was meant to call."""

    def __init__(self, temperature=0.07, normalized_inputs=False):
        super().__init__()
        self.temperature = temperature
        self.normalized_inputs = normalized_inputs

    def forward(self, text_features, image_features):
        if self.normalized_inputs:
            return StableMemoryEfficientLiTLossNormed.apply(text_features, image_features, self.temperature)
        return _f.ContrastiveLossFn.apply(text_features, image_features, self.temperature, MODE_LIT, True, True)


__all__ = [
    "MemoryEfficientLiTLossNormed",
    "MemoryEfficientLiTLoss",
    "StableMemoryEfficientLiTLossNormed",
    "StableMemoryEfficientLiTLoss",
]
