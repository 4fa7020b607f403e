"""Dense PyTorch CPU baseline of the contrastive loss — TEST INFRASTRUCTURE ONLY.

This is the reference's loss definition computed densely on host cores, the
baseline ``bench.py`` times beside the GPU path (never the thing measured or
shipped).  It restates the forward of ``clip_loss.py:159-213`` /
``lit_loss.py:151-205`` and the module glue ``clip_loss.py:259-273`` /
``lit_loss.py:250-263`` as dense fp32 tensor ops:

* ``F.normalize(dim=1)`` when ``normalized_inputs`` is False (clip_loss.py:266-268);
* logits S = x^ y^T / T (the fixed-max shift of clip_loss.py:56 cancels in the
  softmax, so plain cross-entropy is the same loss);
* CLIP: 0.5 (CE(S, arange) + CE(S^T, arange)); LiT: CE(S, arange) with text
  rows (clip_loss.py:206-211, lit_loss.py:199-203);
* ``loss.backward()`` for the gradients (clip_loss.py:215-256).

Its values are checked against the fp64 oracle in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import time

import torch
import torch.nn.functional as F


def dense_step(a: torch.Tensor, b: torch.Tensor, temperature: float, lit: bool, normalized_inputs: bool,
               times: dict | None = None):
    """One fwd+bwd of the dense loss on CPU tensors ``a`` (image for CLIP, text
    for LiT) and ``b``.  Returns (loss, grad_a, grad_b or None).  With
    ``times``, the forward and backward seconds are stored under "fwd" and
    "bwd"."""
    t0 = time.perf_counter()
    a = a.detach().float().requires_grad_(True)
    b = b.detach().float().requires_grad_(not lit)
    xh = a if normalized_inputs else F.normalize(a, dim=1)
    yh = b if normalized_inputs else F.normalize(b, dim=1)
    s = (xh @ yh.T) / temperature
    lab = torch.arange(a.shape[0])
    loss = F.cross_entropy(s, lab)
    if not lit:
        loss = 0.5 * (loss + F.cross_entropy(s.T, lab))
    t1 = time.perf_counter()
    loss.backward()
    t2 = time.perf_counter()
    if times is not None:
        times["fwd"] = t1 - t0
        times["bwd"] = t2 - t1
    return loss.detach(), a.grad, (None if lit else b.grad)
