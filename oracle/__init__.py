"""CPU oracle for the contrastive-loss hot path — TEST INFRASTRUCTURE ONLY.

A plain fp64 restatement of b0nce/MemoryEfficientCLIP's loss and gradients
(clip_loss.py, lit_loss.py), used to check the HIP library.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline); the product
path (``memoryefficientclip_amd``) never calls it.

Pinning (how each function is checked independently of its own formula; all
in ``tests/test_oracle.py``):

* ``clip_forward`` / ``lit_forward`` (fixed-max sums and loss epilogue):
  against ``F.cross_entropy`` on dense logits (library route), against a
  pure-Python log-softmax brute force on tiny inputs, and against the closed
  forms N=1 -> 0, identical unit rows -> ln N, orthonormal rows ->
  ln(1 + (N-1) e^{-1/T}).
* ``clip_backward`` / ``lit_backward`` (closed-form gradient matrix): against
  ``torch.autograd`` through the library route, ``torch.autograd.gradcheck``
  (finite differences) and pure-Python central differences.
* ``normalize`` / ``normalize_backward``: against ``F.normalize`` and its
  autograd, including the clamped (||x|| < eps) case.
* the Stable scaling and ``grad_output``: same loss, gradients times
  sqrt(N T) / times g (invariants, checked against the standard path).
* chunked helpers (``row_sums``, ``col_sums``, ``grad_rows``): against the
  dense functions on the same inputs.

The reference ships no tests, fixtures or golden vectors for this path, so
nothing here is pinned by reference-provided data; the committed fixtures in
``tests/golden/`` are produced by the library route above.
"""
from .contrastive import (  # noqa: F401
    EPS,
    clip_backward,
    clip_forward,
    clip_loss_and_grads,
    col_sums,
    grad_rows,
    lit_backward,
    lit_forward,
    lit_loss_and_grads,
    normalize,
    normalize_backward,
    row_sums,
    similarity_sums,
)
