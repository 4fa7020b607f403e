"""Top-level ``clip_loss`` / ``lit_loss`` module names for drop-in use.

The reference is used as ``from clip_loss import MemoryEfficientCLIPLoss`` and
``from lit_loss import MemoryEfficientLiTLoss`` (its README, lines 29 and 50).
This directory holds two small modules of those names that re-export this
package's classes, so a caller keeps that import unchanged by putting the
directory on the module search path: ``PYTHONPATH`` (``python -m
memoryefficientclip_amd.dropin`` prints it), a ``.pth`` file, or
``sys.path.insert(0, memoryefficientclip_amd.dropin.PATH)``.
"""
import os

PATH = os.path.dirname(os.path.abspath(__file__))
