"""MI355X-native (gfx950) memory-efficient CLIP / LiT contrastive loss.

Drop-in replacement for b0nce/MemoryEfficientCLIP's ``clip_loss`` and
``lit_loss`` modules: the same ``nn.Module`` and ``autograd.Function`` classes,
backed by hand-written HIP kernels in ``lib/libmec.so`` (C ABI:
``include/mec.h``).
"""
from .clip_loss import (
    MemoryEfficientCLIPLoss,
    MemoryEfficientCLIPLossNormed,
    StableMemoryEfficientCLIPLoss,
    StableMemoryEfficientCLIPLossNormed,
)
from .lit_loss import (
    MemoryEfficientLiTLoss,
    MemoryEfficientLiTLossNormed,
    StableMemoryEfficientLiTLoss,
    StableMemoryEfficientLiTLossNormed,
)

__version__ = "0.1.0"

__all__ = [
    "MemoryEfficientCLIPLoss",
    "MemoryEfficientCLIPLossNormed",
    "StableMemoryEfficientCLIPLoss",
    "StableMemoryEfficientCLIPLossNormed",
    "MemoryEfficientLiTLoss",
    "MemoryEfficientLiTLossNormed",
    "StableMemoryEfficientLiTLoss",
    "StableMemoryEfficientLiTLossNormed",
]
