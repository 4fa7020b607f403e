"""``lit_loss``: the reference module's name (b0nce/MemoryEfficientCLIP
``lit_loss.py``), re-exporting this package's LiT classes."""
from memoryefficientclip_amd.lit_loss import (  # noqa: F401
    MemoryEfficientLiTLoss,
    MemoryEfficientLiTLossNormed,
    StableMemoryEfficientLiTLoss,
    StableMemoryEfficientLiTLossNormed,
)
