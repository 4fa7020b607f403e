"""``clip_loss``: the reference module's name (b0nce/MemoryEfficientCLIP
``clip_loss.py``), re-exporting this package's CLIP classes."""
from memoryefficientclip_amd.clip_loss import (  # noqa: F401
    MemoryEfficientCLIPLoss,
    MemoryEfficientCLIPLossNormed,
    StableMemoryEfficientCLIPLoss,
    StableMemoryEfficientCLIPLossNormed,
)
