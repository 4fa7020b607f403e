"""``python -m memoryefficientclip_amd.dropin`` prints the directory to put on
PYTHONPATH so that ``import clip_loss`` / ``import lit_loss`` load this
package's classes."""
from memoryefficientclip_amd.dropin import PATH

print(PATH)
