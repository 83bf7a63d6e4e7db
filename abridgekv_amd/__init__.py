"""MI355X-native abridged-KV attention path (HIP kernels for gfx950 behind a C-ABI library).

Importing the package registers the kernels as torch custom ops (``torch.ops.abridgekv.*``).
"""
from . import torch_ops  # noqa: F401
