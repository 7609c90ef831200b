"""pgmoe: MI355X-native quantized MoE FFN layer for GGUF models.

``HipSparseMoEMLP`` is a drop-in for PyGGUF's ``GGUFSparseMoEMLP``
(pygguf_engine/model.py:849-937) and ``HipDenseMLP`` for its ``GGUFDenseMLP``
(model.py:778-846) on the same kernels; ``pgmoe.ops`` exposes the C-ABI stages.
"""

from .gguf import GGMLType, GGUFFile, GGUFWriter, InMemoryGGUF, MoEConfig
from .dense import HipDenseMLP
from .linear import FusedLinearPack, GGUFQuantLinear, HipQuantLinear
from .moe import HipSparseMoEMLP
from .norm import GGUFRMSNorm, HipRMSNorm, exec_fused_add_rmsnorm, exec_fused_rmsnorm

# The reference's class names, so `from pgmoe import GGUFSparseMoEMLP` swaps the block in.
GGUFSparseMoEMLP = HipSparseMoEMLP
GGUFDenseMLP = HipDenseMLP

__all__ = ["GGMLType", "GGUFFile", "GGUFWriter", "InMemoryGGUF", "MoEConfig", "HipSparseMoEMLP",
           "GGUFSparseMoEMLP", "HipDenseMLP", "GGUFDenseMLP", "GGUFRMSNorm", "HipRMSNorm",
           "exec_fused_add_rmsnorm", "exec_fused_rmsnorm", "GGUFQuantLinear", "HipQuantLinear",
           "FusedLinearPack"]
