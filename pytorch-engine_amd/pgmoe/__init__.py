"""pgmoe: MI355X-native quantized MoE FFN layer for GGUF models.

``HipSparseMoEMLP`` is a drop-in for PyGGUF's ``GGUFSparseMoEMLP``
(pygguf_engine/model.py:849-937); ``pgmoe.ops`` exposes the C-ABI stages.
"""

from .gguf import GGMLType, GGUFFile, GGUFWriter, InMemoryGGUF, MoEConfig
from .moe import HipSparseMoEMLP

# The reference's class name, so `from pgmoe import GGUFSparseMoEMLP` swaps the block in.
GGUFSparseMoEMLP = HipSparseMoEMLP

__all__ = ["GGMLType", "GGUFFile", "GGUFWriter", "InMemoryGGUF", "MoEConfig", "HipSparseMoEMLP",
           "GGUFSparseMoEMLP"]
