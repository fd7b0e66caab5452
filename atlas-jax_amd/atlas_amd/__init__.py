"""atlas_amd: the Atlas memory-layer chunk scan on MI355X (gfx950).

Host-side mirror of the rkstgr/atlas-jax memory-layer / model-forward API over
the C-ABI HIP library libatlas_hip.so (include/atlas_scan.h).
"""

from .config import AtlasConfig
from .memory_layer import (
    POLAR_EXPRESS_COEFFS,
    AtlasMemoryLayer,
    DeepMemoryState,
    LinearMemoryState,
    ShortConv,
    fused_chunk_scan,
    fused_polar_express,
    init_memory_state,
    linear_scan,
    memory_scan,
    polar_express,
    polar_express_ste,
    rms_norm,
)
from .model import MLP, Atlas, Block, initial_memory_states
from .mag import MAGBlock, MAGTransformer, MemoryGate, RotaryEmbedding, SlidingWindowAttention, swa_attention
from .optim import Muon, MuonState, muon_leaf_init, muon_leaf_update, muon_polar_express
from .checkpoint import load_checkpoint, save_checkpoint
from ._lib import AtlasError, get_lib

__all__ = [
    "AtlasConfig", "POLAR_EXPRESS_COEFFS", "AtlasMemoryLayer", "DeepMemoryState", "LinearMemoryState",
    "ShortConv", "fused_chunk_scan", "fused_polar_express", "init_memory_state", "linear_scan",
    "memory_scan", "polar_express", "polar_express_ste", "rms_norm", "AtlasError", "get_lib",
    "MLP", "Block", "Atlas", "initial_memory_states",
    "Muon", "MuonState", "muon_leaf_init", "muon_leaf_update", "muon_polar_express",
    "RotaryEmbedding", "SlidingWindowAttention", "swa_attention", "MemoryGate", "MAGBlock", "MAGTransformer",
    "save_checkpoint", "load_checkpoint",
]
