"""grande_amd: an MI355X-native engine for omg's decision path.

One block-causal pass over a shared state prefix plus isolated question
branches, read out at the answer positions, on hand-written gfx950 HIP
kernels behind the C ABI in include/omg_hip.h (libomg_hip.so).
"""
from ._lib import OmgError
from .engine import (BranchOutput, BranchTokens, DeviceWeight, Engine, EngineBuilder, Group, GroupOutput, PointerHead,
                     PrefixSource, Role, Want, pack, state_check, state_key)
from .model import (BASELINE_CONFIGS, F16, GEMMA4_CONFIGS, LABEL_IDS, Q4, Q8, QTensor, Weights, config_json,
                    export_dir, gemma4_config_json, quantize)

__all__ = [
    "BASELINE_CONFIGS", "BranchOutput", "BranchTokens", "DeviceWeight", "Engine", "EngineBuilder", "F16", "Group",
    "GroupOutput", "LABEL_IDS", "OmgError", "PointerHead", "PrefixSource", "Q4", "Q8", "QTensor", "Role", "Want", "Weights", "config_json",
    "export_dir", "gemma4_config_json", "pack", "quantize", "state_check", "state_key",
]
