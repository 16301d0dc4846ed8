"""MI355X-native (gfx950) graph beam search: a drop-in for the GPU search path of
SophiaSun18/beam_search_collab (modes base, warpN, bwarpN, rabitq).

    from beam_search_collab_amd import GPUGraph, GPUBaseSearchCfg, run_base
    from beam_search_collab_amd import host   # formats, builders, ground truth

The search runs only through libbs_hip.so (hand-written HIP for gfx950); importing the
search API raises if the library is missing.
"""
from .search import (  # noqa: F401
    BS_BASE, BS_GROUP, BS_GROUP_BLOOM, BS_RABITQ, INVALID_ID, MODES, BeamSearchError, GPUBaseSearchCfg,
    GPUGraph, GPURabitqSearchCfg, make_keys, run_base, run_rabitq, run_warp,
)
from . import host  # noqa: F401

__all__ = [
    "GPUGraph", "GPUBaseSearchCfg", "GPURabitqSearchCfg", "run_base", "run_warp", "run_rabitq", "MODES",
    "BS_BASE", "BS_GROUP", "BS_GROUP_BLOOM", "BS_RABITQ", "INVALID_ID", "BeamSearchError", "make_keys", "host",
]
