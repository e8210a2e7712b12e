"""MI355X-native (gfx950) Mamba 4 memory read.

A drop-in for the reference's lm/kernels memory-read API
(``selective_gaussian_memory``, ``selective_decode``,
``selective_initial_state``, ``spd_solve``, ``selective_diagnostics``,
``SelectiveState``, ``SelectiveResult``),
implemented by hand-written HIP kernels behind the C ABI in
``include/mamba4_memread.h``, plus the caller's preprocessing and read gating
(``memory_inputs``, ``gated_read``; lm/models/mamba4.py:183-237, 266-273)
and the order head's gated scan (``order_memory_chunked``, ``order_memory``;
lm/models/mamba4.py:46-95).
"""

from mamba4_amd.memory import (  # noqa: F401
    MEMORY_SOLVE,
    SOLVERS,
    SelectiveResult,
    SelectiveState,
    selective_decode,
    selective_decode_,
    selective_diagnostics,
    selective_gaussian_memory,
    selective_initial_state,
    spd_solve,
)
from mamba4_amd.mixer import (  # noqa: F401
    MemoryInputs,
    MixerRead,
    gated_read,
    memory_inputs,
    mixer_read,
)
from mamba4_amd.flashmamba import mamba3_fused  # noqa: F401
from mamba4_amd.order import order_memory, order_memory_chunked  # noqa: F401

__all__ = [
    "MEMORY_SOLVE",
    "MemoryInputs",
    "MixerRead",
    "SOLVERS",
    "SelectiveResult",
    "SelectiveState",
    "mamba3_fused",
    "gated_read",
    "memory_inputs",
    "mixer_read",
    "order_memory",
    "order_memory_chunked",
    "selective_decode",
    "selective_decode_",
    "selective_diagnostics",
    "selective_gaussian_memory",
    "selective_initial_state",
    "spd_solve",
]
