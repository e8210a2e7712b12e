"""MI355X-native (gfx950) Mamba 4 memory read.

A drop-in for the reference's lm/kernels memory-read API
(``selective_gaussian_memory``, ``selective_decode``,
``selective_initial_state``, ``spd_solve``, ``SelectiveState``,
``SelectiveResult``),
implemented by hand-written HIP kernels behind the C ABI in
``include/mamba4_memread.h``.
"""

from mamba4_amd.memory import (  # noqa: F401
    MEMORY_SOLVE,
    SOLVERS,
    SelectiveResult,
    SelectiveState,
    selective_decode,
    selective_decode_,
    selective_gaussian_memory,
    selective_initial_state,
    spd_solve,
)

__all__ = [
    "MEMORY_SOLVE",
    "SOLVERS",
    "SelectiveResult",
    "SelectiveState",
    "selective_decode",
    "selective_decode_",
    "selective_gaussian_memory",
    "selective_initial_state",
    "spd_solve",
]
