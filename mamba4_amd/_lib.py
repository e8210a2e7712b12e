"""ctypes binding of the C ABI in include/mamba4_memread.h.

``load()`` opens the in-tree ``libmamba4_memread.so`` and raises if it is
missing: there is no fallback implementation.
"""

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libmamba4_memread.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "mamba4_memread.h")
HEADERS = [HEADER, os.path.join(os.path.dirname(HERE), "include", "mamba3_scan.h")]

EINVAL = 1
EHIP = 2
FACTOR_FLOATS = 2176
KEY_DIM = 64
SPD_MAX_DIM = 4096
VALUE_DIM = 64
MAX_VALUE_DIM = 128
MAX_CHUNK = 64
STATIC_SCRATCH_BYTES = 128 << 20  # M4MR_STATIC_SCRATCH_BYTES

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_S = ctypes.c_size_t

class MixerParams(ctypes.Structure):
    """m4mr_mixer_params (include/mamba4_memread.h)."""

    _fields_ = [
        ("beta_bias", ctypes.c_void_p),
        ("dt_bias", ctypes.c_void_p),
        ("a_log", ctypes.c_void_p),
        ("floor_raw", ctypes.c_void_p),
        ("previous", ctypes.c_void_p),
        ("confidence_scale", ctypes.c_void_p),
        ("skip", ctypes.c_void_p),
        ("beta_max", ctypes.c_float),
        ("floor_min", ctypes.c_float),
        ("key_shift", ctypes.c_int),
    ]


SIGNATURES = {
    "m4mr_version": (ctypes.c_char_p, []),
    "m4mr_last_error": (ctypes.c_char_p, []),
    "m4mr_forward": (_I, [_P] * 8 + [_I] * 5 + [_P] * 8 + [_P]),
    "m4mr_forward_bf16": (_I, [_P] * 8 + [_I] * 5 + [_P] * 8 + [_P]),
    "m4mr_mixer_forward": (
        _I,
        [_P] * 5 + [ctypes.POINTER(MixerParams)] + [_P] * 2 + [_I] * 5 + [_P] * 13 + [_P],
    ),
    "m4mr_backward_workspace_bytes": (_S, [_I] * 5),
    "m4mr_mixer_read_backward_workspace_bytes": (_S, [_I] * 5),
    "m4mr_mixer_read_backward": (
        _I,
        [_P] * 4 + [ctypes.POINTER(MixerParams)] + [_I] * 5 + [_P] * 9 + [_P] * 5 + [_P] * 14
        + [_P, _S, _P],
    ),
    "m4mr_mixer_backward": (
        _I,
        [_P] * 7 + [_I] * 6 + [_P] * 4 + [_P] * 4 + [_P] * 8 + [_P, _S, _P],
    ),
    "m4mr_start_counts": (_I, [_I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "m4mr_backward": (
        _I,
        [_P] * 6 + [_I] * 5 + [_P] * 4 + [_P] * 4 + [_P] * 8 + [_P, _S, _P],
    ),
    "m4mr_backward_bf16": (
        _I,
        [_P] * 6 + [_I] * 5 + [_P] * 4 + [_P] * 4 + [_P] * 8 + [_P, _S, _P],
    ),
    "m4mr_backward_noalloc": (
        _I,
        [_P] * 6 + [_I] * 5 + [_P] * 4 + [_P] * 4 + [_P] * 8 + [_P],
    ),
    "m4mr_factored_solve": (_I, [_P, _P, _P, _L, _P]),
    "m4mr_decode_step": (_I, [_P] * 8 + [_L, _I, _I, _P, _P, _P]),
    "m4mr_spd_solve": (_I, [_P, _P, _L, _I, _P, _P, _P]),
    "m4mr_spd_solve_backward": (_I, [_P, _P, _P, _L, _I, _P, _P, _P]),
    "m4mr_spd_factor_floats": (_L, [_I]),
    "m4mr_diagnostics": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "m4mr_prologue_forward": (_I, [_P] * 9 + [_I] * 4 + [ctypes.c_float] * 2 + [_I] + [_P] * 7),
    "m4mr_mixer_workspace_bytes": (_S, [_I] * 3),
    "m4mr_prologue_backward": (
        _I,
        [_P] * 9 + [_I] * 4 + [ctypes.c_float, _I] + [_P] * 6 + [_P] * 9 + [_P, _S, _P],
    ),
    "m4mr_epilogue_forward": (_I, [_P] * 5 + [_I] * 4 + [_P, _P]),
    "m4mr_epilogue_backward": (_I, [_P] * 5 + [_I] * 4 + [_P] * 6 + [_P, _S, _P]),
    "m4mr_order_workspace_bytes": (_S, [_I] * 5),
    "m4mr_order_forward": (_I, [_P] * 3 + [_I] * 5 + [_P, _P, _S, _P]),
    "m4mr_order_backward": (_I, [_P] * 5 + [_I] * 5 + [_P] * 4 + [_S, _P]),
    "m3s_forward": (_I, [_P] * 9 + [_I] * 6 + [_P] * 4 + [_P]),
    "m3s_backward_workspace_bytes": (_S, [_I] * 6),
    "m3s_backward": (_I, [_P] * 9 + [_I] * 6 + [_P] * 4 + [_P] * 9 + [_P, _S, _P]),
    "m3s_forward_bf16": (_I, [_P] * 9 + [_I] * 6 + [_P] * 4 + [_P]),
    "m3s_backward_bf16": (_I, [_P] * 9 + [_I] * 6 + [_P] * 4 + [_P] * 9 + [_P, _S, _P]),
    "m4mr_profile_enable": (None, [_I]),
    "m4mr_profile_select": (None, [ctypes.c_char_p]),
    "m4mr_profile_reset": (None, []),
    "m4mr_profile_read": (
        _I,
        [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_long)],
    ),
    "m4mr_profile_kernel_name": (ctypes.c_char_p, [_I]),
}

_lib = None


class MemreadError(RuntimeError):
    """A HIP launch failure reported by the library."""


def header_functions():
    """Names of the functions declared in include/mamba4_memread.h and
    include/mamba3_scan.h."""
    text = "".join(open(h).read() for h in HEADERS)
    pattern = r"^\s*(?:const\s+)?\w+\**\s+\**((?:m4mr|m3s)_\w+)\s*\("
    return sorted(set(re.findall(pattern, text, re.M)))


def load():
    """Open the HIP library (once) and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(
            f"{LIBRARY} is not built; run `python -m mamba4_amd.build` "
            "(the memory read has no non-HIP implementation)"
        )
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def check(rc):
    """Raise the library's last error for a non-zero return code."""
    if rc == 0:
        return
    message = load().m4mr_last_error().decode()
    if rc == EINVAL:
        raise ValueError(message)
    raise MemreadError(message)


def profile_enable(on=True):
    load().m4mr_profile_enable(1 if on else 0)


def profile_select(kernel=None):
    """Time only launches of `kernel` while profiling is on (None: every kernel)."""
    load().m4mr_profile_select(kernel.encode() if kernel else None)


def profile_reset():
    load().m4mr_profile_reset()


def profile_read(kernel):
    """(total milliseconds, launches) of one kernel since the last reset."""
    total = ctypes.c_double()
    count = ctypes.c_long()
    check(load().m4mr_profile_read(kernel.encode(), ctypes.byref(total), ctypes.byref(count)))
    return total.value, count.value


def start_counts(time, chunk):
    """(NC, NS): chunk start states and evidence start states for T tokens."""
    nc, ns = _I(), _I()
    check(load().m4mr_start_counts(time, chunk, ctypes.byref(nc), ctypes.byref(ns)))
    return nc.value, ns.value


def kernel_names():
    lib = load()
    names, i = [], 0
    while True:
        name = lib.m4mr_profile_kernel_name(i)
        if name is None:
            return names
        names.append(name.decode())
        i += 1
