"""ctypes view of the C ABI in include/murmurative_hip.h.

``load()`` returns the CDLL of libmurmurative_hip.so with argument and result
types set for every declared entry point.  Import torch before calling it on
a GPU host so that the library binds to the HIP runtime torch already loaded.
``EXPORTS`` lists every symbol the header declares.
"""

import ctypes as C
import os

from ._hip_kernels import LIB_PATH

F32, F16, BF16 = 0, 1, 2
OK, ERR_ARG, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
NOALLOC_SCRATCH_BYTES = 64 << 20  # MURM_NOALLOC_SCRATCH_BYTES
TIMING_CLASSES = 10

_p, _i, _l, _d, _sz, _f = C.c_void_p, C.c_int, C.c_int64, C.c_double, C.c_size_t, C.c_float
_geom = [_i, _i, _i, _i, _i, _i, _i]           # dtype, slot_dtype, B, H, N, D, M
_view = [_p, _l, _l, _l]                       # ptr + three element strides
_view4 = [_p, _l, _l, _l, _l]                  # [B,H,N,M] view

SIGNATURES = {
    "murm_version": (C.c_char_p, []),
    "murm_last_error": (C.c_char_p, []),
    "murm_select_attend_workspace_bytes": (_sz, [_i] * 5),
    "murm_select_attend_fwd": (_i, _geom + _view * 3 + _view4 * 2 + [_i, _d, _i] + _view
                               + [_p, _p, _p, _sz, _p]),
    "murm_select_max_m": (_i, [_i, _i]),
    "murm_select_fwd": (_i, _geom + _view * 2 + _view4 * 2 + [_i, _i, _p, _p, _sz, _p]),
    "murm_attend_fwd": (_i, _geom + _view * 3 + [_p, _d] + _view + [_p, _p, _sz, _p]),
    "murm_select_attend_bwd_workspace_bytes": (_sz, [_i] * 5),
    "murm_select_attend_bwd": (_i, _geom + _view + [_p] + _view * 3 + [_p, _p, _d, _p, _p, _p, _p, _sz, _p]),
    "murm_slot_update_workspace_bytes": (_sz, [_i] * 5),
    "murm_slot_update_fwd": (_i, _geom + _view * 4 + [_p, _p, _d, _p, _sz, _p]),
    "murm_slot_update_bwd_workspace_bytes": (_sz, [_i] * 5),
    "murm_slot_update_bwd": (_i, _geom + _view * 4 + [_p, _p, _d, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "murm_slot_diffusion_fwd": (_i, [_i] * 5 + _view * 2 + [_d, _p]),
    "murm_slot_diffusion_bwd": (_i, [_i] * 5 + _view * 2 + [_d, _p, _p, _p]),
    "murm_slot_update_diffuse_fwd": (_i, _geom + _view * 4 + [_p, _p, _d, _d, _p, _sz, _p]),
    "murm_murmurate_workspace_bytes": (_sz, [_i] * 7),
    "murm_murmurate_fwd": (_i, [_i] * 8 + [_d, _d, _i, _i, _d] + _view * 6 + _view4 + _view
                           + [_p, _p, _p, _sz, _p]),
    "murm_murmurate_workspace_offset": (_l, [_i] * 9),
    "murm_murmurate_bwd_workspace_bytes": (_sz, [_i] * 7),
    "murm_murmurate_bwd": (_i, [_i] * 8 + [_d, _d, _d, _i] + _view + [_p] + _view * 3 + [_p, _p, _sz]
                           + _view * 3 + [_p, _p, _p, _sz, _p]),
    "murm_graph_replay": (None, [_i]),
    "murm_graph_cached": (_i, []),
    "murm_timing_enable": (None, [_i]),
    "murm_timing_reset": (None, []),
    "murm_timing_read": (_i, [_i, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "murm_timing_name": (C.c_char_p, [_i]),
    "murm_selftest_mfma": (_i, [_p, _p]),
    "murm_select_attend_fwd_noalloc": (_i, _geom + _view * 3 + _view4 * 2 + [_i, _d, _i] + _view + [_p, _p, _p]),
}
EXPORTS = tuple(SIGNATURES)

_lib = None


def load(path: str = LIB_PATH):
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python murmurative-attention_amd/build.py`")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


def check(rc: int, what: str = "murmurative_hip"):
    if rc != OK:
        msg = load().murm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def graph_replay(on: bool = True):
    """Replay the fused rounds' kernels from captured hipGraphs (see the header)."""
    load().murm_graph_replay(1 if on else 0)


def timing_enable(on: bool = True):
    load().murm_timing_enable(1 if on else 0)


def timing_reset():
    load().murm_timing_reset()


def timing_read():
    """{class name: (total_ms, launches)} for every kernel class with launches."""
    lib = load()
    out = {}
    for c in range(TIMING_CLASSES):
        ms, n = C.c_double(0.0), C.c_int64(0)
        check(lib.murm_timing_read(c, C.byref(ms), C.byref(n)), "murm_timing_read")
        if n.value:
            out[lib.murm_timing_name(c).decode()] = (ms.value, n.value)
    return out
