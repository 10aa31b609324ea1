"""ctypes binding of libg2v_hip.so, the gfx950 HIP library behind ``_C`` (C ABI: include/g2v.h).

Loading fails loudly: there is no CPU fallback for the G2V path.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libg2v_hip.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)

G2V_OK = 0
# the ABI that SIGNATURES describes (g2v_abi_version() of a matching build)
ABI_VERSION = 13
G2V_DTYPE_F32 = 0
G2V_DTYPE_BF16 = 1
_ERRORS = {1: "invalid argument", 2: "HIP runtime error", 3: "size limit exceeded"}

# (name, restype, argtypes) of every exported entry point of include/g2v.h
_vp, _i, _ll, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t
_f3 = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_llp = ctypes.POINTER(ctypes.c_longlong)
SIGNATURES = {
    "g2v_last_error": (ctypes.c_char_p, []),
    "g2v_abi_version": (_i, []),
    "g2v_grid_dims": (_i, [_f3, _f3, _ip, _ip]),
    "g2v_forward_plan_workspace": (_sz, [_i]),
    "g2v_forward_plan": (_i, [_i, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _llp, _vp, _sz, _llp,
                              _vp]),
    "g2v_forward_plan_async": (_i, [_i, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _vp, _vp]),
    "g2v_forward_splat_workspace": (_sz, [_i, _i, _ll, _f3, _f3]),
    "g2v_forward_packed_bytes": (_sz, [_i, _i]),
    "g2v_forward_pack_features": (_i, [_i, _i, _vp, _i, _vp, _sz, _vp]),
    "g2v_forward_splat": (_i, [_i, _i, _vp, _vp, _vp, _i, _vp, _sz, _f3, _f3, _vp, _vp, _vp, _vp, _ll, _vp, _vp,
                               _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "g2v_backward_plan_workspace": (_sz, [_i]),
    "g2v_backward_plan": (_i, [_i, _i, _f3, _f3, _vp, _vp, _vp, _sz, _llp, _vp]),
    "g2v_backward_workspace": (_sz, [_i, _i, _ll, _ll, _f3, _f3]),
    "g2v_backward": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp, _ll, _ll,
                          _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "g2v_backward_prepare": (_i, [_i, _i, _f3, _f3, _vp, _vp, _vp, _i, _ll, _ll, _vp, _vp, _vp, _vp, _sz, _vp]),
    "g2v_backward_prepared": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp, _ll, _ll,
                                   _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "g2v_backward_cosine": (_i, [_i, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp,
                                 _ll, _ll, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                 _i, _vp]),
    "g2v_t2g_workspace": (_sz, [_i, _ll, _f3, _f3]),
    "g2v_build_t2g": (_i, [_i, _f3, _f3, _vp, _vp, _vp, _vp, _ll, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                           _vp, _sz, _vp]),
    "g2v_batch_plan_workspace": (_sz, [_i, _i]),
    "g2v_batch_forward_plan": (_i, [_i, _i, _vp, _vp, _f3, _f3, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _vp, _vp]),
    "g2v_batch_forward_splat_workspace": (_sz, [_i, _i, _i, _ll, _f3, _f3]),
    "g2v_batch_forward_splat": (_i, [_i, _i, _i, _vp, _vp, _vp, _i, _f3, _f3, _vp, _vp, _vp, _vp, _sz, _ll, _vp,
                                     _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "g2v_batch_backward_workspace": (_sz, [_i, _i, _i, _ll, _ll, _f3, _f3]),
    "g2v_batch_backward_prepare": (_i, [_i, _i, _i, _f3, _f3, _vp, _vp, _vp, _i, _ll, _ll, _vp, _vp, _vp, _sz, _vp,
                                        _sz, _vp]),
    "g2v_batch_backward": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _f3, _f3, _vp, _vp, _ll, _ll, _vp, _vp, _vp,
                                _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _sz, _i, _vp]),
    "g2v_cosine_loss_workspace": (_sz, [_ll, _i]),
    "g2v_cosine_loss_forward": (_i, [_ll, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _ip, _vp, _sz, _vp]),
    "g2v_cosine_loss_forward_coef": (_i, [_ll, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _ip, _vp, _vp, _sz, _vp]),
    "g2v_cosine_loss_forward_noalloc": (_i, [_ll, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "g2v_cosine_loss_backward": (_i, [_ll, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "g2v_covariance_from_scale_rotation": (_i, [_i, _vp, _vp, _vp, _vp]),
    "g2v_covariance_from_scale_rotation_backward": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "g2v_profile_enable": (_i, [_i]),
    "g2v_profile_reset": (_i, []),
    "g2v_profile_collect": (_i, []),
    "g2v_profile_entry": (_i, [_i, ctypes.c_char_p, _i, _llp, ctypes.POINTER(ctypes.c_double)]),
}

_lib = None


def load():
    """Load (once) and return the ctypes handle of libg2v_hip.so."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python shelfgaussian-cudagaussianvoxelizer_amd/build.py); there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    # a library built from other sources would be called with mismatched argument lists: refuse it
    # before any entry point runs
    lib.g2v_abi_version.restype = ctypes.c_int
    lib.g2v_abi_version.argtypes = []
    got = lib.g2v_abi_version()
    if got != ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI {got}, this package expects {ABI_VERSION}: rebuild it "
                          "(python shelfgaussian-cudagaussianvoxelizer_amd/build.py)")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str):
    if rc != G2V_OK:
        msg = load().g2v_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({_ERRORS.get(rc, rc)}): {msg}")


def floats(values):
    vals = [float(v) for v in values]
    return (ctypes.c_float * len(vals))(*vals)


def profile_enable(on: bool = True):
    """Bracket every kernel launch of the library with HIP events (per-kernel timing)."""
    load().g2v_profile_enable(1 if on else 0)


def profile_reset():
    load().g2v_profile_reset()


def profile_report():
    """{kernel name: (launches, total ms)} accumulated since the last reset."""
    lib = load()
    n = lib.g2v_profile_collect()
    out = {}
    buf = ctypes.create_string_buffer(128)
    cnt = ctypes.c_longlong(0)
    ms = ctypes.c_double(0.0)
    for i in range(n):
        check(lib.g2v_profile_entry(i, buf, 128, ctypes.byref(cnt), ctypes.byref(ms)), "g2v_profile_entry")
        out[buf.value.decode()] = (int(cnt.value), float(ms.value))
    return out
