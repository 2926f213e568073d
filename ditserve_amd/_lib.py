"""Loader for libditk.so, the C-ABI library holding every HIP kernel.

The library is loaded with ctypes; each entry point takes raw device pointers,
sizes and a hipStream_t, and returns 0 or a status whose message
``ditk_last_error()`` holds.  There is no fallback: if the library is missing
or was not built, every op raises.
"""
import ctypes
import os
import pathlib

_PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = pathlib.Path(os.environ.get("DITK_LIB", _PKG / "libditk.so"))

c_void_p, c_int, c_int64, c_float = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_P = c_void_p


class AdalnJob(ctypes.Structure):
    """ditk_adaln_job of include/ditk.h."""
    _fields_ = [("x", _P), ("ldx", c_int64), ("y", _P), ("ldy", c_int64), ("cu_seqlens", _P), ("shift", _P),
                ("scale", _P), ("mod_stride", c_int64), ("weight", _P), ("bias", _P), ("T", c_int), ("D", c_int),
                ("nseg", c_int), ("norm_kind", c_int), ("eps", c_float)]


class QkNormJob(ctypes.Structure):
    """ditk_qk_norm_job of include/ditk.h."""
    _fields_ = [("q", _P), ("ldq", c_int64), ("k", _P), ("ldk", c_int64), ("q_out", _P), ("ldqo", c_int64),
                ("k_out", _P), ("ldko", c_int64), ("wq", _P), ("wk", _P), ("T", c_int), ("D", c_int),
                ("head_dim", c_int), ("per_head", c_int), ("eps", c_float)]

# name -> (restype, argtypes).  Mirrors include/ditk.h.
SIGNATURES = {
    "ditk_version": (c_int, []),
    "ditk_last_error": (ctypes.c_char_p, []),
    "ditk_adaln": (c_int, [_P, c_int64, _P, c_int64, c_int, c_int, _P, c_int, _P, _P, c_int64, _P, _P,
                           c_float, c_int, _P]),
    "ditk_modulation": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "ditk_qk_norm_rope": (c_int, [_P, c_int64, _P, c_int64, c_int, c_int, c_int, _P, _P, c_float, c_int, _P,
                                  _P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "ditk_qk_norm_rope_out": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, c_int, c_int, c_int, _P,
                                      _P, c_float, c_int, _P, _P, c_int, _P, _P, c_int, c_int, c_int, _P]),
    "ditk_gemm": (c_int, [_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int, c_int, c_int, c_int, _P, c_int64,
                          _P, c_int64, _P, c_int, _P]),
    "ditk_gemm_pair": (c_int, [_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int, _P, c_int64, _P, c_int64, _P, c_int,
                               _P, c_int64, _P, c_int64, _P, _P, c_int64, c_int, _P, c_int64, _P, c_int64, _P, c_int,
                               c_int, c_int, c_int, _P]),
    "ditk_vt_columns": (c_int64, [c_int64, c_int]),
    "ditk_transpose_v": (c_int, [_P, c_int64, _P, c_int64, c_int, c_int, c_int, _P, c_int, _P]),
    "ditk_flash_attn_varlen": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P,
                                       _P, c_int, c_int, c_int, c_int, c_float, _P]),
    "ditk_flash_attn_varlen_q_prescaled": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64,
                                                   _P, _P, c_int, c_int, c_int, c_int, _P]),
    "ditk_joint_attn_q_prescaled": (c_int, [_P, _P, c_int64, _P, _P, c_int64, _P, c_int64, _P, _P, c_int64,
                                            _P, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "ditk_transpose_v_joint": (c_int, [_P, _P, c_int64, _P, c_int64, c_int, c_int, c_int, _P, _P, _P, c_int, _P]),
    "ditk_patchify": (c_int, [_P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "ditk_unpatchify": (c_int, [_P, c_int64, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, _P]),
    "ditk_timestep_embedding": (c_int, [_P, _P, c_int, c_int, c_float, _P]),
    "ditk_cfg_combine": (c_int, [_P, _P, _P, c_int64, c_float, _P]),
    "ditk_joint_copy": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, _P, _P, c_int, c_int, c_int, c_int, _P]),
    "ditk_silu": (c_int, [_P, _P, c_int64, _P]),
    "ditk_adaln_multi": (c_int, [ctypes.POINTER(AdalnJob), c_int, _P]),
    "ditk_qk_norm_multi": (c_int, [ctypes.POINTER(QkNormJob), c_int, _P]),
    "ditk_check_cu_seqlens": (c_int, [_P, c_int, c_int, _P, _P, _P]),
    "ditk_solver_step": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, _P, _P]),
    "ditk_flash_attn_varlen_noalloc": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64,
                                               _P, _P, c_int, c_int, c_int, c_int, c_int, c_float, _P]),
}

_lib = None


class DitkError(RuntimeError):
    """A ditk entry point rejected its arguments or failed to launch."""


def load():
    """Load libditk.so (once) and bind every entry point; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise DitkError(f"{LIB_PATH} is not built: run `python -m ditserve_amd.build` "
                        "(the HIP path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    """Call entry point `name`; raise DitkError with the library's message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ditk_last_error().decode(errors="replace")
        raise DitkError(msg or f"{name} failed with status {rc}")
    return rc
