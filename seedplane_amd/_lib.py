"""ctypes binding of libseedplane_hip.so (the C ABI declared in include/seedplane_hip.h).

The shared library is built in-tree (seedplane_amd/build.py) and loaded from this package directory only.  There is
no fallback: if the library is missing or a call fails, an exception is raised.
"""
import atexit
import ctypes

import numpy as np
import os
from pathlib import Path

LIB_NAME = 'libseedplane_hip.so'
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

SP_OK, SP_EINVAL, SP_ENOMEM, SP_EHIP, SP_ESTATE, SP_ECAPACITY = range(6)
SP_FMT_F32, SP_FMT_F16, SP_FMT_Q8, SP_FMT_Q4 = range(4)
(SP_T_EMBED, SP_T_HEAD, SP_T_FINAL_NORM, SP_T_IN_NORM, SP_T_POST_NORM, SP_T_QKV, SP_T_QKV_BIAS, SP_T_O,
 SP_T_GATE_UP, SP_T_DOWN) = range(10)
SP_F_LOGITS, SP_F_ARGMAX, SP_F_GRAPH, SP_F_PERSISTENT, SP_F_UNFUSED, SP_F_FEED, SP_F_CHAIN = 1, 2, 4, 8, 16, 32, 64
SP_F_DEVCOLS = 128

# Every function the header declares, with its ctypes signature.
c_int, c_int32, c_size_t, c_uint64, c_float = ctypes.c_int, ctypes.c_int32, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float
c_int64 = ctypes.c_int64
c_void_p, c_char_p = ctypes.c_void_p, ctypes.c_char_p


class ModelDesc(ctypes.Structure):
    _fields_ = [('n_layers', c_int32), ('hidden', c_int32), ('n_heads', c_int32), ('n_kv_heads', c_int32),
                ('head_dim', c_int32), ('intermediate', c_int32), ('vocab', c_int32), ('weight_format', c_int32),
                ('tied_head', c_int32), ('max_tokens', c_int32), ('rms_eps', c_float), ('reserved0', c_float),
                ('inv_freq', ctypes.POINTER(c_float))]


class Token(ctypes.Structure):
    _fields_ = [('token', c_int32), ('seq', c_int32), ('pos', c_int32), ('slot', c_int32), ('ctx_lo', c_int32),
                ('ctx_hi', c_int32), ('tree_base', c_int32), ('tree_count', c_int32), ('tree_mask', c_uint64)]


assert ctypes.sizeof(Token) == 40

# the same layout as a numpy structured dtype (columns built in bulk)
TOKEN_DTYPE = np.dtype([(name, np.int32 if ctype is c_int32 else np.uint64) for name, ctype in Token._fields_])
assert TOKEN_DTYPE.itemsize == 40 and all(TOKEN_DTYPE.fields[n][1] == getattr(Token, n).offset for n, _ in Token._fields_)

SIGNATURES = {
    'sp_engine_create': (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(c_void_p)]),
    'sp_engine_destroy': (None, [c_void_p]),
    'sp_engine_last_error': (c_char_p, [c_void_p]),
    'sp_last_error': (c_char_p, []),
    'sp_engine_set_stream': (c_int, [c_void_p, c_void_p]),
    'sp_engine_load': (c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    'sp_engine_kv_reserve': (c_int, [c_void_p, c_int32, c_int32]),
    'sp_engine_kv_grow': (c_int, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    'sp_engine_forward': (c_int, [c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p]),
    'sp_engine_logits': (c_int, [c_void_p, ctypes.POINTER(c_void_p)]),
    'sp_engine_kv_move': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    'sp_engine_sync': (c_int, [c_void_p]),
    'sp_engine_copy_ids': (c_int, [c_void_p, c_int32, c_void_p]),
    'sp_engine_last_path': (c_int, [c_void_p]),
    'sp_engine_persistent_status': (c_int, [c_void_p, c_char_p, c_int32]),
    'sp_persistent_geometry': (c_int, [ctypes.POINTER(ModelDesc), c_int32, c_int32, ctypes.POINTER(c_int32)]),
    'sp_engine_last_dispatches': (c_int, [c_void_p]),
    'sp_engine_time_persistent': (c_int, [c_void_p, ctypes.POINTER(Token), c_int32, ctypes.POINTER(c_float),
                                          ctypes.POINTER(c_uint64)]),
    'sp_engine_time_attention': (c_int, [c_void_p, c_int32, ctypes.POINTER(Token), c_int32, ctypes.POINTER(c_float),
                                         ctypes.POINTER(c_uint64)]),
    'sp_engine_bytes': (c_int, [c_void_p, ctypes.POINTER(c_uint64), ctypes.POINTER(c_uint64)]),
    'sp_engine_kv_fill': (c_int, [c_void_p, c_int32, c_int32, c_int32, c_uint64, c_float]),
    'sp_engine_time_gemv': (c_int, [c_void_p, c_int32, c_int32, c_int32, c_int32, ctypes.POINTER(c_float),
                                    ctypes.POINTER(c_uint64)]),
    'sp_tree_columns': (c_int, [c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int64, c_int32, c_int32, c_void_p]),
    'sp_op_argmax_workspace': (c_size_t, [c_int32, c_int32]),
    'sp_op_argmax': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    'sp_op_argmax_noalloc': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    'sp_weight_create': (c_int, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, ctypes.POINTER(c_void_p)]),
    'sp_weight_destroy': (None, [c_void_p]),
    'sp_weight_bytes': (c_uint64, [c_void_p]),
    'sp_pack_matrix': (c_int, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                               ctypes.POINTER(c_uint64), c_void_p, ctypes.POINTER(c_uint64)]),
    'sp_op_gemv_workspace': (c_size_t, [c_void_p, c_int32]),
    'sp_op_gemv': (c_int, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    'sp_op_sample': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_int32, ctypes.c_double, c_void_p,
                             c_void_p]),
    'sp_op_sample_filtered': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_int32, ctypes.c_double,
                                      c_int32, ctypes.c_double, c_void_p, c_void_p]),
    'sp_op_accept_tree': (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_int32, c_void_p, c_int32, ctypes.c_double, c_int32, c_void_p, c_void_p,
                                  c_void_p, c_void_p]),
    'sp_op_accept_tree_host': (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int32, c_void_p, c_int32, ctypes.c_double, c_int32, c_void_p,
                                       c_void_p, c_void_p]),
    'sp_op_accept_tree_rows': (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int32, ctypes.c_double,
                                       c_int32, c_void_p, c_void_p, c_void_p]),
    'sp_op_draft_link': (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    'sp_engine_set_device_columns': (c_int, [c_void_p, c_void_p, c_void_p]),
    'sp_library_release': (c_int, []),
    'sp_engine_kv_layer': (c_int, [c_void_p, c_int32, ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p)]),
}

_lib = None


def load():
    """Load the in-tree library once; raise ImportError with the build instruction when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get('SEEDPLANE_HIP_LIB', LIB_PATH))
    if not path.is_file():
        raise ImportError(f'{path} is not built: run `python -m seedplane_amd.build` (hipcc --offload-arch=gfx950)')
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    atexit.register(_release_at_exit)
    return lib


def _release_at_exit():
    """Free the library's per-device scratch (sp_library_release) at interpreter exit, while the HIP runtime is
    still whole: its own teardown runs later, in the C exit handlers.  Engines are freed by their finalizers."""
    if _lib is not None:
        _lib.sp_library_release()


class SeedPlaneError(RuntimeError):
    pass


def check(rc, engine=None):
    """Raise the Python exception class the reference raises for the same condition."""
    if rc == SP_OK:
        return
    lib = load()
    msg = (lib.sp_engine_last_error(engine) if engine else lib.sp_last_error()) or b''
    msg = msg.decode('utf-8', 'replace')
    if rc in (SP_EINVAL, SP_ECAPACITY):
        raise ValueError(msg)
    raise SeedPlaneError(f'seedplane_hip error {rc}: {msg}')


def require_gpu():
    """The HIP path is the only path: fail loudly without a GPU or without the library."""
    import torch
    load()
    if not torch.cuda.is_available():
        raise RuntimeError('seedplane_amd needs a ROCm GPU (gfx950); torch.cuda.is_available() is False')
