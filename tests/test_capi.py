"""The C ABI library: it loads, exports every function include/seedplane_hip.h declares with the signatures the
ctypes binding uses, and the struct layouts agree between C and ctypes.  No compute call needs a GPU here."""
import ctypes
import re
import subprocess
import tempfile
from pathlib import Path

import pytest

from seedplane_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / 'include' / 'seedplane_hip.h'


def declared_functions():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return set(re.findall(r'\b(sp_\w+)\s*\(', text))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 19
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert names == set(_lib.SIGNATURES), 'ctypes signatures and header out of sync'


def test_struct_layout_matches_c():
    src = r'''
    #include <stdio.h>
    #include <stddef.h>
    #include "seedplane_hip.h"
    int main(void) {
        printf("%zu %zu %zu %zu %zu\n", sizeof(sp_token), offsetof(sp_token, tree_mask), sizeof(sp_model_desc),
               offsetof(sp_model_desc, rms_eps), offsetof(sp_model_desc, inv_freq));
        return 0;
    }'''
    with tempfile.TemporaryDirectory() as d:
        c = Path(d) / 'layout.c'
        c.write_text(src)
        exe = Path(d) / 'layout'
        subprocess.run(['gcc', '-std=c99', '-I', str(HEADER.parent), str(c), '-o', str(exe)], check=True)
        out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    got = list(map(int, out))
    assert got == [ctypes.sizeof(_lib.Token), _lib.Token.tree_mask.offset, ctypes.sizeof(_lib.ModelDesc),
                   _lib.ModelDesc.rms_eps.offset, _lib.ModelDesc.inv_freq.offset]


def test_workspace_queries_are_pure_host_functions():
    lib = _lib.load()
    assert lib.sp_op_argmax_workspace(0, 10) == 0
    assert lib.sp_op_argmax_workspace(3, 151936) == 3 * 64 * 8
    assert lib.sp_op_gemv_workspace(None, 1) == 0


def test_library_release_without_scratch_is_a_host_no_op():
    # nothing was created on a device in this process: the release makes no HIP call and succeeds
    assert _lib.load().sp_library_release() == _lib.SP_OK


def test_new_entry_points_reject_bad_arguments_before_any_gpu_call():
    lib = _lib.load()
    assert lib.sp_op_draft_link(None, 8, 0, None, None, None, None) == _lib.SP_EINVAL
    d = ctypes.c_void_p(16)             # never dereferenced: the size check fails first
    assert lib.sp_op_draft_link(d, 16, 4, d, d, d, None) == _lib.SP_EINVAL       # 80 drafted nodes > 64
    assert b'64-bit' in lib.sp_last_error()
    assert lib.sp_engine_set_device_columns(None, None, None) == _lib.SP_EINVAL
    assert lib.sp_op_accept_tree_rows(None, None, 1, 10, 10, 1, None, None, None, None, 0, None, None, 1, 0.8, 1,
                                      None, None, None) == _lib.SP_EINVAL


def test_null_arguments_are_rejected_with_einval():
    lib = _lib.load()
    assert lib.sp_engine_create(None, None) == _lib.SP_EINVAL
    assert lib.sp_engine_forward(None, 1, None, 0, None, None) == _lib.SP_EINVAL
    assert b'NULL' in lib.sp_last_error()
    with pytest.raises(ValueError):
        _lib.check(_lib.SP_EINVAL)


def test_accept_tree_host_rejects_bad_arguments_before_any_gpu_call():
    """The host-array acceptance entry point checks its arrays and sizes before it touches the GPU."""
    lib = _lib.load()
    ints = (ctypes.c_int32 * 1024)()
    u = (ctypes.c_double * 4)(0.1, 0.2, 0.3, 0.4)
    p = lambda a: ctypes.cast(a, ctypes.c_void_p)
    out = (ctypes.c_int32 * 8)()

    def call(token=ints, n_nodes=3, n_trials_total=2, uu=u, n_u=4):
        return lib.sp_op_accept_tree_host(None, None, 1000, 1000, n_nodes, p(token) if token else None, p(ints),
                                          p(ints), p(ints), n_trials_total, p(uu) if uu else None, n_u, 0.8, 1,
                                          None, None, p(out))
    assert call(token=None) == _lib.SP_EINVAL
    assert call(uu=None) == _lib.SP_EINVAL
    assert call(n_nodes=0) == _lib.SP_EINVAL
    assert call(n_nodes=65) == _lib.SP_EINVAL
    assert call(n_trials_total=1025) == _lib.SP_EINVAL
    assert call(n_u=0) == _lib.SP_EINVAL


def test_engine_create_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip('a GPU is present')
    import numpy as np
    lib = _lib.load()
    inv = np.ones(32, np.float32)
    d = _lib.ModelDesc(2, 128, 2, 1, 64, 256, 50, _lib.SP_FMT_F16, 1, 8, 1e-6, 0.0,
                       inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    h = ctypes.c_void_p()
    rc = lib.sp_engine_create(ctypes.byref(d), ctypes.byref(h))
    assert rc == _lib.SP_EHIP and not h.value
    assert b'device' in lib.sp_last_error()


def test_engine_rejects_unsupported_shapes_before_touching_the_gpu():
    import numpy as np
    lib = _lib.load()
    inv = np.ones(48, np.float32)
    d = _lib.ModelDesc(2, 96 * 4, 4, 1, 96, 256, 50, _lib.SP_FMT_F16, 1, 8, 1e-6, 0.0,
                       inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    h = ctypes.c_void_p()
    assert lib.sp_engine_create(ctypes.byref(d), ctypes.byref(h)) == _lib.SP_EINVAL
    assert b'head_dim' in lib.sp_last_error()


def _columns_numpy(tok, depth, masks, seq, P, S, window):
    """The column rule written out with numpy: node i at pos P + depth[i], slot (P + i) mod S, context
    [max(0, pos - window + 1) or 0, P - 1], tree block based at P mod S."""
    import numpy as np
    n = len(tok)
    cols = np.zeros(n, dtype=_lib.TOKEN_DTYPE)
    pos = P + depth
    cols['token'], cols['seq'], cols['pos'] = tok, seq, pos
    cols['slot'] = (P + np.arange(n)) % S
    cols['ctx_lo'] = 0 if not window else np.maximum(0, pos - window + 1)
    cols['ctx_hi'], cols['tree_base'], cols['tree_count'], cols['tree_mask'] = P - 1, P % S, n, masks
    return cols


@pytest.mark.parametrize('P,S,window', [(0, 4096, 0), (2048, 4096, 0), (4090, 4096, 0), (9000, 1088, 1024),
                                        (3, 64, 2), (123456, 70000, 0)])
def test_tree_columns_match_the_column_rule(P, S, window):
    """sp_tree_columns (host only) against the rule for flattened random trees, with ring wrap-around and windows."""
    import numpy as np
    from seedplane_amd.speculative import flatten
    lib = _lib.load()
    rng = np.random.default_rng(P)
    for nb, depth in [(1, 1), (8, 4), (5, 7), (3, 21)]:
        tree = flatten(7, [list(rng.integers(0, 50, depth)) for _ in range(nb)])
        tok, dep, masks = tree.column_arrays()
        out = np.empty(tree.size, dtype=_lib.TOKEN_DTYPE)
        rc = lib.sp_tree_columns(tree.size, tok.ctypes.data, dep.ctypes.data, masks.ctypes.data, 3, P, S, window,
                                 out.ctypes.data)
        assert rc == _lib.SP_OK
        assert out.tobytes() == _columns_numpy(tok, dep, masks, 3, P, S, window).tobytes()


def test_tree_columns_reject_bad_arguments():
    import numpy as np
    lib = _lib.load()
    a = np.zeros(65, np.int32)
    m = np.zeros(65, np.uint64)
    out = np.empty(65, dtype=_lib.TOKEN_DTYPE)
    call = lambda n=2, P=10, S=16, w=0, d=a: lib.sp_tree_columns(n, a.ctypes.data, d.ctypes.data, m.ctypes.data, 0,
                                                                  P, S, w, out.ctypes.data)
    assert call() == _lib.SP_OK
    assert call(n=0) == _lib.SP_EINVAL and call(n=65) == _lib.SP_EINVAL
    assert call(S=0) == _lib.SP_EINVAL and call(P=-1) == _lib.SP_EINVAL and call(w=-1) == _lib.SP_EINVAL
    assert call(P=2 ** 31) == _lib.SP_EINVAL
    assert call(d=np.full(65, 64, np.int32)) == _lib.SP_EINVAL
    assert lib.sp_tree_columns(2, None, a.ctypes.data, m.ctypes.data, 0, 1, 16, 0, out.ctypes.data) == _lib.SP_EINVAL
