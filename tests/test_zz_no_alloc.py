"""The allocation-free argmax (sp_op_argmax_noalloc), called through the C ABI, gives the same ids as sp_op_argmax with
a caller workspace (bit-exact), on two calls in a row whose second input is smaller, and rejects sizes beyond its
512-row maximum."""
import ctypes

import numpy as np
import pytest
import torch

from seedplane_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _rows(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g)
    x[::3] = torch.round(x[::3] * 2) / 2              # ties inside and across the 64 block ranges
    x[1::7, cols // 3] = 9.0
    x[1::7, cols - 1] = 9.0                           # a tie at the maximum: the first index wins
    return x


def _with_workspace(lib, x):
    rows, cols = x.shape
    ws = torch.empty(lib.sp_op_argmax_workspace(rows, cols), dtype=torch.uint8, device=x.device)
    out = torch.full((rows,), -1, dtype=torch.int32, device=x.device)
    _lib.check(lib.sp_op_argmax(_ptr(x), rows, cols, _ptr(out), _ptr(ws), _stream()))
    return out


def test_noalloc_argmax_equals_workspace_argmax_on_two_calls(gpu_device):
    lib = _lib.load()
    print('noalloc argmax: 512 x 151936 then 7 x 1000', flush=True)
    for rows, cols, seed in ((512, 151936, 1), (7, 1000, 2)):
        x = _rows(rows, cols, seed)
        xd = x.to(gpu_device)
        out = torch.full((rows,), -1, dtype=torch.int32, device=gpu_device)
        _lib.check(lib.sp_op_argmax_noalloc(_ptr(xd), rows, cols, _ptr(out), _stream()))
        ref = _with_workspace(lib, xd)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (rows, cols)
        assert np.array_equal(out.cpu().numpy(), x.numpy().argmax(axis=1)), (rows, cols)   # first index on ties


def test_noalloc_argmax_rejects_sizes_beyond_its_maximum(gpu_device):
    lib = _lib.load()
    x = torch.zeros((513, 10), dtype=torch.float32, device=gpu_device)
    out = torch.zeros(513, dtype=torch.int32, device=gpu_device)
    assert lib.sp_op_argmax_noalloc(_ptr(x), 513, 10, _ptr(out), _stream()) == _lib.SP_EINVAL
    assert b'512' in lib.sp_last_error()
    assert lib.sp_op_argmax_noalloc(None, 4, 10, _ptr(out), _stream()) == _lib.SP_EINVAL
    assert lib.sp_op_argmax_noalloc(_ptr(x), 0, 10, _ptr(out), _stream()) == _lib.SP_EINVAL
