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


_CAPTURE = r'''
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
from seedplane_amd import _lib
lib = _lib.load()
dev = torch.device('cuda:0')
P = lambda t: ctypes.c_void_p(t.data_ptr())
rows, cols = 33, 151936
x = torch.randn(rows, cols, device=dev)
out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
ref = torch.full((rows,), -1, dtype=torch.int32, device=dev)
ws = torch.empty(lib.sp_op_argmax_workspace(rows, cols), dtype=torch.uint8, device=dev)
warm = sys.argv[2] == 'warm'
if warm:        # a call outside capture first: the scratch address is looked up then
    _lib.check(lib.sp_op_argmax_noalloc(P(x), rows, cols, P(out), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.graph(g, stream=s):
    _lib.check(lib.sp_op_argmax_noalloc(P(x), rows, cols, P(out), ctypes.c_void_p(s.cuda_stream)))
for i in range(4):
    x.copy_(torch.randn(rows, cols, device=dev))
    x[i, 1000 + i] = 50.0                              # a known winner per replay
    g.replay()
    torch.cuda.synchronize()
    _lib.check(lib.sp_op_argmax(P(x), rows, cols, P(ref), P(ws), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert torch.equal(out, ref), (i, out[:4], ref[:4])
    assert int(out[i]) == 1000 + i
print('capture ok', sys.argv[2])
'''


@pytest.mark.parametrize('order', ['first', 'warm'])
def test_noalloc_argmax_under_graph_capture(gpu_device, order):
    """Captured into a hipGraph on a non-null stream -- as the process's first call of the entry point (its scratch
    address is looked up during the capture) and after a warm call -- and replayed four times over new inputs, with
    eager work between replays: every replay equals sp_op_argmax.  A fresh process makes 'first' really first."""
    import subprocess
    import sys
    from pathlib import Path
    print(f'noalloc argmax under graph capture ({order})', flush=True)
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, '-c', _CAPTURE, root, order], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert f'capture ok {order}' in r.stdout
