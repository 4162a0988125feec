"""Kernel-level parity through the C ABI: block-dequant GEMV (all formats, 1..64 columns) and the two-pass argmax."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.quant_ref import dequant_q4, dequant_q8
from seedplane_amd import _lib

pytestmark = pytest.mark.gpu


def _weights(fmt, rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    if fmt == 'f16':
        w = (torch.randn(rows, cols, generator=g) * 0.05).half()
        return _lib.SP_FMT_F16, (w.view(torch.int16).numpy(), None, None), w.float()
    if fmt == 'q8':
        c = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
        s = (torch.randn(rows, cols // 32, generator=g) * 0.002).abs().half()
        return _lib.SP_FMT_Q8, (c.numpy(), s.view(torch.int16).numpy(), None), dequant_q8(c, s)
    p = torch.randint(0, 256, (rows, cols // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s = (torch.randn(rows, cols // 32, generator=g) * 0.002).abs().half()
    z = (torch.rand(rows, cols // 32, generator=g) + 7.0).half()
    return _lib.SP_FMT_Q4, (p.numpy(), s.view(torch.int16).numpy(), z.view(torch.int16).numpy()), dequant_q4(p, s, z)


def _ptr(a):
    return None if a is None else ctypes.c_void_p(np.ascontiguousarray(a).ctypes.data)


class Weight:
    def __init__(self, fmt, arrays, rows, cols):
        self.lib = _lib.load()
        self.arrays = [None if a is None else np.ascontiguousarray(a) for a in arrays]
        h = ctypes.c_void_p()
        _lib.check(self.lib.sp_weight_create(fmt, rows, cols, *[_ptr(a) for a in self.arrays], ctypes.byref(h)))
        self.h = h

    def __del__(self):
        self.lib.sp_weight_destroy(self.h)

    def gemv(self, x, rows, ws=None):
        m = x.shape[0]
        if ws is None:
            ws = torch.zeros(self.lib.sp_op_gemv_workspace(self.h, m), dtype=torch.uint8, device=x.device)
        y = torch.empty((m, rows), dtype=torch.float32, device=x.device)
        stream = torch.cuda.current_stream().cuda_stream
        _lib.check(self.lib.sp_op_gemv(self.h, ctypes.c_void_p(x.data_ptr()), m, ctypes.c_void_p(y.data_ptr()),
                                       ctypes.c_void_p(ws.data_ptr()), ctypes.c_void_p(stream)))
        torch.cuda.synchronize()
        return y, ws


@pytest.mark.parametrize('fmt', ['f16', 'q8', 'q4'])
@pytest.mark.parametrize('rows,cols', [(1000, 1536), (2048, 8960), (48, 256)])
@pytest.mark.parametrize('m', [1, 3, 16, 17, 33, 64])
def test_gemv_matches_dequantized_matmul(gpu_device, fmt, rows, cols, m):
    print(f'gemv fmt={fmt} rows={rows} cols={cols} m={m}', flush=True)
    code, arrays, wdeq = _weights(fmt, rows, cols, seed=rows + cols + m)
    w = Weight(code, arrays, rows, cols)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(m, cols, generator=g).half()
    ref = x.double() @ wdeq.double().T                      # exact codes, fp16 activations, float64 sum
    y, ws = w.gemv(x.to(gpu_device), rows)
    err = float((y.double().cpu() - ref).abs().max() / ref.abs().max())
    assert err < 2e-5, err
    # same workspace again: the split-K arrival counters must have been left at zero, and the fixed reduction
    # order makes the result bit-identical
    y2, _ = w.gemv(x.to(gpu_device), rows, ws=ws)
    assert torch.equal(y, y2), 'GEMV must be deterministic and leave its counters zeroed'


def _argmax(logits):
    lib = _lib.load()
    rows, cols = logits.shape
    ws = torch.empty(lib.sp_op_argmax_workspace(rows, cols), dtype=torch.uint8, device=logits.device)
    out = torch.full((rows,), -1, dtype=torch.int32, device=logits.device)
    _lib.check(lib.sp_op_argmax(ctypes.c_void_p(logits.data_ptr()), rows, cols, ctypes.c_void_p(out.data_ptr()),
                                ctypes.c_void_p(ws.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    return out.cpu()


def test_argmax_first_index_on_ties(gpu_device):
    V = 151936
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, V, generator=g)
    x[1, 5] = 100.0; x[1, 150000] = 100.0                  # tie across blocks -> 5
    x[2, 77777] = 9.0; x[2, 77778] = 9.0                    # tie inside a block -> 77777
    x[3] = 0.0                                              # all equal -> 0 (reference special case)
    x[4, V - 1] = 50.0                                      # last element
    x[5, :] = -1e30; x[5, 123] = -1e29
    got = _argmax(x.to(gpu_device))
    assert got.tolist() == torch.argmax(x, dim=1).tolist() == [int(torch.argmax(x[0])), 5, 77777, 0, V - 1, 123]


@pytest.mark.parametrize('cols', [1, 50, 64, 1000, 152064])
def test_argmax_matches_torch_random(gpu_device, cols):
    g = torch.Generator().manual_seed(cols)
    x = torch.randint(-3, 4, (9, cols), generator=g).float()     # many exact ties
    assert _argmax(x.to(gpu_device)).tolist() == torch.argmax(x, dim=1).tolist()
