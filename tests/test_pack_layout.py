"""The tiled HBM layout, checked on the CPU: pack with the library's host packer, then read the tiles back exactly
as the GEMV kernel's lanes do (lane l -> row l % 16, k-subset l / 16; Q8 bytes 0-7 / 8-15 = blocks 2kt / 2kt+1;
Q4 dword s = group s with code i at nibble (i/2) + 4*(i%2); per-row side data) and compare the emulated GEMV with
the closed-form dequantised product."""
import ctypes

import numpy as np
import pytest
import torch

from oracle.quant_ref import dequant_q4, dequant_q8
from seedplane_amd import _lib


def pack(fmt, rows, cols, data, scales=None, zeros=None, pair=False):
    lib = _lib.load()
    cb, sb = ctypes.c_uint64(), ctypes.c_uint64()
    ptr = lambda a: None if a is None else ctypes.c_void_p(a.ctypes.data)
    _lib.check(lib.sp_pack_matrix(fmt, rows, cols, ptr(data), ptr(scales), ptr(zeros), int(pair), None,
                                  ctypes.byref(cb), None, ctypes.byref(sb)))
    codes = np.zeros(cb.value, np.uint8)
    side = np.zeros(max(sb.value // 2, 1), np.uint16)
    _lib.check(lib.sp_pack_matrix(fmt, rows, cols, ptr(data), ptr(scales), ptr(zeros), int(pair),
                                  ctypes.c_void_p(codes.ctypes.data), ctypes.byref(cb),
                                  ctypes.c_void_p(side.ctypes.data), ctypes.byref(sb)))
    return codes, side


def emulate(fmt, codes, side, rows_pad, cols, x):
    """y[m][n] the way k_gemv computes it (per quant block: dot of exact codes with x, then scale / zero)."""
    KT = {1: 32, 2: 64, 3: 128}[fmt]
    nkt = cols // KT
    ng = rows_pad // 16
    y = np.zeros((x.shape[0], rows_pad))
    tiles = codes.reshape(ng, nkt, 64, 16)          # [group][kt][lane][16 bytes]
    for rg in range(ng):
        for kt in range(nkt):
            for lane in range(64):
                r, g = lane % 16, lane // 16
                n = rg * 16 + r
                b = tiles[rg, kt, lane]
                if fmt == 1:
                    w = b.view(np.float16).astype(np.float64)
                    y[:, n] += x[:, kt * 32 + 8 * g: kt * 32 + 8 * g + 8] @ w
                elif fmt == 2:
                    sc = side.reshape(ng, nkt, 16, 2)[rg, kt, r].view(np.float16).astype(np.float64)
                    for s in range(2):
                        c = b[8 * s: 8 * s + 8].view(np.int8).astype(np.float64)
                        k0 = kt * 64 + 32 * s + 8 * g
                        y[:, n] += sc[s] * (x[:, k0:k0 + 8] @ c)
                else:
                    sz = side.reshape(ng, nkt, 16, 4, 2)[rg, kt, r].view(np.float16).astype(np.float64)
                    d = b.view(np.uint32)
                    for s in range(4):
                        v = int(d[s])
                        c = []
                        for j in range(4):                                   # q4_pair(v, j)
                            c += [(v >> (4 * j)) & 15, (v >> (16 + 4 * j)) & 15]
                        c = np.array(c, np.float64)
                        k0 = kt * 128 + 32 * s + 8 * g
                        xs = x[:, k0:k0 + 8]
                        y[:, n] += sz[s, 0] * (xs @ c - sz[s, 1] * xs.sum(1))
    return y


@pytest.mark.parametrize('fmt', [1, 2, 3])
def test_emulated_gemv_matches_dequant(fmt):
    rows, cols = 40, 256
    g = torch.Generator().manual_seed(fmt)
    if fmt == 1:
        w = (torch.randn(rows, cols, generator=g) * 0.1).half()
        arrays = (w.view(torch.int16).numpy(), None, None)
        ref_w = w.double()
    elif fmt == 2:
        c = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
        s = (torch.randn(rows, cols // 32, generator=g) * 0.002).abs().half()
        arrays = (c.numpy(), s.view(torch.int16).numpy(), None)
        ref_w = dequant_q8(c, s).double()
    else:
        p = torch.randint(0, 256, (rows, cols // 2), generator=g, dtype=torch.int32).to(torch.uint8)
        s = (torch.randn(rows, cols // 32, generator=g) * 0.002).abs().half()
        z = (torch.rand(rows, cols // 32, generator=g) + 7.0).half()
        arrays = (p.numpy(), s.view(torch.int16).numpy(), z.view(torch.int16).numpy())
        ref_w = dequant_q4(p, s, z).double()
    codes, side = pack(fmt, rows, cols, *[None if a is None else np.ascontiguousarray(a) for a in arrays])
    x = torch.randn(3, cols, generator=g).half().double().numpy()
    y = emulate(fmt, codes, side, 48, cols, x)[:, :rows]
    ref = x @ ref_w.numpy().T
    assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-12


def test_gate_up_pairing_interleaves_row_groups():
    rows, cols = 64, 64
    w = np.arange(rows * cols, dtype=np.float32).reshape(rows, cols).astype(np.float16)
    codes, _ = pack(1, rows, cols, np.ascontiguousarray(w.view(np.int16)), pair=True)
    tiles = codes.reshape(4, 2, 64, 16)
    # packed row group 1 = up rows 32..47 (second half), group 2 = gate rows 16..31
    first_k = lambda rg, r: tiles[rg, 0, r].view(np.float16)[0]
    assert float(first_k(1, 0)) == float(w[32, 0]) and float(first_k(2, 3)) == float(w[19, 0])


def test_packer_rejects_bad_shapes():
    lib = _lib.load()
    cb, sb = ctypes.c_uint64(), ctypes.c_uint64()
    a = np.zeros((16, 100), np.int8)
    rc = lib.sp_pack_matrix(2, 16, 100, ctypes.c_void_p(a.ctypes.data), ctypes.c_void_p(a.ctypes.data), None, 0, None,
                            ctypes.byref(cb), None, ctypes.byref(sb))
    assert rc == _lib.SP_EINVAL and b'multiple' in lib.sp_last_error()
