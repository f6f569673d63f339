"""Known-answer test of the gfx950 K/V tile loader (the role tests/bshd_tdm.hip:8-45
plays for the reference's gfx1250 TDM loader).

The probe library (build/libfav4_loader_kat.so, built by __graft_entry__.build()
from csrc/loader_kat.hip with the kernels' own DMA and operand-offset helpers)
loads one 64-key (8 or 4 waves) or 32-key (1 wave) tile of K and V into LDS and
returns (a) the raw LDS image and (b) every lane's MFMA operand registers as the
QK^T and PV steps read them.  K/V hold the integer pattern
1 + (r*137 + h*71 + d*13 + b*29) % 1021 as 16-bit words (row r, head h, dim d,
batch b; never 0), so a wrong row stride, head offset, swizzle or lane mapping
shows as a wrong word, and rows past the slice's end must read 0.

Expected values, stated independently of the kernel code:
* LDS: tile row r keeps its 16 granules (8 words each) at granule positions
  g ^ (r % 16) for K and g ^ (4 (r % 4) + (r / 4) % 4) for V.
* K operand (A of S^T = K.Q^T, v_mfma_f32_32x32x16_bf16: A[m][k] in lane
  m + 32 (k / 8), element k % 8): lane l, d-chunk c, element e holds key
  l % 32 of the 32-key block, dim 16c + 8 (l / 32) + e.
* V^T operand (A of O^T += V^T.P^T for a 16-key unit): lane l, 32-dim block
  db, element e holds dim 32 db + l % 32 and key 8 (e / 4) + 4 (l / 32) + e % 4
  of the unit -- the key order in which the S accumulator (C[m][n] in lane
  n + 32 ((m / 4) % 2), element 4 (m / 8) + m % 4) hands P to the same MFMA.
"""
import ctypes as C

import numpy as np
import pytest

from tests.conftest import ROOT

KAT_LIB = ROOT / "build" / "libfav4_loader_kat.so"
HIP_ERROR_INVALID_VALUE = 1


def _lib():
    import torch  # noqa: F401  (torch's HIP runtime first, as the package's loader does)
    if not KAT_LIB.exists():
        import __graft_entry__
        __graft_entry__.import_package().build_library()
    lib = C.CDLL(str(KAT_LIB))
    lib.fav4_kat_loader.argtypes = [C.c_void_p, C.c_void_p] + [C.c_int] * 7 + [C.c_void_p] * 4
    lib.fav4_kat_loader.restype = C.c_int
    return lib


def pattern(batch, sk, heads):
    b, r, h, d = np.meshgrid(np.arange(batch), np.arange(sk), np.arange(heads), np.arange(128), indexing="ij")
    return (1 + (r * 137 + h * 71 + d * 13 + b * 29) % 1021).astype(np.uint16)


def k_swz(r):
    return r % 16


def v_swz(r):
    return 4 * (r % 4) + (r // 4) % 4


def expected(x, b, h, t, bn, sk):
    """The tile's [bn, 128] words (0 past sk)."""
    tile = np.zeros((bn, 128), np.uint16)
    rows = np.arange(t * bn, min(sk, (t + 1) * bn))
    tile[:len(rows)] = x[b, rows, h]
    return tile


def lds_image(tile, swz):
    out = np.zeros_like(tile)
    for r in range(tile.shape[0]):
        for g in range(16):
            pos = g ^ swz(r)
            out[r, pos * 8:(pos + 1) * 8] = tile[r, g * 8:(g + 1) * 8]
    return out


def k_operands(tile):
    bn = tile.shape[0]
    out = np.zeros((bn // 32, 8, 64, 8), np.uint16)
    for kb in range(bn // 32):
        for c in range(8):
            for lane in range(64):
                key = kb * 32 + lane % 32
                d0 = 16 * c + 8 * (lane // 32)
                out[kb, c, lane] = tile[key, d0:d0 + 8]
    return out


def v_operands(tile):
    bn = tile.shape[0]
    out = np.zeros((bn // 16, 4, 64, 8), np.uint16)
    for u in range(bn // 16):
        for db in range(4):
            for lane in range(64):
                for e in range(8):
                    key = 16 * u + 8 * (e // 4) + 4 * (lane // 32) + e % 4
                    out[u, db, lane, e] = tile[key, 32 * db + lane % 32]
    return out


def test_probe_rejects_bad_arguments():
    """Host-side checks of the probe entry point (no GPU call is made)."""
    lib = _lib()
    ok = dict(k=0x10000, v=0x20000, batch=2, heads=3, sk=64, b=1, h=2, t=0, waves=8, lds=0x30000, kop=0x40000,
              vop=0x50000)
    bad = [dict(b=2), dict(h=3), dict(t=1), dict(waves=2), dict(sk=0), dict(k=0x10008), dict(k=None),
           dict(heads=1 << 16, sk=1 << 16)]
    for change in bad:
        a = dict(ok, **change)
        got = lib.fav4_kat_loader(a["k"], a["v"], a["batch"], a["heads"], a["sk"], a["b"], a["h"], a["t"],
                                  a["waves"], a["lds"], a["kop"], a["vop"], None)
        assert got == HIP_ERROR_INVALID_VALUE, change


CASES = [(w, heads, sk, t) for w in (8, 4) for heads in (3, 8, 513) for sk in (1, 17, 47, 64) for t in (0,)]
CASES += [(w, heads, 64 + 17, 1) for w in (8, 4) for heads in (3, 513)]
CASES += [(1, heads, sk, 0) for heads in (3, 8, 513) for sk in (1, 17, 31, 32)]
CASES += [(1, heads, 32 + 5, 1) for heads in (3, 513)]


@pytest.mark.gpu
@pytest.mark.parametrize("waves,heads,sk,t", CASES, ids=[f"w{w}_h{h}_rows{s}_tile{t}" for w, h, s, t in CASES])
def test_loader_kat(waves, heads, sk, t):
    import torch
    lib = _lib()
    dev = torch.device("cuda:0")
    bn = 32 if waves == 1 else 64
    batch, b, h = 2, 1, heads - 1                  # the last head of the second batch
    print(f"loader KAT waves={waves} heads={heads} rows={sk} tile={t}", flush=True)
    kx = pattern(batch, sk, heads)
    vx = (kx.astype(np.int64) * 7 % 1021 + 1).astype(np.uint16)   # a different pattern for V
    kd = torch.from_numpy(kx.view(np.int16)).to(dev)
    vd = torch.from_numpy(vx.view(np.int16)).to(dev)
    lds = torch.zeros(2 * bn * 128, device=dev, dtype=torch.int16)
    kop = torch.zeros(waves * (bn // 32) * 8 * 64 * 8, device=dev, dtype=torch.int16)
    vop = torch.zeros(waves * (bn // 16) * 4 * 64 * 8, device=dev, dtype=torch.int16)
    st = lib.fav4_kat_loader(kd.data_ptr(), vd.data_ptr(), batch, heads, sk, b, h, t, waves, lds.data_ptr(),
                             kop.data_ptr(), vop.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == 0, st
    torch.cuda.synchronize()
    got_lds = lds.cpu().numpy().view(np.uint16).reshape(2, bn, 128)
    got_k = kop.cpu().numpy().view(np.uint16).reshape(waves, bn // 32, 8, 64, 8)
    got_v = vop.cpu().numpy().view(np.uint16).reshape(waves, bn // 16, 4, 64, 8)
    kt, vt = expected(kx, b, h, t, bn, sk), expected(vx, b, h, t, bn, sk)
    np.testing.assert_array_equal(got_lds[0], lds_image(kt, k_swz))
    np.testing.assert_array_equal(got_lds[1], lds_image(vt, v_swz))
    for w in range(waves):
        np.testing.assert_array_equal(got_k[w], k_operands(kt))
        np.testing.assert_array_equal(got_v[w], v_operands(vt))
    assert (kt[sk - t * bn:] == 0).all() and (kt[:sk - t * bn] != 0).all()   # the zero fill is exercised
