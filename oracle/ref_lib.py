"""ctypes wrapper of oracle/_ref/libphase_linear_ref.so: the reference's own
Android phase-linear C++ (RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp,
kernels/*.cpp) compiled from its sources by oracle/Makefile.  Test
infrastructure and CPU baseline only; returns None from load() when the
library was not built (it needs the reference checkout)."""
from __future__ import annotations

import ctypes
import os

import numpy as np

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libphase_linear_ref.so")
_lib = None


def load():
    global _lib
    if _lib is None and os.path.exists(_PATH):
        lib = ctypes.CDLL(_PATH)
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        lib.ref_phase_linear.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, ctypes.c_char_p, i32]
        lib.ref_phase_linear.restype = i32
        lib.ref_wide_linear.argtypes = [vp, i32, i32, i32, i32, i32, i32, i32, ctypes.POINTER(vp),
                                        ctypes.POINTER(vp), ctypes.POINTER(vp), vp, vp, i32, i32,
                                        ctypes.c_char_p, i32]
        lib.ref_wide_linear.restype = i32
        lib.ref_float_to_half_bits.argtypes = [ctypes.c_float]
        lib.ref_float_to_half_bits.restype = ctypes.c_uint16
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def phase_linear(xr, xi, codes, g_re, g_im, block):
    """phaseLinearReference on unpacked codes [N, K] and fp16 gammas [N, K/block]."""
    lib = load()
    xr = np.ascontiguousarray(xr, np.float32)
    xi = np.ascontiguousarray(xi, np.float32)
    tokens, k = xr.shape
    n = codes.shape[0]
    packed = np.ascontiguousarray(_pack(codes))
    gr = np.ascontiguousarray(g_re, np.float16).view(np.uint16)
    gi = np.ascontiguousarray(g_im, np.float16).view(np.uint16)
    yr = np.zeros((tokens, n), np.float32)
    yi = np.zeros((tokens, n), np.float32)
    err = ctypes.create_string_buffer(512)
    rc = lib.ref_phase_linear(_p(xr), _p(xi), tokens, k, n, block, _p(packed), _p(gr), _p(gi), _p(yr), _p(yi),
                              err, 512)
    if rc:
        raise RuntimeError(err.value.decode())
    return yr, yi


def wide_linear(x, planes, g_re, g_im, bias, block, mode=0, threads=1):
    """wideLinearReference (mode 0), fp16 fused cache (1) or fused scalar (2)
    on 4 unpacked planes u_s0, u_s1, w_s0, w_s1 [N', K'] with fp16 gammas."""
    lib = load()
    x = np.ascontiguousarray(x, np.float32)
    tokens, real_in = x.shape
    n_c, k_c = planes[0].shape
    keep = [np.ascontiguousarray(_pack(p)) for p in planes]
    keep += [np.ascontiguousarray(g, np.float16).view(np.uint16) for g in g_re]
    keep += [np.ascontiguousarray(g, np.float16).view(np.uint16) for g in g_im]
    arr = ctypes.c_void_p * 4
    cp = arr(*[_p(a) for a in keep[0:4]])
    gr = arr(*[_p(a) for a in keep[4:8]])
    gi = arr(*[_p(a) for a in keep[8:12]])
    b = np.ascontiguousarray(bias, np.float32)
    y = np.zeros((tokens, 2 * n_c), np.float32)
    err = ctypes.create_string_buffer(512)
    rc = lib.ref_wide_linear(_p(x), tokens, real_in, 2 * n_c, k_c, n_c, n_c, block, cp, gr, gi, _p(b), _p(y),
                             mode, threads, err, 512)
    if rc:
        raise RuntimeError(err.value.decode())
    return y


def _pack(codes):
    c = np.asarray(codes, np.uint8)
    rows, k = c.shape
    c = c.reshape(rows, k // 4, 4)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)
