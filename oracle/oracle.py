"""numpy/ctypes front end of the C oracle (conv3d_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; the product never imports it.

Every function takes and returns float32 numpy arrays in NCDHW (activations)
and PyTorch parameter layouts (weights), and accumulates in double.  See
conv3d_oracle.c for the reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_conv3d.so"

FAULT_NONE = 0
FAULT_FWD_PAD_OFF_BY_ONE = 1
FAULT_DX_NO_FLIP = 2
FAULT_DW_SWAP_HW = 3
FAULT_CONVT_TAP_ORDER = 4
FAULT_DB_DROPPED = 5

_lib = None


def build(force: bool = False) -> Path:
    if force or not LIB.exists() or LIB.stat().st_mtime < (HERE / "conv3d_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE), "liboracle_conv3d.so"], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(str(LIB))
        fp = ctypes.POINTER(ctypes.c_float)
        i = ctypes.c_int
        lib.oracle_conv3d_fwd.argtypes = [fp, fp, fp, fp] + [i] * 10
        lib.oracle_conv3d_dx.argtypes = [fp, fp, fp] + [i] * 10
        lib.oracle_conv3d_dw.argtypes = [fp, fp, fp, fp] + [i] * 10
        lib.oracle_convt_fwd.argtypes = [fp, fp, fp, fp] + [i] * 6
        lib.oracle_convt_dx.argtypes = [fp, fp, fp] + [i] * 6
        lib.oracle_convt_dw.argtypes = [fp, fp, fp, fp] + [i] * 6
        lib.oracle_set_fault.argtypes = [i]
        lib.oracle_round_bf16.argtypes = [fp, ctypes.c_int64]
        _lib = lib
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def set_fault(f: int) -> None:
    _load().oracle_set_fault(int(f))


def _pad3(p):
    return (p, p, p) if isinstance(p, int) else tuple(int(v) for v in p)


def conv3d_fwd(x, w, b=None, padding=0):
    x, w = _f32(x), _f32(w)
    b = None if b is None else _f32(b)
    n, cin, d, h, wd = x.shape
    cout, k = w.shape[0], w.shape[2]
    pd, ph, pw = _pad3(padding)
    y = np.empty((n, cout, d + 2 * pd - k + 1, h + 2 * ph - k + 1, wd + 2 * pw - k + 1), np.float32)
    _load().oracle_conv3d_fwd(_p(x), _p(w), _p(b), _p(y), n, cin, d, h, wd, cout, k, pd, ph, pw)
    return y


def conv3d_dx(dy, w, x_shape, padding=0):
    dy, w = _f32(dy), _f32(w)
    n, cin, d, h, wd = (int(v) for v in x_shape)
    cout, k = w.shape[0], w.shape[2]
    pd, ph, pw = _pad3(padding)
    dx = np.empty((n, cin, d, h, wd), np.float32)
    _load().oracle_conv3d_dx(_p(dy), _p(w), _p(dx), n, cin, d, h, wd, cout, k, pd, ph, pw)
    return dx


def conv3d_dw(x, dy, k, padding=0):
    x, dy = _f32(x), _f32(dy)
    n, cin, d, h, wd = x.shape
    cout = dy.shape[1]
    pd, ph, pw = _pad3(padding)
    dw = np.empty((cout, cin, k, k, k), np.float32)
    db = np.empty((cout,), np.float32)
    _load().oracle_conv3d_dw(_p(x), _p(dy), _p(dw), _p(db), n, cin, d, h, wd, cout, k, pd, ph, pw)
    return dw, db


def convt_fwd(x, w, b=None):
    x, w = _f32(x), _f32(w)
    b = None if b is None else _f32(b)
    n, cin, d, h, wd = x.shape
    cout = w.shape[1]
    y = np.empty((n, cout, 2 * d, 2 * h, 2 * wd), np.float32)
    _load().oracle_convt_fwd(_p(x), _p(w), _p(b), _p(y), n, cin, d, h, wd, cout)
    return y


def convt_dx(dy, w, x_shape):
    dy, w = _f32(dy), _f32(w)
    n, cin, d, h, wd = (int(v) for v in x_shape)
    cout = w.shape[1]
    dx = np.empty((n, cin, d, h, wd), np.float32)
    _load().oracle_convt_dx(_p(dy), _p(w), _p(dx), n, cin, d, h, wd, cout)
    return dx


def convt_dw(x, dy):
    x, dy = _f32(x), _f32(dy)
    n, cin, d, h, wd = x.shape
    cout = dy.shape[1]
    dw = np.empty((cin, cout, 2, 2, 2), np.float32)
    db = np.empty((cout,), np.float32)
    _load().oracle_convt_dw(_p(x), _p(dy), _p(dw), _p(db), n, cin, d, h, wd, cout)
    return dw, db


def round_bf16(a):
    a = np.array(a, dtype=np.float32, copy=True, order="C")
    _load().oracle_round_bf16(_p(a), a.size)
    return a
