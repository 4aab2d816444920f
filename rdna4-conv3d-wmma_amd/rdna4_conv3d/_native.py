"""ctypes binding of librdna4_conv3d_hip.so (the gfx950 kernels behind the C ABI
declared in include/rdna4_conv3d.h).

This module is the marshaller that replaces the reference's Triton launch
wrappers (src/rdna4_conv3d/conv3d_wmma.py:1048-1214, 1462-1542): it builds the
plain-C descriptor from tensor shapes and strides, allocates outputs (in the
input's memory format) and the workspace through PyTorch's caching allocator,
and enqueues the kernels on the current PyTorch stream.  Nothing is computed in
Python.  There is no fallback here: if the library cannot be loaded, every
call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from functools import lru_cache
from pathlib import Path
from typing import Optional, Sequence, Tuple

import torch  # imported first: the library reuses the HIP runtime torch loaded

LIB_NAME = "librdna4_conv3d_hip.so"
ABI_VERSION = 1

R3C_OK, R3C_UNSUPPORTED, R3C_INVALID, R3C_HIP_ERROR = 0, 1, 2, 3
R3C_F16, R3C_BF16, R3C_F32 = 0, 1, 2

_DTYPE_CODE = {torch.float16: R3C_F16, torch.bfloat16: R3C_BF16, torch.float32: R3C_F32}


class ConvDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("n", ctypes.c_int32), ("cin", ctypes.c_int32), ("d", ctypes.c_int32),
        ("h", ctypes.c_int32), ("w", ctypes.c_int32),
        ("cout", ctypes.c_int32), ("od", ctypes.c_int32), ("oh", ctypes.c_int32),
        ("ow", ctypes.c_int32),
        ("kernel", ctypes.c_int32),
        ("pad_d", ctypes.c_int32), ("pad_h", ctypes.c_int32), ("pad_w", ctypes.c_int32),
        ("x_strides", ctypes.c_int64 * 5),
        ("y_strides", ctypes.c_int64 * 5),
    ]


class BnDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("n", ctypes.c_int32), ("c", ctypes.c_int32),
        ("s", ctypes.c_int64),
        ("y_strides", ctypes.c_int64 * 2),
        ("g_strides", ctypes.c_int64 * 2),
        ("o_strides", ctypes.c_int64 * 2),
        ("training", ctypes.c_int32),
        ("eps", ctypes.c_float), ("momentum", ctypes.c_float),
    ]


class PoolDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("n", ctypes.c_int32), ("c", ctypes.c_int32), ("d", ctypes.c_int32), ("h", ctypes.c_int32),
        ("w", ctypes.c_int32),
        ("x_strides", ctypes.c_int64 * 2),
        ("y_strides", ctypes.c_int64 * 2),
    ]


class NativeError(RuntimeError):
    """A native entry point returned R3C_INVALID or R3C_HIP_ERROR."""


class NativeUnsupported(RuntimeError):
    """A native entry point returned R3C_UNSUPPORTED (caller may fall back)."""


_lib = None
_lib_err: Optional[str] = None
_lock = threading.Lock()


def library_path() -> Path:
    override = os.environ.get("RDNA4_CONV3D_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / LIB_NAME


def _bind(lib: ctypes.CDLL) -> None:
    P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    D = ctypes.POINTER(ConvDesc)
    lib.r3c_abi_version.restype = I32
    lib.r3c_abi_version.argtypes = []
    lib.r3c_last_error.restype = ctypes.c_char_p
    lib.r3c_last_error.argtypes = []
    lib.r3c_device_supported.restype = I32
    lib.r3c_device_supported.argtypes = [I32]
    for name in ("conv3d_fwd", "conv3d_dx", "conv3d_dw", "convt_k2s2_fwd", "convt_k2s2_dx", "convt_k2s2_dw"):
        f = getattr(lib, f"r3c_{name}_workspace")
        f.restype = I64
        f.argtypes = [D]
    for name in ("conv3d_fwd", "convt_k2s2_fwd"):
        f = getattr(lib, f"r3c_{name}")
        f.restype = I32
        f.argtypes = [D, P, P, P, P, P, I64, P]
    for name in ("conv3d_dx", "convt_k2s2_dx"):
        f = getattr(lib, f"r3c_{name}")
        f.restype = I32
        f.argtypes = [D, P, P, P, P, I64, P]
    for name in ("conv3d_dw", "convt_k2s2_dw"):
        f = getattr(lib, f"r3c_{name}")
        f.restype = I32
        f.argtypes = [D, P, P, P, I32, P, I32, P, I64, P]
    B = ctypes.POINTER(BnDesc)
    lib.r3c_bn_relu_workspace.restype = I64
    lib.r3c_bn_relu_workspace.argtypes = [B]
    lib.r3c_bn_relu_fwd.restype = I32
    lib.r3c_bn_relu_fwd.argtypes = [B, P, P, P, P, P, P, P, P, P, I64, P]
    lib.r3c_bn_relu_bwd.restype = I32
    lib.r3c_bn_relu_bwd.argtypes = [B, P, P, P, P, P, P, P, P, P, P, I64, P]
    lib.r3c_conv3d_cat_workspace.restype = ctypes.c_int64
    lib.r3c_conv3d_cat_workspace.argtypes = [D, I32, ctypes.c_int64, I32]
    lib.r3c_conv3d_cat_fwd.restype = I32
    lib.r3c_conv3d_cat_fwd.argtypes = [D, I32, P, P, ctypes.c_int64, P, P, P, P, ctypes.c_int64, P]
    lib.r3c_conv3d_cat_dx.restype = I32
    lib.r3c_conv3d_cat_dx.argtypes = [D, I32, P, P, P, P, ctypes.c_int64, P, ctypes.c_int64, P]
    lib.r3c_conv3d_cat_dw.restype = I32
    lib.r3c_conv3d_cat_dw.argtypes = [D, I32, P, P, ctypes.c_int64, P, P, I32, P, I32, P, ctypes.c_int64, P]
    S = ctypes.POINTER(I32)
    lib.r3c_conv3d_strided_workspace.restype = I64
    lib.r3c_conv3d_strided_workspace.argtypes = [D, S, I32]
    lib.r3c_conv3d_strided_fwd.restype = I32
    lib.r3c_conv3d_strided_fwd.argtypes = [D, S, P, P, P, P, P, I64, P]
    lib.r3c_conv3d_strided_dx.restype = I32
    lib.r3c_conv3d_strided_dx.argtypes = [D, S, P, P, P, P, I64, P]
    lib.r3c_conv3d_strided_dw.restype = I32
    lib.r3c_conv3d_strided_dw.argtypes = [D, S, P, P, P, I32, P, I32, P, I64, P]
    lib.r3c_probe_mfma.restype = I32
    lib.r3c_probe_mfma.argtypes = [I32, I32, I32, P, P]
    Q = ctypes.POINTER(PoolDesc)
    lib.r3c_maxpool2_fwd.restype = I32
    lib.r3c_maxpool2_fwd.argtypes = [Q, P, P, P, P]
    lib.r3c_maxpool2_bwd.restype = I32
    lib.r3c_maxpool2_bwd.argtypes = [Q, P, P, P, P]
    lib.r3c_maxpool2_bwd_add.restype = I32
    lib.r3c_maxpool2_bwd_add.argtypes = [Q, P, P, P, ctypes.POINTER(ctypes.c_int64), P, P]
    lib.r3c_conv3d_dw_static.restype = I32
    lib.r3c_conv3d_dw_static.argtypes = [D, P, P, P, I32, P, I32, P]
    lib.r3c_timing_enable.restype = I32
    lib.r3c_timing_enable.argtypes = [I32]
    lib.r3c_timing_set_tag.restype = None
    lib.r3c_timing_set_tag.argtypes = [I32]
    lib.r3c_timing_filter.restype = None
    lib.r3c_timing_filter.argtypes = [I32, I32]
    lib.r3c_timing_collect.restype = I32
    lib.r3c_timing_collect.argtypes = [I32, ctypes.POINTER(I32), ctypes.POINTER(I32), ctypes.POINTER(ctypes.c_float)]


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise RuntimeError if absent."""
    global _lib, _lib_err
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        try:
            lib = ctypes.CDLL(str(path))
            _bind(lib)
            ver = lib.r3c_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"ABI version {ver}, expected {ABI_VERSION}")
        except (OSError, AttributeError, RuntimeError) as e:
            _lib_err = f"cannot load {path}: {e}"
            raise RuntimeError(
                f"rdna4_conv3d native library unavailable ({_lib_err}); "
                "build it with `python __graft_entry__.py build` or "
                "`python rdna4-conv3d-wmma_amd/build_native.py`") from e
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def device_supported(device_index: int) -> bool:
    return bool(load().r3c_device_supported(int(device_index)))


KERNEL_KINDS = ("pack", "row", "wgrad", "reduce", "layout", "split_epilogue", "bn", "pool")


def timing_enable(on: bool) -> None:
    """Start (clearing old records) or stop per-launch kernel timing in the library."""
    load().r3c_timing_enable(1 if on else 0)


def timing_tag(tag: int) -> None:
    """Tag attached to the kernels this thread launches next."""
    load().r3c_timing_set_tag(int(tag))


def timing_filter(tag: int = -1, kind: Optional[str] = None) -> None:
    """Record only launches with this tag and kernel kind name (-1 / None = any)."""
    load().r3c_timing_filter(int(tag), -1 if kind is None else KERNEL_KINDS.index(kind))


def timing_collect(max_records: int = 1 << 16):
    """Wait for recorded launches; return [(tag, kind name, ms)] and clear them."""
    lib = load()
    tags = (ctypes.c_int32 * max_records)()
    kinds = (ctypes.c_int32 * max_records)()
    ms = (ctypes.c_float * max_records)()
    n = lib.r3c_timing_collect(max_records, tags, kinds, ms)
    return [(int(tags[i]), KERNEL_KINDS[kinds[i]], float(ms[i])) for i in range(min(n, max_records))]


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _dims5(t: torch.Tensor) -> Tuple[int, ...]:
    if t.dim() != 5:
        raise ValueError(f"expected a 5-D tensor, got {tuple(t.shape)}")
    return tuple(int(s) for s in t.shape)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream_handle(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check(lib, rc: int, what: str) -> None:
    if rc == R3C_OK:
        return
    msg = lib.r3c_last_error().decode(errors="replace")
    if rc == R3C_UNSUPPORTED:
        raise NativeUnsupported(f"{what}: {msg}")
    raise NativeError(f"{what} failed (code {rc}): {msg}")


def is_channels_last(t: torch.Tensor) -> bool:
    return t.dim() == 5 and t.is_contiguous(memory_format=torch.channels_last_3d)


def _dense(t: torch.Tensor) -> torch.Tensor:
    """NCDHW-contiguous or channels_last_3d tensors pass through; others are densified."""
    if t.is_contiguous() or is_channels_last(t):
        return t
    return t.contiguous()


def _empty_like_layout(shape: Sequence[int], like: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    fmt = torch.channels_last_3d if (is_channels_last(like) and not like.is_contiguous()) else torch.contiguous_format
    return torch.empty(tuple(shape), device=like.device, dtype=dtype, memory_format=fmt)


def make_desc(x_shape, y_shape, kernel: int, padding, dtype: torch.dtype, x_strides, y_strides) -> ConvDesc:
    d = ConvDesc()
    d.dtype = _DTYPE_CODE[dtype]
    d.n, d.cin, d.d, d.h, d.w = (int(v) for v in x_shape)
    _, d.cout, d.od, d.oh, d.ow = (int(v) for v in y_shape)
    d.kernel = int(kernel)
    d.pad_d, d.pad_h, d.pad_w = (int(p) for p in padding)
    for i in range(5):
        d.x_strides[i] = int(x_strides[i])
        d.y_strides[i] = int(y_strides[i])
    return d


def _workspace(nbytes: int, device: torch.device, what: str) -> torch.Tensor:
    """Workspace of the size the library asked for; a negative size means no
    plan runs this descriptor (NativeUnsupported: the caller falls back)."""
    if nbytes < 0:
        raise NativeUnsupported(f"{what}: no native plan for this descriptor")
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _dense_strides(shape, channels_last: bool):
    """Element strides of a dense NCDHW (or channels_last_3d) tensor of `shape`."""
    n, c, d, h, w = (int(v) for v in shape)
    if channels_last:
        return (d * h * w * c, 1, h * w * c, w * c, c)
    return (c * d * h * w, d * h * w, h * w, w, 1)


def _passed_strides(t: torch.Tensor):
    """Strides of the tensor the entry points pass on (see _dense)."""
    if t.is_contiguous() or is_channels_last(t):
        return tuple(int(v) for v in t.stride())
    return _dense_strides(t.shape, False)


def _out_channels_last(t: torch.Tensor) -> bool:
    return is_channels_last(t) and not t.is_contiguous()


@lru_cache(maxsize=4096)
def _plans_ok(transpose: bool, x_shape, x_strides, y_shape, y_strides, kernel: int, padding, dtype_code: int) -> bool:
    lib = load()
    x_shape = tuple(x_shape)
    d = ConvDesc()
    d.dtype = dtype_code
    d.n, d.cin, d.d, d.h, d.w = x_shape
    _, d.cout, d.od, d.oh, d.ow = y_shape
    d.kernel = kernel
    d.pad_d, d.pad_h, d.pad_w = padding
    for i in range(5):
        d.x_strides[i] = x_strides[i]
        d.y_strides[i] = y_strides[i]
    names = ("convt_k2s2_fwd", "convt_k2s2_dx", "convt_k2s2_dw") if transpose else ("conv3d_fwd", "conv3d_dx",
                                                                                       "conv3d_dw")
    return all(getattr(lib, f"r3c_{nm}_workspace")(ctypes.byref(d)) >= 0 for nm in names)


def conv_plans_ok(x: torch.Tensor, weight_shape, padding, dtype: torch.dtype) -> bool:
    """True when the library has plans for this Conv3d's forward, dX and dW
    (dY assumed in the output's layout, which follows x).  The workspace
    queries return -1 for descriptors no plan runs, e.g. a sample of 1 GiB or
    more (32-bit buffer offsets).  Cached per shape, strides and dtype."""
    n, cin, d, h, w = (int(v) for v in x.shape)
    k = int(weight_shape[2])
    pd = tuple(int(p) for p in padding)
    y_shape = (n, int(weight_shape[0]), d + 2 * pd[0] - k + 1, h + 2 * pd[1] - k + 1, w + 2 * pd[2] - k + 1)
    return _plans_ok(False, tuple(x.shape), _passed_strides(x), y_shape,
                     _dense_strides(y_shape, _out_channels_last(x)), k, pd, _DTYPE_CODE[dtype])


def convt_plans_ok(x: torch.Tensor, weight_shape, dtype: torch.dtype) -> bool:
    """conv_plans_ok for ConvTranspose3d k=2 s=2 (weight (Cin, Cout, 2, 2, 2))."""
    n, cin, d, h, w = (int(v) for v in x.shape)
    y_shape = (n, int(weight_shape[1]), 2 * d, 2 * h, 2 * w)
    return _plans_ok(True, tuple(x.shape), _passed_strides(x), y_shape,
                     _dense_strides(y_shape, _out_channels_last(x)), 2, (0, 0, 0), _DTYPE_CODE[dtype])


# ---------------------------------------------------------------------------
# Conv3d
# ---------------------------------------------------------------------------
def conv3d_fwd(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], padding,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = conv3d(x, weight) + bias; stride 1, k in {1, 3}.  y keeps x's layout."""
    lib = load()
    x = _dense(x)
    weight = weight.contiguous()
    n, cin, d, h, w = _dims5(x)
    cout, k = int(weight.shape[0]), int(weight.shape[2])
    od, oh, ow = (d + 2 * padding[0] - k + 1, h + 2 * padding[1] - k + 1, w + 2 * padding[2] - k + 1)
    y = out if out is not None else _empty_like_layout((n, cout, od, oh, ow), x, x.dtype)
    desc = make_desc(x.shape, y.shape, k, padding, x.dtype, x.stride(), y.stride())
    ws = _workspace(lib.r3c_conv3d_fwd_workspace(ctypes.byref(desc)), x.device, "r3c_conv3d_fwd")
    b = bias.contiguous() if bias is not None else None
    rc = lib.r3c_conv3d_fwd(ctypes.byref(desc), _ptr(x), _ptr(weight), _ptr(b), _ptr(y), _ptr(ws),
                            ws.numel(), _stream_handle(x.device))
    _check(lib, rc, "r3c_conv3d_fwd")
    return y


def conv3d_dx(go: torch.Tensor, weight: torch.Tensor, x_shape, padding, like: torch.Tensor) -> torch.Tensor:
    """dX of a stride-1 Conv3d; dX takes `like`'s memory format."""
    lib = load()
    go = _dense(go)
    weight = weight.contiguous()
    k = int(weight.shape[2])
    gx = _empty_like_layout(tuple(int(v) for v in x_shape), like, go.dtype)
    desc = make_desc(gx.shape, go.shape, k, padding, go.dtype, gx.stride(), go.stride())
    ws = _workspace(lib.r3c_conv3d_dx_workspace(ctypes.byref(desc)), go.device, "r3c_conv3d_dx")
    rc = lib.r3c_conv3d_dx(ctypes.byref(desc), _ptr(go), _ptr(weight), _ptr(gx), _ptr(ws), ws.numel(),
                           _stream_handle(go.device))
    _check(lib, rc, "r3c_conv3d_dx")
    return gx


def conv3d_dw(x: torch.Tensor, go: torch.Tensor, weight_shape, padding, dw_dtype: torch.dtype,
              want_db: bool = False, db_dtype: Optional[torch.dtype] = None):
    """(dW in OIDHW of dw_dtype, db or None).  Deterministic split-K."""
    lib = load()
    x = _dense(x)
    go = _dense(go)
    k = int(weight_shape[2])
    desc = make_desc(x.shape, go.shape, k, padding, x.dtype, x.stride(), go.stride())
    dw = torch.empty(tuple(int(v) for v in weight_shape), device=x.device, dtype=dw_dtype)
    db = None
    if want_db:
        db = torch.empty((int(weight_shape[0]),), device=x.device, dtype=db_dtype or dw_dtype)
    ws = _workspace(lib.r3c_conv3d_dw_workspace(ctypes.byref(desc)), x.device, "r3c_conv3d_dw")
    rc = lib.r3c_conv3d_dw(ctypes.byref(desc), _ptr(x), _ptr(go), _ptr(dw), _DTYPE_CODE[dw_dtype], _ptr(db),
                           _DTYPE_CODE[db.dtype] if db is not None else R3C_F32, _ptr(ws), ws.numel(),
                           _stream_handle(x.device))
    _check(lib, rc, "r3c_conv3d_dw")
    return dw, db


# ---------------------------------------------------------------------------
# Conv3d with stride > 1 (the r3c_conv3d_strided_* entry points)
# ---------------------------------------------------------------------------
def _stride3(stride):
    return (ctypes.c_int32 * 3)(*(int(s) for s in stride))


def strided_out_shape(x_shape, weight_shape, stride, padding):
    n, _, d, h, w = (int(v) for v in x_shape)
    k = int(weight_shape[2])
    sp = [(L + 2 * int(p) - k) // int(s) + 1 for L, p, s in zip((d, h, w), padding, stride)]
    return (n, int(weight_shape[0]), *sp)


@lru_cache(maxsize=4096)
def _strided_plans_ok(x_shape, x_strides, y_shape, y_strides, kernel: int, padding, stride, dtype_code: int) -> bool:
    lib = load()
    d = ConvDesc()
    d.dtype = dtype_code
    d.n, d.cin, d.d, d.h, d.w = x_shape
    _, d.cout, d.od, d.oh, d.ow = y_shape
    d.kernel = kernel
    d.pad_d, d.pad_h, d.pad_w = padding
    for i in range(5):
        d.x_strides[i] = x_strides[i]
        d.y_strides[i] = y_strides[i]
    st = _stride3(stride)
    return all(lib.r3c_conv3d_strided_workspace(ctypes.byref(d), st, p) >= 0 for p in (0, 1, 2))


def strided_plans_ok(x: torch.Tensor, weight_shape, stride, padding, dtype: torch.dtype) -> bool:
    """True when the library has strided forward, dX and dW plans for this
    convolution (dY in the output's layout, which follows x)."""
    y_shape = strided_out_shape(x.shape, weight_shape, stride, padding)
    if min(y_shape[2:]) < 1:
        return False
    return _strided_plans_ok(tuple(int(v) for v in x.shape), _passed_strides(x), y_shape,
                             _dense_strides(y_shape, _out_channels_last(x)), int(weight_shape[2]),
                             tuple(int(p) for p in padding), tuple(int(s) for s in stride), _DTYPE_CODE[dtype])


def conv3d_strided_fwd(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], stride,
                       padding) -> torch.Tensor:
    """y = conv3d(x, weight, stride) + bias, k in {1, 3}; y keeps x's layout."""
    lib = load()
    x = _dense(x)
    weight = weight.contiguous()
    k = int(weight.shape[2])
    y = _empty_like_layout(strided_out_shape(x.shape, weight.shape, stride, padding), x, x.dtype)
    desc = make_desc(x.shape, y.shape, k, padding, x.dtype, x.stride(), y.stride())
    st = _stride3(stride)
    ws = _workspace(lib.r3c_conv3d_strided_workspace(ctypes.byref(desc), st, 0), x.device, "r3c_conv3d_strided_fwd")
    b = bias.contiguous() if bias is not None else None
    rc = lib.r3c_conv3d_strided_fwd(ctypes.byref(desc), st, _ptr(x), _ptr(weight), _ptr(b), _ptr(y), _ptr(ws),
                                    ws.numel(), _stream_handle(x.device))
    _check(lib, rc, "r3c_conv3d_strided_fwd")
    return y


def conv3d_strided_dx(go: torch.Tensor, weight: torch.Tensor, x_shape, stride, padding,
                      like: torch.Tensor) -> torch.Tensor:
    """dX of a strided Conv3d; dX takes `like`'s memory format."""
    lib = load()
    go = _dense(go)
    weight = weight.contiguous()
    k = int(weight.shape[2])
    gx = _empty_like_layout(tuple(int(v) for v in x_shape), like, go.dtype)
    desc = make_desc(gx.shape, go.shape, k, padding, go.dtype, gx.stride(), go.stride())
    st = _stride3(stride)
    ws = _workspace(lib.r3c_conv3d_strided_workspace(ctypes.byref(desc), st, 1), go.device, "r3c_conv3d_strided_dx")
    rc = lib.r3c_conv3d_strided_dx(ctypes.byref(desc), st, _ptr(go), _ptr(weight), _ptr(gx), _ptr(ws), ws.numel(),
                                   _stream_handle(go.device))
    _check(lib, rc, "r3c_conv3d_strided_dx")
    return gx


def conv3d_strided_dw(x: torch.Tensor, go: torch.Tensor, weight_shape, stride, padding, dw_dtype: torch.dtype,
                      want_db: bool = False, db_dtype: Optional[torch.dtype] = None):
    """(dW in OIDHW of dw_dtype, db or None) of a strided Conv3d; deterministic."""
    lib = load()
    x = _dense(x)
    go = _dense(go)
    k = int(weight_shape[2])
    desc = make_desc(x.shape, go.shape, k, padding, x.dtype, x.stride(), go.stride())
    st = _stride3(stride)
    dw = torch.empty(tuple(int(v) for v in weight_shape), device=x.device, dtype=dw_dtype)
    db = None
    if want_db:
        db = torch.empty((int(weight_shape[0]),), device=x.device, dtype=db_dtype or dw_dtype)
    ws = _workspace(lib.r3c_conv3d_strided_workspace(ctypes.byref(desc), st, 2), x.device, "r3c_conv3d_strided_dw")
    rc = lib.r3c_conv3d_strided_dw(ctypes.byref(desc), st, _ptr(x), _ptr(go), _ptr(dw), _DTYPE_CODE[dw_dtype],
                                   _ptr(db), _DTYPE_CODE[db.dtype] if db is not None else R3C_F32, _ptr(ws),
                                   ws.numel(), _stream_handle(x.device))
    _check(lib, rc, "r3c_conv3d_strided_dw")
    return dw, db


# ---------------------------------------------------------------------------
# ConvTranspose3d k=2 s=2
# ---------------------------------------------------------------------------
def convt_fwd(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
    lib = load()
    x = _dense(x)
    weight = weight.contiguous()
    n, cin, d, h, w = _dims5(x)
    cout = int(weight.shape[1])
    y = _empty_like_layout((n, cout, 2 * d, 2 * h, 2 * w), x, x.dtype)
    desc = make_desc(x.shape, y.shape, 2, (0, 0, 0), x.dtype, x.stride(), y.stride())
    ws = _workspace(lib.r3c_convt_k2s2_fwd_workspace(ctypes.byref(desc)), x.device, "r3c_convt_k2s2_fwd")
    b = bias.contiguous() if bias is not None else None
    rc = lib.r3c_convt_k2s2_fwd(ctypes.byref(desc), _ptr(x), _ptr(weight), _ptr(b), _ptr(y), _ptr(ws),
                                ws.numel(), _stream_handle(x.device))
    _check(lib, rc, "r3c_convt_k2s2_fwd")
    return y


def convt_dx(go: torch.Tensor, weight: torch.Tensor, x_shape, like: torch.Tensor) -> torch.Tensor:
    lib = load()
    go = _dense(go)
    weight = weight.contiguous()
    gx = _empty_like_layout(tuple(int(v) for v in x_shape), like, go.dtype)
    desc = make_desc(gx.shape, go.shape, 2, (0, 0, 0), go.dtype, gx.stride(), go.stride())
    ws = _workspace(lib.r3c_convt_k2s2_dx_workspace(ctypes.byref(desc)), go.device, "r3c_convt_k2s2_dx")
    rc = lib.r3c_convt_k2s2_dx(ctypes.byref(desc), _ptr(go), _ptr(weight), _ptr(gx), _ptr(ws), ws.numel(),
                               _stream_handle(go.device))
    _check(lib, rc, "r3c_convt_k2s2_dx")
    return gx


def convt_dw(x: torch.Tensor, go: torch.Tensor, weight_shape, dw_dtype: torch.dtype, want_db: bool = False,
             db_dtype: Optional[torch.dtype] = None):
    lib = load()
    x = _dense(x)
    go = _dense(go)
    desc = make_desc(x.shape, go.shape, 2, (0, 0, 0), x.dtype, x.stride(), go.stride())
    dw = torch.empty(tuple(int(v) for v in weight_shape), device=x.device, dtype=dw_dtype)
    db = None
    if want_db:
        db = torch.empty((int(weight_shape[1]),), device=x.device, dtype=db_dtype or dw_dtype)
    ws = _workspace(lib.r3c_convt_k2s2_dw_workspace(ctypes.byref(desc)), x.device, "r3c_convt_k2s2_dw")
    rc = lib.r3c_convt_k2s2_dw(ctypes.byref(desc), _ptr(x), _ptr(go), _ptr(dw), _DTYPE_CODE[dw_dtype], _ptr(db),
                               _DTYPE_CODE[db.dtype] if db is not None else R3C_F32, _ptr(ws), ws.numel(),
                               _stream_handle(x.device))
    _check(lib, rc, "r3c_convt_k2s2_dw")
    return dw, db


# ---------------------------------------------------------------------------
# BatchNorm3d + ReLU (NCDHW planes)
# ---------------------------------------------------------------------------
def bn_plane_ok(t: torch.Tensor) -> bool:
    """A 5-D tensor whose (sample, channel) planes are contiguous runs of D*H*W
    positions, with sizes, strides and address the 16-byte kernels accept."""
    if t.dim() != 5 or t.dtype not in _DTYPE_CODE:
        return False
    n, c, d, h, w = (int(v) for v in t.shape)
    s = d * h * w
    st = t.stride()
    if not (st[4] == 1 and (w == 1 or st[3] == w) and (h == 1 or st[2] == h * w)):
        return False
    vec = 4 if t.dtype == torch.float32 else 8
    return s % vec == 0 and st[0] % vec == 0 and st[1] % vec == 0 and t.data_ptr() % 16 == 0


def _bn_desc(y: torch.Tensor, g: Optional[torch.Tensor], o: torch.Tensor, training: bool, eps: float,
             momentum: float) -> BnDesc:
    d = BnDesc()
    d.dtype = _DTYPE_CODE[y.dtype]
    d.n, d.c = int(y.shape[0]), int(y.shape[1])
    d.s = int(y.shape[2] * y.shape[3] * y.shape[4])
    d.y_strides[0], d.y_strides[1] = int(y.stride(0)), int(y.stride(1))
    gg = g if g is not None else y
    d.g_strides[0], d.g_strides[1] = int(gg.stride(0)), int(gg.stride(1))
    d.o_strides[0], d.o_strides[1] = int(o.stride(0)), int(o.stride(1))
    d.training = 1 if training else 0
    d.eps = float(eps)
    d.momentum = float(momentum)
    return d


def bn_relu_fwd(y: torch.Tensor, gamma, beta, running_mean, running_var, training: bool, momentum: float,
                eps: float):
    """(z, save_mean, save_invstd): z = relu(batchnorm(y)) in y's dtype, NCDHW."""
    lib = load()
    z = torch.empty(y.shape, device=y.device, dtype=y.dtype)
    c = int(y.shape[1])
    save_mean = torch.empty(c, device=y.device, dtype=torch.float32)
    save_invstd = torch.empty(c, device=y.device, dtype=torch.float32)
    d = _bn_desc(y, None, z, training, eps, momentum)
    ws = _workspace(lib.r3c_bn_relu_workspace(ctypes.byref(d)), y.device, "r3c_bn_relu_fwd")
    rc = lib.r3c_bn_relu_fwd(ctypes.byref(d), _ptr(y), _ptr(gamma), _ptr(beta), _ptr(running_mean),
                             _ptr(running_var), _ptr(z), _ptr(save_mean), _ptr(save_invstd), _ptr(ws), ws.numel(),
                             _stream_handle(y.device))
    _check(lib, rc, "r3c_bn_relu_fwd")
    return z, save_mean, save_invstd


def bn_relu_bwd(dz: torch.Tensor, y: torch.Tensor, gamma, beta, save_mean, save_invstd, training: bool,
                want_dgamma: bool, want_dbeta: bool):
    """(dy, dgamma or None, dbeta or None) of z = relu(batchnorm(y))."""
    lib = load()
    dy = torch.empty(y.shape, device=y.device, dtype=y.dtype)
    c = int(y.shape[1])
    dgamma = torch.empty(c, device=y.device, dtype=torch.float32) if want_dgamma else None
    dbeta = torch.empty(c, device=y.device, dtype=torch.float32) if want_dbeta else None
    d = _bn_desc(y, dz, dy, training, 0.0, 0.0)
    ws = _workspace(lib.r3c_bn_relu_workspace(ctypes.byref(d)), y.device, "r3c_bn_relu_bwd")
    rc = lib.r3c_bn_relu_bwd(ctypes.byref(d), _ptr(dz), _ptr(y), _ptr(gamma), _ptr(beta), _ptr(save_mean),
                             _ptr(save_invstd), _ptr(dy), _ptr(dgamma), _ptr(dbeta), _ptr(ws), ws.numel(),
                             _stream_handle(y.device))
    _check(lib, rc, "r3c_bn_relu_bwd")
    return dy, dgamma, dbeta


# ---------------------------------------------------------------------------
# MaxPool3d(2)
# ---------------------------------------------------------------------------
def pool_ok(t: torch.Tensor) -> bool:
    """A tensor the MaxPool3d(2) kernels take: dense (d, h, w) planes, even d
    and h, w a multiple of 8, strides and address allowing 16-byte vectors."""
    if t.dim() != 5 or t.dtype not in _DTYPE_CODE:
        return False
    n, c, d, h, w = (int(v) for v in t.shape)
    st = t.stride()
    if not (st[4] == 1 and st[3] == w and st[2] == h * w):
        return False
    vec = 4 if t.dtype == torch.float32 else 8
    return (d % 2 == 0 and h % 2 == 0 and w % 8 == 0 and st[0] % vec == 0 and st[1] % vec == 0
            and t.data_ptr() % 16 == 0)


def _pool_desc(x_shape, x_strides, y_strides, dtype) -> PoolDesc:
    d = PoolDesc()
    d.dtype = _DTYPE_CODE[dtype]
    d.n, d.c, d.d, d.h, d.w = (int(v) for v in x_shape)
    d.x_strides[0], d.x_strides[1] = int(x_strides[0]), int(x_strides[1])
    d.y_strides[0], d.y_strides[1] = int(y_strides[0]), int(y_strides[1])
    return d


def maxpool2_fwd(x: torch.Tensor):
    """(y, idx): MaxPool3d(2) of x and the one-byte window index of each maximum."""
    lib = load()
    n, c, d, h, w = (int(v) for v in x.shape)
    y = torch.empty((n, c, d // 2, h // 2, w // 2), device=x.device, dtype=x.dtype)
    idx = torch.empty((n, c, d // 2, h // 2, w // 2), device=x.device, dtype=torch.uint8)
    desc = _pool_desc(x.shape, x.stride(), y.stride(), x.dtype)
    rc = lib.r3c_maxpool2_fwd(ctypes.byref(desc), _ptr(x), _ptr(y), _ptr(idx), _stream_handle(x.device))
    _check(lib, rc, "r3c_maxpool2_fwd")
    return y, idx


def maxpool2_bwd(dy: torch.Tensor, idx: torch.Tensor, x_shape, add: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dx of MaxPool3d(2) (NCDHW, every element written), plus `add` (a
    gradient of x from another consumer, pool_ok layout) when given."""
    lib = load()
    dx = torch.empty(tuple(int(v) for v in x_shape), device=dy.device, dtype=dy.dtype)
    desc = _pool_desc(dx.shape, dx.stride(), dy.stride(), dy.dtype)
    if add is None:
        rc = lib.r3c_maxpool2_bwd(ctypes.byref(desc), _ptr(dy), _ptr(idx), _ptr(dx), _stream_handle(dy.device))
    else:
        st = (ctypes.c_int64 * 2)(int(add.stride(0)), int(add.stride(1)))
        rc = lib.r3c_maxpool2_bwd_add(ctypes.byref(desc), _ptr(dy), _ptr(idx), _ptr(add), st, _ptr(dx),
                                      _stream_handle(dy.device))
    _check(lib, rc, "r3c_maxpool2_bwd")
    return dx


# ---------------------------------------------------------------------------
# Conv3d over a channel concatenation [a, b] (no torch.cat)
# ---------------------------------------------------------------------------
def cat_tensors_ok(xa: torch.Tensor, xb: torch.Tensor) -> bool:
    """Pairs the concatenation entry points take: contiguous NCDHW, same
    dtype, device and (n, d, h, w), a's channels a multiple of 8, 16-byte
    aligned."""
    if xa.dim() != 5 or xb.dim() != 5 or xa.dtype != xb.dtype or xa.device != xb.device:
        return False
    if xa.shape[0] != xb.shape[0] or xa.shape[2:] != xb.shape[2:] or int(xa.shape[1]) % 8:
        return False
    return (xa.is_contiguous() and xb.is_contiguous() and xa.data_ptr() % 16 == 0 and xb.data_ptr() % 16 == 0
            and xa.numel() > 0 and xb.numel() > 0)


def _cat_desc(xa_shape, cb: int, y_shape, k: int, padding, dtype, y_strides) -> ConvDesc:
    n, ca, d, h, w = (int(v) for v in xa_shape)
    x_shape = (n, ca + int(cb), d, h, w)
    xs = _dense_strides((n, ca, d, h, w), False)
    return make_desc(x_shape, y_shape, k, padding, dtype, xs, y_strides)


@lru_cache(maxsize=1024)
def _cat_plans_ok(xa_shape, cb: int, y_shape, padding, dtype_code: int) -> bool:
    lib = load()
    d = _cat_desc(xa_shape, cb, y_shape, 3, padding, torch.bfloat16, _dense_strides(y_shape, False))
    d.dtype = dtype_code
    xb_s0 = int(cb) * int(xa_shape[2]) * int(xa_shape[3]) * int(xa_shape[4])
    return all(lib.r3c_conv3d_cat_workspace(ctypes.byref(d), int(xa_shape[1]), xb_s0, p) >= 0 for p in (0, 1, 2))


def cat_plans_ok(xa: torch.Tensor, xb: torch.Tensor, weight_shape, padding, dtype: torch.dtype) -> bool:
    """True when all three passes of a k=3 Conv3d over cat(xa, xb) have plans."""
    n, ca, d, h, w = (int(v) for v in xa.shape)
    pd = tuple(int(v) for v in padding)
    y_shape = (n, int(weight_shape[0]), d + 2 * pd[0] - 2, h + 2 * pd[1] - 2, w + 2 * pd[2] - 2)
    return _cat_plans_ok(tuple(int(v) for v in xa.shape), int(xb.shape[1]), y_shape, pd, _DTYPE_CODE[dtype])


def conv3d_cat_fwd(xa, xb, weight, bias, padding):
    """conv3d(cat((xa, xb), 1), weight) + bias, k = 3, without the concatenation."""
    lib = load()
    weight = weight.contiguous()
    n, ca, d, h, w = _dims5(xa)
    cout = int(weight.shape[0])
    y = torch.empty((n, cout, d + 2 * padding[0] - 2, h + 2 * padding[1] - 2, w + 2 * padding[2] - 2),
                    device=xa.device, dtype=xa.dtype)
    desc = _cat_desc(xa.shape, xb.shape[1], y.shape, 3, padding, xa.dtype, y.stride())
    xb_s0 = int(xb.stride(0))
    ws = _workspace(lib.r3c_conv3d_cat_workspace(ctypes.byref(desc), ca, xb_s0, 0), xa.device, "r3c_conv3d_cat_fwd")
    b = bias.contiguous() if bias is not None else None
    rc = lib.r3c_conv3d_cat_fwd(ctypes.byref(desc), ca, _ptr(xa), _ptr(xb), xb_s0, _ptr(weight), _ptr(b), _ptr(y),
                                _ptr(ws), ws.numel(), _stream_handle(xa.device))
    _check(lib, rc, "r3c_conv3d_cat_fwd")
    return y


def conv3d_cat_dx(go, weight, xa_shape, xb_shape, padding):
    """(dxa, dxb): the dX of a k=3 Conv3d over cat(xa, xb), split by channels."""
    lib = load()
    go = go.contiguous()
    weight = weight.contiguous()
    dxa = torch.empty(tuple(int(v) for v in xa_shape), device=go.device, dtype=go.dtype)
    dxb = torch.empty(tuple(int(v) for v in xb_shape), device=go.device, dtype=go.dtype)
    ca = int(xa_shape[1])
    desc = _cat_desc(xa_shape, xb_shape[1], go.shape, 3, padding, go.dtype, go.stride())
    xb_s0 = int(dxb.stride(0))
    ws = _workspace(lib.r3c_conv3d_cat_workspace(ctypes.byref(desc), ca, xb_s0, 1), go.device, "r3c_conv3d_cat_dx")
    rc = lib.r3c_conv3d_cat_dx(ctypes.byref(desc), ca, _ptr(go), _ptr(weight), _ptr(dxa), _ptr(dxb), xb_s0, _ptr(ws),
                               ws.numel(), _stream_handle(go.device))
    _check(lib, rc, "r3c_conv3d_cat_dx")
    return dxa, dxb


def conv3d_cat_dw(xa, xb, go, weight_shape, padding, dw_dtype, want_db=False, db_dtype=None):
    """(dW, db or None) of a k=3 Conv3d over cat(xa, xb)."""
    lib = load()
    go = go.contiguous()
    ca = int(xa.shape[1])
    desc = _cat_desc(xa.shape, xb.shape[1], go.shape, 3, padding, xa.dtype, go.stride())
    dw = torch.empty(tuple(int(v) for v in weight_shape), device=xa.device, dtype=dw_dtype)
    db = None
    if want_db:
        db = torch.empty((int(weight_shape[0]),), device=xa.device, dtype=db_dtype or dw_dtype)
    xb_s0 = int(xb.stride(0))
    ws = _workspace(lib.r3c_conv3d_cat_workspace(ctypes.byref(desc), ca, xb_s0, 2), xa.device, "r3c_conv3d_cat_dw")
    rc = lib.r3c_conv3d_cat_dw(ctypes.byref(desc), ca, _ptr(xa), _ptr(xb), xb_s0, _ptr(go), _ptr(dw),
                               _DTYPE_CODE[dw_dtype], _ptr(db), _DTYPE_CODE[db.dtype] if db is not None else R3C_F32,
                               _ptr(ws), ws.numel(), _stream_handle(xa.device))
    _check(lib, rc, "r3c_conv3d_cat_dw")
    return dw, db


def probe_mfma(shape: int, blocks: int, iters: int, out: torch.Tensor) -> None:
    """Launch the MFMA shape probe on out's device (see include/rdna4_conv3d.h)."""
    lib = load()
    rc = lib.r3c_probe_mfma(int(shape), int(blocks), int(iters), _ptr(out), _stream_handle(out.device))
    _check(lib, rc, "r3c_probe_mfma")
