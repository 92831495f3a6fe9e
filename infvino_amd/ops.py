"""Single-op entry points of the C ABI (include/ivh.h) for Python callers: one operation on
device buffers the caller owns, given as integer device pointers (e.g. a torch tensor's
data_ptr()), enqueued on `stream` (a hipStream_t as an integer, None for the null stream).
The op-level counterpart of the reference's scripts/kernel_check.py driving one kernel at a
time.  Every call raises RuntimeError with the library's message on failure."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ConvDesc, _check, lib

ACT_NONE, ACT_SILU, ACT_RELU, ACT_HSWISH, ACT_HSIGMOID, ACT_SIGMOID = range(6)
EW_ADD, EW_SUB, EW_MUL, EW_DIV = range(4)
POOL_MAX, POOL_RESIZE = 0, 1


def conv_desc(cin, cout, h, w, k=1, stride=1, pad=0, groups=1, act=ACT_NONE, has_bias=True,
              channels_last=True) -> ConvDesc:
    return ConvDesc(cin, cout, h, w, k, stride, pad, groups, act, int(bool(has_bias)), int(bool(channels_last)))


def conv_out_dims(d: ConvDesc):
    ho, wo = C.c_int(), C.c_int()
    _check(lib().ivh_conv_out_dims(C.byref(d), C.byref(ho), C.byref(wo)))
    return ho.value, wo.value


def conv_packed_bytes(d: ConvDesc) -> int:
    n = C.c_size_t()
    _check(lib().ivh_conv_packed_bytes(C.byref(d), C.byref(n)))
    return n.value


def pack_conv_weights(d: ConvDesc, w: np.ndarray, bias: np.ndarray | None, packed_dev: int) -> None:
    """w: plan-order fp16 bits [cout][cin/groups][k][k]; bias: fp16 bits [cout] or None."""
    w = np.ascontiguousarray(w, np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, np.uint16)
    _check(lib().ivh_pack_conv_weights(C.byref(d), w.ctypes.data_as(C.c_void_p),
                                       None if b is None else b.ctypes.data_as(C.c_void_p), C.c_void_p(packed_dev)))


def _vp(p):
    return None if p is None else C.c_void_p(p)


def conv2d(d: ConvDesc, x: int, packed: int, res: int | None, y: int, batch: int, stream=None) -> None:
    _check(lib().ivh_conv2d_f16(C.byref(d), _vp(x), _vp(packed), _vp(res), _vp(y), batch, _vp(stream)))


def dwconv(d: ConvDesc, x: int, packed: int, res: int | None, y: int, batch: int, stream=None) -> None:
    _check(lib().ivh_dwconv_f16(C.byref(d), _vp(x), _vp(packed), _vp(res), _vp(y), batch, _vp(stream)))


def gemv(d: ConvDesc, x: int, packed: int, y: int, batch: int, stream=None) -> None:
    _check(lib().ivh_gemv_f16(C.byref(d), _vp(x), _vp(packed), _vp(y), batch, _vp(stream)))


def eltwise(op: int, a: int, b: int | None, y: int, n: int, batch: int, b_scalar=False, stream=None) -> None:
    _check(lib().ivh_eltwise_f16(op, _vp(a), _vp(b), int(b_scalar), _vp(y), n, batch, _vp(stream)))


def pool(kind: int, x: int, y: int, c: int, h: int, w: int, k: int, s: int, p: int, batch: int, stream=None) -> None:
    _check(lib().ivh_pool_f16(kind, _vp(x), _vp(y), c, h, w, k, s, p, batch, _vp(stream)))


def softmax(x: int, y: int, outer: int, axis: int, inner: int, batch: int, stream=None) -> None:
    _check(lib().ivh_softmax_f16(_vp(x), _vp(y), outer, axis, inner, batch, _vp(stream)))


def bmm(a: int, b: int, y: int, bb: int, m: int, k: int, n: int, batch: int, stream=None) -> None:
    _check(lib().ivh_bmm_f16(_vp(a), _vp(b), _vp(y), bb, m, k, n, batch, _vp(stream)))
