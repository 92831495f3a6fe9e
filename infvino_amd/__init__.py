"""infvino_amd: MI355X (gfx950) HIP backend for infvino plans.

Python mirror of the reference's host interface, bound through the C ABI of
libinfvino_hip.so (include/ivh.h):
  PlanModel   <-> infvino::PlanModel (include/infvino/PlanModel.hpp:57-234)
  HipBackend  <-> infvino::ClBackend (include/infvino/ClBackend.hpp:29-53)
  Tensor      <-> infvino::Tensor    (include/infvino/Tensor.hpp:15-45)
Same method names, argument meaning and error behaviour (RuntimeError with the
reference's message).  The extra `batch` arguments run `batch` images per call.

There is no CPU fallback: if the HIP library is missing or fails to load, every
entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libinfvino_hip.so")

IVH_FLAG_NO_GRAPH = 0x1
IVH_FLAG_NO_REUSE = 0x2
IVH_FLAG_NO_FUSE = 0x4
IVH_FLAG_NCHW_ONLY = 0x8
IVH_FLAG_DIRECT_ONLY = 0x10
IVH_FLAG_ASYNC = 0x20
IVH_FLAG_DRY_RUN = 0x40
IVH_FLAG_NO_SPLITK = 0x80
IVH_FLAG_NO_HALO = 0x100
IVH_FLAG_NO_RESIDENT = 0x200
IVH_FLAG_NO_FUSE_DECODE = 0x400
IVH_FLAG_PROFILE = 0x800
IVH_FLAG_NO_FUSE_ATTN = 0x1000
IVH_FLAG_NO_PIPE = 0x2000
IVH_FLAG_PIPE_ANY = 0x4000
IVH_FLAG_NO_FUSE_PAIR = 0x8000
IVH_FLAG_NO_S2_PERSIST = 0x10000
IVH_FLAG_NO_PW = 0x20000
IVH_FLAG_NO_WIDE = 0x40000
IVH_FLAG_NO_PINGPONG = 0x80000
IVH_FLAG_NO_FUSE_UPSAMPLE = 0x100000
IVH_FLAG_NO_FUSE_SIBLINGS = 0x200000

# every symbol include/ivh.h declares, with (restype, argtypes)
_vp, _i, _u32, _sz, _d = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t, C.c_double
_ip, _szp, _dp, _i64p = C.POINTER(C.c_int), C.POINTER(C.c_size_t), C.POINTER(C.c_double), C.POINTER(C.c_int64)
class ConvDesc(C.Structure):
    """ivh_conv_desc (include/ivh.h)."""
    _fields_ = [(n, C.c_int) for n in ("cin", "cout", "h", "w", "k", "stride", "pad", "groups", "act",
                                       "has_bias", "channels_last")]


_cdp = C.POINTER(ConvDesc)

SIGNATURES = {
    "ivh_last_error": (C.c_char_p, []),
    "ivh_version": (_i, [_ip, _ip]),
    "ivh_device_count": (_i, [_ip]),
    "ivh_device_info": (_i, [_i, C.c_char_p, _sz, _ip, _ip]),
    "ivh_runtime_version": (_i, [C.c_char_p, _sz]),
    "ivh_create": (_i, [C.c_char_p, _i, _i, _u32, C.POINTER(_vp)]),
    "ivh_destroy": (_i, [_vp]),
    "ivh_input_dims": (_i, [_vp, _i64p, _ip]),
    "ivh_input_numel": (_i, [_vp, _szp]),
    "ivh_output_count": (_i, [_vp, _ip]),
    "ivh_output_dims": (_i, [_vp, _i, _i64p, _ip]),
    "ivh_output_numel": (_i, [_vp, _i, _szp]),
    "ivh_max_batch": (_i, [_vp, _ip]),
    "ivh_set_input_f16": (_i, [_vp, _vp, _i]),
    "ivh_set_input_f32": (_i, [_vp, _vp, _i]),
    "ivh_set_input_f32_noalloc": (_i, [_vp, _vp, _i]),
    "ivh_run": (_i, [_vp, _i]),
    "ivh_sync": (_i, [_vp]),
    "ivh_read_output_f16": (_i, [_vp, _i, _vp, _i]),
    "ivh_read_output_f32": (_i, [_vp, _i, _vp, _i]),
    "ivh_read_tensor_f16": (_i, [_vp, C.c_char_p, _vp, _i]),
    "ivh_tensor_numel": (_i, [_vp, C.c_char_p, _szp]),
    "ivh_last_run_ms": (_i, [_vp, _dp]),
    "ivh_node_count": (_i, [_vp, _ip]),
    "ivh_profile_nodes": (_i, [_vp, _i, _i, _dp, _i]),
    "ivh_node_times": (_i, [_vp, _dp, _ip, _i]),
    "ivh_clear_profile": (_i, [_vp]),
    "ivh_node_info": (_i, [_vp, _i, C.c_char_p, _sz, C.c_char_p, _sz, C.c_char_p, _sz, _dp, _dp]),
    "ivh_node_tag": (_i, [_vp, _i, C.c_char_p, _sz]),
    "ivh_memory_info": (_i, [_vp, _i, _szp, _szp]),
    # single-op entry points (device pointers as integers, stream None = null stream)
    "ivh_conv_out_dims": (_i, [_cdp, _ip, _ip]),
    "ivh_conv_packed_bytes": (_i, [_cdp, _szp]),
    "ivh_pack_conv_weights": (_i, [_cdp, _vp, _vp, _vp]),
    "ivh_conv2d_f16": (_i, [_cdp, _vp, _vp, _vp, _vp, _i, _vp]),
    "ivh_dwconv_f16": (_i, [_cdp, _vp, _vp, _vp, _vp, _i, _vp]),
    "ivh_gemv_f16": (_i, [_cdp, _vp, _vp, _vp, _i, _vp]),
    "ivh_eltwise_f16": (_i, [_i, _vp, _vp, _i, _vp, _sz, _i, _vp]),
    "ivh_pool_f16": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "ivh_softmax_f16": (_i, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "ivh_bmm_f16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
}

_lib = None


def lib():
    """Loads libinfvino_hip.so; raises if it is absent (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"infvino_amd: HIP library not built: {LIB_PATH} "
                               "(run __graft_entry__.build() or make -C infvino_amd/csrc)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib().ivh_last_error().decode(errors="replace"))


def device_count() -> int:
    n = C.c_int(0)
    _check(lib().ivh_device_count(C.byref(n)))
    return n.value


def device_info(device: int = 0) -> dict:
    name = C.create_string_buffer(256)
    cu, mhz = C.c_int(), C.c_int()
    _check(lib().ivh_device_info(device, name, 256, C.byref(cu), C.byref(mhz)))
    return {"name": name.value.decode(), "compute_units": cu.value, "clock_mhz": mhz.value}


def _dims(fn, *args):
    rank = C.c_int(8)
    buf = (C.c_int64 * 8)()
    _check(fn(*args, buf, C.byref(rank)))
    return [int(buf[i]) for i in range(rank.value)]


def _u16(a, n):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    if a.dtype != np.uint16 or a.size != n:
        raise RuntimeError(f"expected {n} fp16 values, got {a.size} of {a.dtype}")
    return a


class PlanModel:
    """Executes a plan on one GPU (infvino::PlanModel, include/infvino/PlanModel.hpp:57-234)."""

    def __init__(self, plan_path: str, device: int = 0, max_batch: int = 1, flags: int = 0):
        self._h = C.c_void_p()
        _check(lib().ivh_create(plan_path.encode(), device, max_batch, flags, C.byref(self._h)))
        self.plan_path = plan_path
        self.max_batch = max_batch

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().ivh_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- shape queries ------------------------------------------------------
    def inputDims(self):
        return _dims(lib().ivh_input_dims, self._h)

    def inputNumel(self) -> int:
        n = C.c_size_t()
        _check(lib().ivh_input_numel(self._h, C.byref(n)))
        return n.value

    def outputCount(self) -> int:
        n = C.c_int()
        _check(lib().ivh_output_count(self._h, C.byref(n)))
        return n.value

    def outputDims(self, i: int):
        return _dims(lib().ivh_output_dims, self._h, i)

    def outputNumel(self, i: int) -> int:
        n = C.c_size_t()
        _check(lib().ivh_output_numel(self._h, i, C.byref(n)))
        return n.value

    def tensorNumel(self, name: str) -> int:
        n = C.c_size_t()
        _check(lib().ivh_tensor_numel(self._h, name.encode(), C.byref(n)))
        return n.value

    # -- execution ----------------------------------------------------------
    def setInput(self, fp16, batch: int = 1):
        a = _u16(fp16, self.inputNumel() * batch)
        _check(lib().ivh_set_input_f16(self._h, a.ctypes.data, batch))

    def setInputF32(self, f32, batch: int = 1):
        a = np.ascontiguousarray(f32, dtype=np.float32)
        if a.size != self.inputNumel() * batch:
            raise RuntimeError(f"input numel mismatch: got {a.size}, expected {self.inputNumel() * batch}")
        _check(lib().ivh_set_input_f32(self._h, a.ctypes.data, batch))

    def run(self, batch: int = 1):
        _check(lib().ivh_run(self._h, batch))

    def sync(self):
        _check(lib().ivh_sync(self._h))

    def readOutput(self, i: int, batch: int = 1) -> np.ndarray:
        out = np.empty(self.outputNumel(i) * batch, np.uint16)
        _check(lib().ivh_read_output_f16(self._h, i, out.ctypes.data, batch))
        return out

    def readOutputF32(self, i: int, batch: int = 1) -> np.ndarray:
        out = np.empty(self.outputNumel(i) * batch, np.float32)
        _check(lib().ivh_read_output_f32(self._h, i, out.ctypes.data, batch))
        return out

    def readTensor(self, name: str, batch: int = 1):
        """fp16 NCHW copy of any declared tensor, or None for an unknown name."""
        n = self.tensorNumel(name)
        if n == 0:
            return None
        out = np.empty(n * batch, np.uint16)
        _check(lib().ivh_read_tensor_f16(self._h, name.encode(), out.ctypes.data, batch))
        return out

    def lastRunMs(self) -> float:
        v = C.c_double()
        _check(lib().ivh_last_run_ms(self._h, C.byref(v)))
        return v.value

    # -- profiling ----------------------------------------------------------
    def nodeCount(self) -> int:
        n = C.c_int()
        _check(lib().ivh_node_count(self._h, C.byref(n)))
        return n.value

    def profileNodes(self, batch: int = 1, iters: int = 5) -> np.ndarray:
        n = self.nodeCount()
        buf = (C.c_double * n)()
        _check(lib().ivh_profile_nodes(self._h, batch, iters, buf, n))
        return np.array(buf[:], np.float64)

    def nodeInfo(self, i: int) -> dict:
        op, kern, desc = C.create_string_buffer(64), C.create_string_buffer(64), C.create_string_buffer(256)
        fl, by = C.c_double(), C.c_double()
        _check(lib().ivh_node_info(self._h, i, op, 64, kern, 64, desc, 256, C.byref(fl), C.byref(by)))
        return {"op": op.value.decode(), "kernel": kern.value.decode(), "desc": desc.value.decode(),
                "flops": fl.value, "bytes": by.value}

    def nodeTag(self, i: int) -> str:
        """Kernel label plus launch detail (tile config, K step, split, build) of node i."""
        t = C.create_string_buffer(256)
        _check(lib().ivh_node_tag(self._h, i, t, 256))
        return t.value.decode()

    def memoryInfo(self, batch: int = 1):
        a, w = C.c_size_t(), C.c_size_t()
        _check(lib().ivh_memory_info(self._h, batch, C.byref(a), C.byref(w)))
        return a.value, w.value


@dataclass
class Tensor:
    """infvino::Tensor: shape + row-major f32 data (include/infvino/Tensor.hpp:15-45)."""
    shape: list
    data: np.ndarray = field(repr=False)

    def numel(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1


class HipBackend:
    """Drop-in for infvino::ClBackend (include/infvino/ClBackend.hpp:29-53; src/ClBackend.cpp:13-65):
    f32 NCHW blob in, fp16 on the device, f32 Tensors out.  infer() accepts B images
    (numel = B * prod(inputDims())) up to max_batch; B = 1 is the reference behaviour."""

    def __init__(self, plan: str, device: int = 0, max_batch: int = 1, flags: int = 0):
        if not plan:
            raise RuntimeError("HipBackend: ModelInfo.plan is empty")
        self.model = PlanModel(plan, device, max_batch, flags)
        self._in_dims = self.model.inputDims()
        self._out_shapes = [self.model.outputDims(i) for i in range(self.model.outputCount())]
        self._last = 0.0

    def inputDims(self):
        return list(self._in_dims)

    def outputShapes(self):
        return [list(s) for s in self._out_shapes]

    def lastInferMs(self) -> float:
        return self._last

    @staticmethod
    def image(batched, b: int, batch: int):
        """Image b of a B-image infer() result, each tensor with dim 0 divided by B, so
        per-image consumers (the reference's PoseDecoder / nms read a [1, C, N] tensor)
        run unchanged on each image of a batched inference."""
        if batch < 1 or b < 0 or b >= batch:
            raise RuntimeError("HipBackend: image index out of range")
        out = []
        for t in batched:
            flat = np.asarray(t.data).ravel()
            if not t.shape or flat.size % batch or t.shape[0] % batch:
                raise RuntimeError("HipBackend: tensor does not hold the batch")
            per = flat.size // batch
            shape = [t.shape[0] // batch] + list(t.shape[1:])
            out.append(Tensor(shape, flat[per * b:per * (b + 1)].reshape(shape)))
        return out

    def infer(self, input_f32, numel: int | None = None):
        x = np.ascontiguousarray(input_f32, dtype=np.float32).ravel()
        numel = x.size if numel is None else numel
        per = self.model.inputNumel()
        if numel == 0 or numel % per or numel // per > self.model.max_batch:
            raise RuntimeError(f"HipBackend: input numel mismatch: got {numel}, expected {per}")
        b = numel // per
        self.model.setInputF32(x[:numel], b)
        self.model.run(b)
        self._last = self.model.lastRunMs()
        outs = []
        for i, s in enumerate(self._out_shapes):
            d = self.model.readOutputF32(i, b)
            shape = list(s) if b == 1 else [b * s[0]] + list(s[1:])
            outs.append(Tensor(shape, d.reshape(shape) if shape else d))
        return outs
