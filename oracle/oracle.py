"""CPU oracle for infvino's plan-driven conv/GEMM hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, as the checker.  The product (infvino_amd) never
imports this module.

* `lib()` loads liboracle.so (oracle/ivo_oracle.c), the C restatement of the
  reference kernels' arithmetic.
* `Plan` parses the reference's text plan format (include/infvino/PlanModel.hpp:5-12,
  parser src/PlanModel.cpp:447-573) with no fusion and no layout change.
* `run_plan()` executes a plan image by image in NCHW fp16 storage, dispatching
  each node to the restatement of the reference kernel that src/PlanModel.cpp's
  run() (3127-4178) would launch for it with no tuning cache present.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32, REF = 0, 1

_lib = None


def build() -> None:
    """Compiles liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        vp = C.c_void_p
        ci, cl = C.c_int, C.c_long
        L.ivo_h2f.argtypes = [C.c_uint16]
        L.ivo_h2f.restype = C.c_float
        L.ivo_f2h.argtypes = [C.c_float]
        L.ivo_f2h.restype = C.c_uint16
        L.ivo_f2h_trunc.argtypes = [C.c_float]
        L.ivo_f2h_trunc.restype = C.c_uint16
        L.ivo_act.argtypes = [C.c_float, ci]
        L.ivo_act.restype = C.c_float
        for n in ("ivo_f32_to_f16_trunc_bulk", "ivo_f32_to_f16_rne_bulk"):
            getattr(L, n).argtypes = [f32p, u16p, cl]
        L.ivo_f16_to_f32_bulk.argtypes = [u16p, f32p, cl]
        L.ivo_conv2d.argtypes = [u16p, ci, ci, ci, u16p, ci, ci, ci, ci, ci, vp, vp, u16p,
                                 ci, ci, ci, ci, ci]
        L.ivo_ew_binary.argtypes = [u16p, u16p, u16p, cl, ci, ci]
        L.ivo_ew_binary_bcast.argtypes = [u16p, u16p, u16p, cl, ci, ci, i32p]
        L.ivo_ew_unary.argtypes = [u16p, u16p, cl, ci]
        L.ivo_bias_add.argtypes = [u16p, u16p, u16p, cl, ci]
        L.ivo_copy_c.argtypes = [u16p, u16p, ci, ci, ci, ci]
        L.ivo_slice_axis.argtypes = [u16p, u16p, ci, ci, ci, ci, ci]
        L.ivo_concat4.argtypes = [vp, ci, vp, ci, vp, ci, vp, ci, u16p, ci, ci]
        L.ivo_maxpool.argtypes = [u16p, u16p] + [ci] * 8
        L.ivo_resize_nn.argtypes = [u16p, u16p, ci, ci, ci, ci]
        L.ivo_softmax_axis.argtypes = [u16p, u16p, ci, ci, ci]
        L.ivo_permute_0213.argtypes = [u16p, u16p, ci, ci, ci, ci]
        L.ivo_gap.argtypes = [u16p, u16p, ci, ci]
        L.ivo_bmm.argtypes = [u16p, u16p, u16p, ci, ci, ci, ci]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ------------------------------------------------------------------ f16 helpers

def f2h_trunc(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().ivo_f32_to_f16_trunc_bulk(x, out, x.size)
    return out


def f2h(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().ivo_f32_to_f16_rne_bulk(x, out, x.size)
    return out


def h2f(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().ivo_f16_to_f32_bulk(h, out, h.size)
    return out


# ------------------------------------------------------------------ single ops

def conv2d(x, w, bias, res, Cin, H, W, Cout, K, S, P, G, Ho, Wo, act, mode=F32, family=0):
    """One image: x [Cin*H*W] u16, w [Cout*(Cin/G)*K*K] u16 -> y [Cout*Ho*Wo] u16."""
    y = np.empty(Cout * Ho * Wo, np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, np.uint16)
    r = None if res is None else np.ascontiguousarray(res, np.uint16)
    lib().ivo_conv2d(np.ascontiguousarray(x, np.uint16), Cin, H, W,
                     np.ascontiguousarray(w, np.uint16), Cout, K, S, P, G,
                     _ptr(b), _ptr(r), y, Ho, Wo, act, mode, family)
    return y


# ------------------------------------------------------------------ plan model

@dataclass
class Node:
    op: str
    ins: list
    outs: list
    attr: dict = field(default_factory=dict)

    def i(self, key, default=0):
        v = self.attr.get(key)
        return default if v is None else int(v)


@dataclass
class Plan:
    """A parsed plan: the grammar of include/infvino/PlanModel.hpp:5-12."""
    path: str
    input_name: str = ""
    input_dims: list = field(default_factory=list)
    dims: dict = field(default_factory=dict)
    inits: dict = field(default_factory=dict)       # name -> u16 array
    nodes: list = field(default_factory=list)
    outputs: list = field(default_factory=list)

    @staticmethod
    def load(path: str) -> "Plan":
        p = Plan(path)
        pdir = os.path.dirname(os.path.abspath(path))
        with open(path) as f:
            for line in f:
                line = line.strip()
                if not line or line.startswith("#"):
                    continue
                tok = line.split()
                kind = tok[0]
                if kind == "input":
                    p.dims[tok[1]] = [int(v) for v in tok[2:]]
                    if not p.input_name:
                        p.input_name, p.input_dims = tok[1], p.dims[tok[1]]
                elif kind == "init":
                    name, fn = tok[1], tok[2]
                    d = [int(v) for v in tok[3:]]
                    p.dims[name] = d
                    fp = fn if fn.startswith("/") else os.path.join(pdir, fn)
                    n = int(np.prod(d)) if d else 1
                    p.inits[name] = np.fromfile(fp, dtype=np.uint16, count=n)
                elif kind == "tensor":
                    p.dims[tok[1]] = [int(v) for v in tok[2:]]
                elif kind == "node":
                    ins = [] if tok[2] == "-" else tok[2].split(",")
                    outs = tok[3].split(",")
                    attr = {}
                    for kv in tok[4:]:
                        if "=" in kv:
                            k, v = kv.split("=", 1)
                            attr[k] = v
                    p.nodes.append(Node(tok[1], ins, outs, attr))
                elif kind == "output":
                    if len(tok) > 1:
                        p.outputs.append(tok[1])
        if not p.input_name:
            raise RuntimeError("plan has no 'input' line")
        if not p.outputs:
            raise RuntimeError("plan has no 'output' line")
        return p

    def numel(self, name):
        d = self.dims[name]
        return int(np.prod(d)) if d else 1


def _chw(d):
    """(C, H, W) from the last three dims, as src/PlanModel.cpp:3561-3564 reads them."""
    base = len(d) - 3 if len(d) >= 3 else 0
    dd = list(d) + [1] * 3
    return dd[base], dd[base + 1], dd[base + 2]


def run_node(p: Plan, n: Node, T: dict, mode: int) -> None:
    """Executes one node for one image; T maps tensor name -> flat u16 array."""
    L = lib()
    g = lambda i: None if (i >= len(n.ins) or n.ins[i] == "-") else T[n.ins[i]]
    out = n.outs[0]
    nout = p.numel(out)
    op = n.op
    if op in ("reshape", "flatten"):
        T[out] = T[n.ins[0]]
        return
    if op == "conv3x3":
        x, w, b, r = g(0), g(1), g(2), g(3)
        Cin, H, W = _chw(p.dims[n.ins[0]])
        Cout = _chw(p.dims[out])[0]
        T[out] = conv2d(x, w, b, r, Cin, H, W, Cout, 3, n.i("stride", 1), n.i("pad", 1), 1,
                        n.i("Hout"), n.i("Wout"), n.i("act"), mode, 0)
        return
    if op == "conv1x1":
        w, x, b, r = g(0), g(1), g(2), g(3)
        wd = p.dims[n.ins[0]]
        Cout, Cin = wd[0], wd[1]
        N = p.numel(n.ins[1]) // Cin
        T[out] = conv2d(x, w, b, r, Cin, N, 1, Cout, 1, 1, 0, 1, N, 1, n.i("act"), mode,
                        1 if N == 1 else 0)
        return
    if op == "conv_general":
        x, w, b = g(0), g(1), g(2)
        Cin, H, W = _chw(p.dims[n.ins[0]])
        Cout = _chw(p.dims[out])[0]
        K, G = n.i("K", 3), n.i("G", 1)
        dw = (G == Cin and Cin == Cout and K in (3, 5))
        T[out] = conv2d(x, w, b, None, Cin, H, W, Cout, K, n.i("S", 1), n.i("P", 1), G,
                        n.i("Hout"), n.i("Wout"), n.i("act"), mode, 0 if dw else 2)
        return
    y = np.empty(nout, np.uint16)
    if op == "ew_binary":
        a, b = g(0), g(1)
        if "bdims" in n.attr and n.i("b_scalar") != 1:
            dims = np.array([int(v) for v in n.attr["bdims"].split(",")], np.int32)
            L.ivo_ew_binary_bcast(a, b, y, nout, n.i("op"), len(dims) // 3, dims)
        else:
            L.ivo_ew_binary(a, b, y, nout, n.i("op"), n.i("b_scalar"))
    elif op == "ew_unary":
        L.ivo_ew_unary(g(0), y, nout, n.i("op"))
    elif op == "bias_add":
        L.ivo_bias_add(g(0), g(1), y, nout, n.i("HW", 1))
    elif op == "copy_c":
        L.ivo_copy_c(g(0), y, n.i("HW", 1), n.i("c0"), n.i("cnt"), n.i("dst_off"))
    elif op == "slice_axis":
        L.ivo_slice_axis(g(0), y, n.i("outer", 1), n.i("axdim"), n.i("inner", 1),
                         n.i("start"), n.i("len"))
    elif op == "concat4":
        cs = [n.i("ca"), n.i("cb"), n.i("cc"), n.i("cd")]
        srcs = [g(i) if cs[i] else None for i in range(4)]
        L.ivo_concat4(_ptr(srcs[0]), cs[0], _ptr(srcs[1]), cs[1], _ptr(srcs[2]), cs[2],
                      _ptr(srcs[3]), cs[3], y, n.i("outer", 1), n.i("inner", 1))
    elif op == "maxpool":
        L.ivo_maxpool(g(0), y, n.i("C"), n.i("H"), n.i("W"), n.i("Hout"), n.i("Wout"),
                      n.i("K", 5), n.i("S", 1), n.i("P", 2))
    elif op == "resize_nn":
        L.ivo_resize_nn(g(0), y, n.i("C"), n.i("H"), n.i("W"), n.i("S", 2))
    elif op == "softmax_axis":
        L.ivo_softmax_axis(g(0), y, n.i("outer", 1), n.i("axdim"), n.i("inner", 1))
    elif op == "permute_0213":
        L.ivo_permute_0213(g(0), y, n.i("D1", 1), n.i("D2", 1), n.i("I", 1), n.i("mode"))
    elif op == "gap":
        L.ivo_gap(g(0), y, n.i("C"), n.i("HW", 1))
    elif op == "bmm":
        ad, bd = p.dims[n.ins[0]], p.dims[n.ins[1]]
        at = lambda d, i: d[i] if i < len(d) else 1
        B0, B1, M, K = at(ad, 0), at(ad, 1), at(ad, 2), ad[-1]
        N = bd[-1]
        L.ivo_bmm(g(0), g(1), y, B0 * B1, M, K, N)
    elif op == "gemm":
        # src/PlanModel.cpp:3935-3940: M = A.dims[0], K = A.dims[1], N = numel(B) / K (B of
        # any rank); the kernel is gemm_f16 (kernels/gemm.cl:183-669), i.e. a 1x1 conv
        # with W = A [M][K] and X = B [K][N] pixels, no bias, no activation (family 0).
        ad = p.dims[n.ins[0]]
        M, K = ad[0], ad[1]
        N = p.numel(n.ins[1]) // K
        a, b = g(0)[:M * K], g(1)[:K * N]
        y[:] = conv2d(b, a, None, None, K, N, 1, M, 1, 1, 0, 1, N, 1, 0, mode, 0)
    else:
        raise RuntimeError(f"unknown op: {op}")
    T[out] = y


def run_plan(p: Plan, x: np.ndarray, batch: int = 1, mode: int = F32, keep: bool = False):
    """Runs the plan on `batch` images (x: u16, batch*inputNumel elements).

    Returns a list (one per output) of u16 arrays of shape [batch, numel]; with
    keep=True also returns, per image, the dict of every tensor."""
    n_in = p.numel(p.input_name)
    x = np.ascontiguousarray(x, np.uint16).reshape(batch, n_in)
    outs = [np.empty((batch, p.numel(o)), np.uint16) for o in p.outputs]
    kept = []
    for b in range(batch):
        T = dict(p.inits)
        T[p.input_name] = x[b]
        for n in p.nodes:
            run_node(p, n, T, mode)
        for i, o in enumerate(p.outputs):
            outs[i][b] = T[o]
        if keep:
            kept.append(T)
    return (outs, kept) if keep else outs


# ------------------------------------------------------------------ metrics

def rel_errors(got: np.ndarray, ref: np.ndarray):
    """(mean_rel, max_rel, max_abs, scale_rel) as scripts/kernel_check.py:397-406 and
    scripts/model_check.py:196-201 define them: errors relative to max|ref|."""
    g = got.astype(np.float64).ravel()
    r = ref.astype(np.float64).ravel()
    d = np.abs(g - r)
    amax = float(np.max(np.abs(r))) if r.size else 0.0
    denom = amax if amax > 0 else 1.0
    mean_rel = float(np.mean(d) / (np.mean(np.abs(r)) if np.mean(np.abs(r)) > 0 else 1.0))
    max_rel = float(np.max(d) / denom) if d.size else 0.0
    return mean_rel, max_rel, float(np.max(d)) if d.size else 0.0, float(np.mean(d) / denom)
