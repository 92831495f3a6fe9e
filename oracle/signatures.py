"""Tuning signatures of a plan's nodes, as the reference computes them.

TEST INFRASTRUCTURE ONLY: used by tests/ to compare the plans this repository writes
(infvino_amd/planwriter.py) with the reference's own record of the nodes its lowered plans
contain: config/tuning.json holds one entry per node signature of the YOLOv8n-pose /
YOLO11n-pose / MobileNetV3-small plans that onnx2plan wrote from real ultralytics and
torchvision exports.  A plan whose every signature is one of those entries has the same
node types, shapes and attributes as the reference's plans.

Restated (no code of the reference is run or imported):
  * the default graph rewrites the reference applies after parsing, before its autotuner
    lists signatures (src/PlanModel.cpp:553-558): fuseConcatConv1x1 (575-664) and
    fuseResidualAdd (667-740); the opt-in SPPF and channel-scale fusions are off;
  * PlanModel::nodeSignature (src/PlanModel.cpp:4245-4308) and smallSig (2595-2679);
  * OpSignature::str (src/Tuning.cpp:85-115) and its factories (116-178);
  * tuningSignatures (src/PlanModel.cpp:4310-4327): conv_general nodes other than
    depthwise are not listed.
"""
from __future__ import annotations

import copy

import numpy as np


def _ai(n, key, default=0):
    v = n.attr.get(key)
    return default if v is None else int(v)


def _numel(p, name):
    d = p.dims[name]
    return int(np.prod(d)) if d else 1


def _chan(d):
    return int(d[len(d) - 3 if len(d) >= 3 else 0])


def fuse_default(p):
    """A copy of plan p's node list after fuseConcatConv1x1 and fuseResidualAdd."""
    nodes = [copy.deepcopy(n) for n in p.nodes]
    nodes = _fuse_concat_conv1x1(p, nodes)
    return _fuse_residual_add(p, nodes)


def _producers_uses(nodes):
    producer, uses = {}, {}
    for i, n in enumerate(nodes):
        for o in n.outs:
            if o != "-":
                producer[o] = i
    for n in nodes:
        for t in n.ins:
            if t != "-":
                uses[t] = uses.get(t, 0) + 1
    return producer, uses


def _fuse_concat_conv1x1(p, nodes):
    """src/PlanModel.cpp:575-664: concat4 (outer 1, single use) feeding a conv1x1's input
    becomes conv1x1_cat4; a concat source that is a single-use copy_c of the same count with
    dst_off 0 is read from its parent at the copy's offset and the copy is dropped."""
    producer, uses = _producers_uses(nodes)
    remove = set()
    for n in nodes:
        if n.op != "conv1x1" or len(n.ins) < 2 or n.ins[1] == "-":
            continue
        x = n.ins[1]
        pi = producer.get(x)
        if pi is None:
            continue
        cat = nodes[pi]
        if cat.op != "concat4" or uses.get(x, 0) != 1 or _ai(cat, "outer", 1) != 1:
            continue
        cnts = [_ai(cat, k, 0) for k in ("ca", "cb", "cc", "cd")]
        if cnts[0] <= 0:
            continue
        srcs = list(cat.ins[:4]) + ["-"] * (4 - len(cat.ins[:4]))
        offs = [0, 0, 0, 0]
        ok = True
        for j in range(4):
            if cnts[j] <= 0:
                continue
            s = srcs[j]
            if s == "-" or s not in p.dims:
                ok = False
                break
            ci = producer.get(s)
            if ci is not None:
                cp = nodes[ci]
                if (cp.op == "copy_c" and uses.get(s, 0) == 1 and _ai(cp, "cnt", 0) == cnts[j]
                        and _ai(cp, "dst_off", 0) == 0 and cp.ins[0] in p.dims):
                    offs[j] = _ai(cp, "c0", 0)
                    srcs[j] = cp.ins[0]
                    remove.add(ci)
        if not ok:
            continue
        for j in (1, 2, 3):
            if cnts[j] <= 0:
                srcs[j], offs[j] = srcs[0], 0
        for k, v in zip(("cat_ca", "cat_cb", "cat_cc", "cat_cd"), cnts):
            n.attr[k] = str(v)
        for k, v in zip(("cat_o0", "cat_o1", "cat_o2", "cat_o3"), offs):
            n.attr[k] = str(v)
        n.ins = [n.ins[0], srcs[0], srcs[1], srcs[2], srcs[3]] + list(n.ins[2:])
        n.op = "conv1x1_cat4"
        remove.add(pi)
    return [n for i, n in enumerate(nodes) if i not in remove]


def _fuse_residual_add(p, nodes):
    """src/PlanModel.cpp:667-740: ew_binary add without broadcasting whose operand is the
    single-use, non-output result of a conv1x1 / conv1x1_cat4 (no residual yet) produced after
    the other operand becomes that conv's residual."""
    producer, uses = _producers_uses(nodes)
    outputs = set(p.outputs)
    remove = set()
    for i, e in enumerate(nodes):
        if e.op != "ew_binary" or _ai(e, "op", 0) != 0:
            continue
        if "bdims" in e.attr and _ai(e, "b_scalar", 0) != 1:
            continue
        if len(e.ins) < 2:
            continue
        for k in (0, 1):
            pname, rname = e.ins[k], e.ins[1 - k]
            pi = producer.get(pname)
            if pi is None:
                continue
            c = nodes[pi]
            if c.op not in ("conv1x1", "conv1x1_cat4"):
                continue
            if uses.get(pname, 0) != 1 or pname in outputs:
                continue
            if len(c.outs) != 1 or c.outs[0] != pname:
                continue
            if rname == "-" or rname not in p.dims or pname not in p.dims:
                continue
            rs = 6 if c.op == "conv1x1_cat4" else 3
            if len(c.ins) > rs and c.ins[rs] != "-":
                continue
            ri = producer.get(rname)
            if ri is None or ri >= pi:
                continue
            if len(c.ins) <= rs:
                c.ins = list(c.ins) + ["-"] * (rs + 1 - len(c.ins))
            c.ins[rs] = rname
            c.outs = [e.outs[0]]
            remove.add(i)
            del producer[pname]
            producer[e.outs[0]] = pi
            break
    return [n for i, n in enumerate(nodes) if i not in remove]


def _str(op, act=0, **f):
    """OpSignature::str (src/Tuning.cpp:85-115), dtype f16, batch 1."""
    if op == "gemm":
        body = f"M{f['M']}N{f['N']}K{f['K']}"
    elif op == "conv3x3":
        body = f"W{f['W']}H{f['H']}s{f['s']}p{f['p']}_Cin{f['Cin']}_Cout{f['Cout']}"
    elif op in ("conv_general", "depthwise"):
        body = (f"W{f['W']}H{f['H']}s{f['s']}p{f['p']}_Cin{f['Cin']}_Cout{f['Cout']}"
                f"_K{f['K']}_G{f['G']}")
    elif op == "conv1x1":
        body = f"Cout{f['Cout']}_N{f['N']}_Cin{f['Cin']}"
    elif op == "conv1x1_cat4":
        body = f"Cout{f['Cout']}_N{f['N']}_Cin{f['Cin']}_cat" + ",".join(str(v) for v in f["params"])
    elif op == "gap":
        body = f"C{f['Cin']}_HW{f['N']}"
    else:
        params = f.get("params") or []
        body = ",".join(str(v) for v in params) if params else "0x0@0x0"
    return f"{op}|{body}_act{act}_f16"


def _small(p, n):
    """smallSig (src/PlanModel.cpp:2595-2679)."""
    nout = _numel(p, n.outs[0])
    if n.op == "ew_binary":
        op, bs = _ai(n, "op", 0), _ai(n, "b_scalar", 0)
        if "bdims" in n.attr and bs != 1:
            C = 0
            na, nb = _numel(p, n.ins[0]), _numel(p, n.ins[1])
            ts = n.ins[0] if (na != nout and nb == nout) else (n.ins[1] if (nb != nout and na == nout) else None)
            if ts is not None and _numel(p, ts) > 0:
                sd = p.dims[ts]
                nonunit = [i for i, d in enumerate(sd) if d != 1]
                tl = n.ins[1] if ts == n.ins[0] else n.ins[0]
                ld = p.dims[tl]
                chidx = len(ld) - 3 if len(ld) >= 3 else 0
                if len(nonunit) == 1 and nonunit[0] == chidx and ld[chidx] == _numel(p, ts):
                    C = _numel(p, ts)
            vals = [int(v) for v in n.attr["bdims"].split(",") if v != ""]
            rank = len(vals) // 3
            eff = sum(1 for r in range(rank) if vals[r] != 1)
            return _str("ew_binary_bcast", params=[nout, op, bs, C, eff])
        return _str("ew_binary", params=[nout, op, bs])
    if n.op == "ew_unary":
        return _str("ew_unary", params=[nout, _ai(n, "op", 0)])
    if n.op == "copy_c":
        return _str("copy_c", params=[_ai(n, "HW", 1), _ai(n, "cnt", 0)])
    if n.op == "slice_axis":
        return _str("slice_axis", params=[_ai(n, "outer", 1), _ai(n, "axdim", 0), _ai(n, "inner", 1),
                                          _ai(n, "start", 0), _ai(n, "len", 0)])
    if n.op == "concat4":
        return _str("concat4", params=[_ai(n, "outer", 1), _ai(n, "inner", 1), _ai(n, "ca", 0),
                                       _ai(n, "cb", 0), _ai(n, "cc", 0), _ai(n, "cd", 0)])
    if n.op == "maxpool":
        return _str("maxpool", params=[_ai(n, "C", 0), _ai(n, "H", 0), _ai(n, "W", 0), _ai(n, "Hout", 0),
                                       _ai(n, "Wout", 0), _ai(n, "K", 5), _ai(n, "S", 1), _ai(n, "P", 2)])
    if n.op == "resize_nn":
        return _str("resize_nn", params=[_ai(n, "C", 0), _ai(n, "H", 0), _ai(n, "W", 0), _ai(n, "S", 2)])
    if n.op == "permute_0213":
        return _str("permute_0213", params=[_ai(n, "D1", 1), _ai(n, "D2", 1), _ai(n, "I", 1), _ai(n, "mode", 0)])
    if n.op == "softmax_axis":
        return _str("softmax_axis", params=[_ai(n, "outer", 1), _ai(n, "axdim", 0), _ai(n, "inner", 1)])
    if n.op == "bmm":
        ad, bd = p.dims[n.ins[0]], p.dims[n.ins[1]]
        at = lambda d, i: int(d[i]) if i < len(d) else 1  # noqa: E731
        return _str("bmm", params=[at(ad, 0), at(ad, 1), at(ad, 2), at(ad, len(ad) - 1), at(bd, len(bd) - 1)])
    if n.op == "gap":
        return _str("gap", Cin=_ai(n, "C", 0), N=_ai(n, "HW", 1))
    return _str(n.op)


_SMALL = {"ew_binary", "ew_unary", "copy_c", "slice_axis", "concat4", "maxpool", "resize_nn",
          "permute_0213", "bmm", "softmax_axis", "gap"}


def node_signature(p, n):
    """(signature, listed) for one node: PlanModel::nodeSignature; `listed` is False where
    tuningSignatures would skip the node (non-depthwise conv_general, unknown ops)."""
    if n.op == "conv3x3":
        Cin, Cout = _chan(p.dims[n.ins[0]]), _chan(p.dims[n.outs[0]])
        return _str("conv3x3", _ai(n, "act", 0), W=_ai(n, "Wout", 0), H=_ai(n, "Hout", 0),
                    s=_ai(n, "stride", 1), p=_ai(n, "pad", 1), Cin=Cin, Cout=Cout), True
    if n.op == "gemm":
        ad = p.dims[n.ins[0]]
        M, K = int(ad[0]), int(ad[1])
        return _str("gemm", M=M, N=_numel(p, n.ins[1]) // K, K=K), True
    if n.op == "conv1x1_cat4":
        wd = p.dims[n.ins[0]]
        Cout, Cin = int(wd[0]), int(wd[1])
        HW = _numel(p, n.outs[0]) // Cout if Cout > 0 else 0
        params = [_ai(n, k, 0) for k in ("cat_ca", "cat_cb", "cat_cc", "cat_cd")]
        return _str("conv1x1_cat4", _ai(n, "act", 0), Cout=Cout, N=HW, Cin=Cin, params=params), True
    if n.op == "conv1x1":
        wd = p.dims[n.ins[0]]
        Cout, Cin = int(wd[0]), int(wd[1])
        N = _numel(p, n.ins[1]) // Cin if Cin > 0 else 0
        return _str("conv1x1", _ai(n, "act", 0), Cout=Cout, N=N, Cin=Cin), True
    if n.op == "conv_general":
        K, S, P, G = _ai(n, "K", 3), _ai(n, "S", 1), _ai(n, "P", 1), _ai(n, "G", 1)
        Cin, Cout = _chan(p.dims[n.ins[0]]), _chan(p.dims[n.outs[0]])
        f = dict(W=_ai(n, "Wout", 0), H=_ai(n, "Hout", 0), s=S, p=P, Cin=Cin, Cout=Cout, K=K, G=G)
        if G == Cin and K in (3, 5) and Cin == Cout:
            return _str("depthwise", _ai(n, "act", 0), **f), True
        return _str("conv_general", _ai(n, "act", 0), **f), False
    if n.op in _SMALL:
        return _small(p, n), True
    return _str(n.op), False


def plan_signatures(p):
    """[(node index in the fused list, op, signature)] for every node tuningSignatures lists."""
    out = []
    for i, n in enumerate(fuse_default(p)):
        if n.op in ("reshape", "flatten"):
            continue
        sig, listed = node_signature(p, n)
        if listed:
            out.append((i, n.op, sig))
    return out
