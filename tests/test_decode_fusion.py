"""Fused Detect / Pose decode tail (the executor's fuseDecode pass and its kernel).

CPU: the pass matches the YOLO pose plans and nothing else (dry runs), rejects a tail that
differs in one operand order or one unary op, and the fused formula -- restated here in
numpy with the fp16 rounding of every node the chain stores -- reproduces the oracle's
node-by-node chain on real head tensors.  GPU: the fused kernel against the same plan run
node by node (IVH_FLAG_NO_FUSE_DECODE), on both of its code paths."""
import os
import shutil

import numpy as np
import pytest

import infvino_amd as ia
from infvino_amd import planwriter as pw
from oracle import oracle as O

DRY = ia.IVH_FLAG_DRY_RUN


def _kernels(path, flags=0, batch=2):
    m = ia.PlanModel(path, 0, batch, DRY | flags)
    m.run(batch)
    ks = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    m.close()
    return ks


@pytest.mark.parametrize("name,legacy", [("yolov8n-pose", False), ("yolo11n-pose", False),
                                         ("yolov8n-pose", True), ("yolo11n-pose", True)])
def test_decode_tail_fused(plans, name, legacy):
    """Both export forms of the head: ultralytics 8.4's (separate box / score concats, lt / rb
    by slice_axis, one three-way output concat) and the older one (one box + class concat
    split by copy_c, nested output concats)."""
    path = plans(name, legacy=True)[0] if legacy else plans(name)[0]
    fused = _kernels(path)
    chain = _kernels(path, ia.IVH_FLAG_NO_FUSE_DECODE)
    assert fused.count("pose_decode") == 1 and "pose_decode" not in chain
    assert "pose_decode" not in _kernels(path, ia.IVH_FLAG_NO_FUSE)
    # the tail's softmax, permute and slices are gone (YOLO11's attention keeps its own)
    for k, n in (("softmax_axis", 1), ("permute_0213", 1), ("slice_axis", 2 if legacy else 4)):
        assert chain.count(k) - fused.count(k) == n, k
    launches = lambda ks: sum(k != "(view)" for k in ks)
    assert launches(chain) - launches(fused) >= 15


def test_decode_tail_absent_elsewhere(plans):
    assert "pose_decode" not in _kernels(plans("mobilenetv3-small")[0])


def _variant(path, tmp_path, old, new, name):
    """Copy of a plan (its init files alongside) with one line edited."""
    d = tmp_path / name
    shutil.copytree(os.path.dirname(path), d)
    text = open(path).read()
    assert text.count(old) == 1, old
    p = d / os.path.basename(path)
    p.write_text(text.replace(old, new))
    return str(p)


def test_decode_tail_mismatch_not_fused(plans, tmp_path):
    path = plans("yolov8n-pose", imgsz=320)[0]
    text = open(path).read()
    # x1y1 = anchors - lt  ->  lt - anchors: a different function, left node by node
    line = next(l for l in text.splitlines() if l.startswith("node ew_binary anchors") and " op=1 " in l)
    ins = line.split()[2].split(",")
    swapped = line.replace(",".join(ins), ",".join(ins[::-1]), 1)
    p1 = _variant(path, tmp_path, line, swapped, "swap")
    assert "pose_decode" not in _kernels(p1)
    # keypoint visibility sigmoid -> ReLU
    vis = [l for l in text.splitlines() if l.startswith("node ew_unary") and " op=0 " in l][-1]
    p2 = _variant(path, tmp_path, vis, vis.replace(" op=0 ", f" op={pw.UN_RELU} "), "relu")
    assert "pose_decode" not in _kernels(p2)
    # centre as sum * c instead of sum / c is the same shape (box_div = 0): fused
    div = next(l for l in text.splitlines() if l.startswith("node ew_binary") and " op=3 " in l)
    p3 = _variant(path, tmp_path, div, div.replace(" op=3 ", " op=2 "), "mul")
    assert _kernels(p3).count("pose_decode") == 1


# ------------------------------------------------------------- the fused formula on CPU

def _heads(p):
    """Per-scale head tensors feeding the anchor concats: (box list, class list, keypoint
    list); in the older export form the box list holds box + class channels and the class
    list is empty."""
    src = {n.outs[0]: n.ins[0] for n in p.nodes if n.op == "reshape"}
    cats = [n for n in p.nodes if n.op == "concat4" and n.i("inner", 1) == 1 and n.i("ca") > 1]
    by_outer = {n.i("outer"): [src[t] for t in n.ins if t != "-"] for n in cats}
    if 65 in by_outer:
        return by_outer[65], [], by_outer[51]
    return by_outer[64], by_outer[1], by_outer[51]


def _rh(v):
    return np.asarray(v, np.float32).astype(np.float16).astype(np.float32)


def _decode_restated(p, T):
    """Pose decode of one image from its head tensors, each node's fp16 rounding kept (the
    fused kernel's formula, with the oracle's softmax division)."""
    xs, cs, ks = _heads(p)
    f = lambda t: O.h2f(T[t]).reshape(p.dims[t][1], -1)
    X = np.concatenate([f(t) for t in xs], 1)
    if cs:
        X = np.concatenate([X, np.concatenate([f(t) for t in cs], 1)], 0)
    K = np.concatenate([f(t) for t in ks], 1)
    A = X.shape[1]
    init = lambda stem: O.h2f(next(v for k, v in p.inits.items() if k.startswith(stem)))
    anc, st, ancm = init("anchors").reshape(2, A), init("strides"), init("anc_m").reshape(2, A)
    # the DFL projection's weights: the one bias-free conv1x1 with one output channel
    n = next(n for n in p.nodes if n.op == "conv1x1" and p.dims[n.ins[0]][0] == 1 and len(n.ins) > 2 and n.ins[2] == "-")
    w = O.h2f(p.inits[n.ins[0]]).ravel()
    two = [O.h2f(v)[0] for k, v in sorted(p.inits.items()) if k.startswith("two")]
    box = X[:64].reshape(4, 16, A)
    e = np.exp(box - box.max(1, keepdims=True))
    sm = _rh(e / e.sum(1, keepdims=True))
    d = _rh(np.einsum("k,jka->ja", w, sm))
    x1, y1, x2, y2 = _rh(anc[0] - d[0]), _rh(anc[1] - d[1]), _rh(anc[0] + d[2]), _rh(anc[1] + d[3])
    cx, cy = _rh(_rh(x1 + x2) / two[0]), _rh(_rh(y1 + y2) / two[0])
    out = [_rh(cx * st), _rh(cy * st), _rh(_rh(x2 - x1) * st), _rh(_rh(y2 - y1) * st),
           _rh(1.0 / (1.0 + np.exp(-X[64])))]
    for k in range(17):
        out.append(_rh(_rh(_rh(K[3 * k] * two[1]) + ancm[0]) * st))
        out.append(_rh(_rh(_rh(K[3 * k + 1] * two[1]) + ancm[1]) * st))
        out.append(_rh(1.0 / (1.0 + np.exp(-K[3 * k + 2]))))
    return np.stack(out)


def _ulps(a, b):
    """fp16 ulp distance of two arrays of fp16 values (given as float32)."""
    def key(v):
        u = v.astype(np.float16).view(np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7fff), u)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("legacy", [False, True])
def test_decode_formula_matches_chain(plans, legacy):
    path = plans("yolov8n-pose", imgsz=128, legacy=legacy)[0]
    p = O.Plan.load(path)
    x = O.f2h(np.random.default_rng(4).random(p.numel(p.input_name)).astype(np.float32))
    outs, kept = O.run_plan(p, x, 1, keep=True)
    ref = O.h2f(outs[0][0]).reshape(56, -1)
    got = _decode_restated(p, kept[0])
    u = _ulps(got, ref)
    assert u.max() <= 2 and (u == 0).mean() > 0.98, (u.max(), (u == 0).mean())
    # a dropped term is not within tolerance: e.g. the strides factor on the keypoints
    bad = got.copy()
    bad[5] = _rh(bad[5] / O.h2f(p.inits[next(k for k in p.inits if k.startswith("strides"))]))
    assert _ulps(bad, ref).max() > 2


# ------------------------------------------------------------------ GPU: fused vs chain

def _small_pose(out_dir, nc, nk, legacy=False):
    """A 128x128 toy backbone (strides 8 / 16 / 32) under a pose head with nc classes and
    nk keypoints: counts the decode kernel has no compile-time instance for."""
    pb = pw.PlanBuilder(out_dir, seed=3)
    x = pb.input("images", [1, 3, 128, 128])
    x = pb.conv(pb.conv(x, 16, 3, 2), 32, 3, 2)
    f3 = pb.conv(x, 32, 3, 2)
    f4 = pb.conv(f3, 64, 3, 2)
    f5 = pb.conv(f4, 64, 3, 2)
    pb.output(pw._pose_head(pb, [f3, f4, f5], nc=nc, nk=(nk, 3), legacy=legacy))
    return pb.write()


@pytest.mark.parametrize("legacy", [False, True])
def test_decode_tail_fused_other_counts(tmp_path, legacy):
    assert _kernels(_small_pose(str(tmp_path), 2, 5, legacy)).count("pose_decode") == 1


def test_detect_head_fused(tmp_path):
    """A Detect head (80 classes, no keypoints; ultralytics 8.4 form) takes the decode too."""
    pb = pw.PlanBuilder(str(tmp_path), seed=3)
    x = pb.input("images", [1, 3, 128, 128])
    x = pb.conv(pb.conv(x, 16, 3, 2), 32, 3, 2)
    f3 = pb.conv(x, 32, 3, 2)
    f4 = pb.conv(f3, 64, 3, 2)
    f5 = pb.conv(f4, 64, 3, 2)
    pb.output(pw._pose_head(pb, [f3, f4, f5], nc=80, nk=None))
    assert _kernels(pb.write()).count("pose_decode") == 1


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch,flags", [("yolov8n-pose", 3, 0), ("yolo11n-pose", 2, 0),
                                               ("yolov8n-pose", 2, ia.IVH_FLAG_NCHW_ONLY),
                                               ("small-nc2-nk5", 3, 0), ("legacy-yolov8n-pose", 2, 0),
                                               ("legacy-small-nc2-nk5", 3, 0)])
def test_decode_fused_vs_chain_gpu(plans, tmp_path, name, batch, flags):
    """The YOLO heads take the compile-time-count kernel, the toy head (2 classes, 5
    keypoints) the run-time-count one; both export forms of the head."""
    legacy = name.startswith("legacy-")
    base = name[len("legacy-"):] if legacy else name
    print(f"decode {name} batch {batch} flags {flags:#x}", flush=True)
    if base.startswith("small"):
        path = _small_pose(str(tmp_path), 2, 5, legacy)
    else:
        path = plans(base, legacy=True)[0] if legacy else plans(base)[0]
    p = O.Plan.load(path)
    x = O.f2h(np.random.default_rng(7).random(p.numel(p.input_name) * batch).astype(np.float32))
    res = {}
    for extra in (0, ia.IVH_FLAG_NO_FUSE_DECODE):
        m = ia.PlanModel(path, 0, batch, flags | extra)
        m.setInput(x, batch)
        m.run(batch)
        res[extra] = O.h2f(m.readOutput(0, batch))
        if extra == 0:
            assert [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())].count("pose_decode") == 1
        m.close()
    a, b = res[0], res[ia.IVH_FLAG_NO_FUSE_DECODE]
    u = _ulps(a, b)
    print(f"{name} b{batch} flags {flags:#x}: max {u.max()} ulp, exact {(u == 0).mean():.6f}")
    ny, A = p.dims[p.outputs[0]][1:]
    for i in np.argsort(-u)[:8]:
        if u[i]:
            print(f"  row {(i // A) % ny} anchor {i % A} image {i // (ny * A)}: fused {a[i]!r} chain {b[i]!r} ({u[i]} ulp)")
    # A rare 1-ulp flip of a DFL distance (fp32 summation order) moves a box edge by one
    # distance ulp times the stride; where anchor - distance cancels that is many ulps of a
    # small output, so box rows are bounded in pixels (half a pixel), the rest in ulps.
    boxr = (np.arange(a.size) // A) % ny < 4
    assert (u == 0).mean() > 0.9999
    assert np.abs(a - b)[boxr].max() <= 0.5 and u[~boxr].max() <= 2
