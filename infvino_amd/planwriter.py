"""Random-init plan writer: emits model.plan + fp16 init .bin files in the reference's
plan format, for the models and op sweeps the hot path is measured on.

The reference lowers ONNX exports with scripts/onnx2plan.py (needs `onnx` and
downloaded weights, neither available offline).  This module builds the same
graphs directly and lowers them with the same rules:
  * plan grammar            include/infvino/PlanModel.hpp:5-12
  * conv routing            scripts/onnx2plan.py:169-226  (3x3 g=1 s1/s2 -> conv3x3,
                            1x1 g=1 -> conv1x1 [w,x,b,res], else conv_general)
  * activation folding      scripts/onnx2plan.py:101-147  (SiLU -> act=1 everywhere;
                            conv3x3 folds only HardSwish; conv1x1/Gemm fold
                            Sigmoid5/ReLU2/HS3/HSig4; conv_general folds HS3/ReLU2/HSig4)
  * ew_binary broadcasting  scripts/onnx2plan.py:244-277  (bdims = out,a_strides,b_strides)
  * concat / split / slice  scripts/onnx2plan.py:278-345
  * weights                 astype(float16) (RNE), raw little-endian (:61-71)
Weights are random (He-normal convs, N(0, 0.01) bias: BN folded into conv+bias).
Topologies: YOLOv8n-pose (ultralytics yolov8-pose.yaml, scale n), MobileNetV3-small
(torchvision), YOLO11n-pose (ultralytics yolo11-pose.yaml, scale n).
"""
from __future__ import annotations

import os

import numpy as np

ACT_NONE, ACT_SILU, ACT_RELU, ACT_HSWISH, ACT_HSIGMOID, ACT_SIGMOID = 0, 1, 2, 3, 4, 5
# ew_unary codes (kernels/ops.cl:50-63 / onnx2plan.py:239-243)
UN_SIGMOID, UN_SILU, UN_RELU, UN_HSWISH, UN_HSIGMOID = 0, 1, 2, 3, 4
_ACT_TO_UNARY = {ACT_SILU: UN_SILU, ACT_RELU: UN_RELU, ACT_HSWISH: UN_HSWISH,
                 ACT_HSIGMOID: UN_HSIGMOID, ACT_SIGMOID: UN_SIGMOID}
# which activations each conv route folds (onnx2plan.py:135-147); SiLU always folds
_FOLD_CONV3 = {ACT_SILU, ACT_HSWISH}
_FOLD_1X1 = {ACT_SILU, ACT_SIGMOID, ACT_RELU, ACT_HSWISH, ACT_HSIGMOID}
_FOLD_GENERAL = {ACT_SILU, ACT_HSWISH, ACT_RELU, ACT_HSIGMOID}


def _bdims(oshape, ashape, bshape):
    """Broadcast spec exactly as scripts/onnx2plan.py:249-266 computes it."""
    rank = len(oshape)

    def align(s):
        return [1] * (rank - len(s)) + list(s)

    def strides(aligned):
        st = [0] * rank
        acc = 1
        for i in range(rank - 1, -1, -1):
            st[i] = 0 if (aligned[i] == 1 and oshape[i] != 1) else acc
            acc *= aligned[i]
        return st

    a_st, b_st = strides(align(ashape)), strides(align(bshape))
    return ",".join(str(v) for v in list(oshape) + a_st + b_st)


class PlanBuilder:
    """Collects plan lines and writes init .bin files into out_dir."""

    def __init__(self, out_dir: str, seed: int = 0):
        self.dir = out_dir
        os.makedirs(out_dir, exist_ok=True)
        self.rng = np.random.default_rng(seed)
        self.lines: list[str] = []
        self.shapes: dict[str, list[int]] = {}
        self.inits: set[str] = set()
        self._n = 0
        self.flops = 0  # conv/gemm FLOPs per image (2*MAC)

    # -- primitives ---------------------------------------------------------
    def name(self, stem="t"):
        self._n += 1
        return f"{stem}{self._n}"

    def input(self, name, dims):
        self.shapes[name] = list(dims)
        self.lines.append("input {} {}".format(name, " ".join(str(d) for d in dims)))
        return name

    def init(self, arr, stem="w", name=None):
        name = name or self.name(stem)
        a = np.asarray(arr, dtype=np.float32).astype(np.float16)
        fn = f"init_{name}.bin"
        a.tofile(os.path.join(self.dir, fn))
        self.shapes[name] = list(a.shape)
        self.inits.add(name)
        self.lines.append("init {} {} {}".format(name, fn, " ".join(str(d) for d in a.shape)))
        return name

    def tensor(self, dims, name=None):
        name = name or self.name()
        self.shapes[name] = list(dims)
        self.lines.append("tensor {} {}".format(name, " ".join(str(d) for d in dims)))
        return name

    def node(self, kind, ins, outs, **attrs):
        a = " ".join(f"{k}={v}" for k, v in attrs.items() if v is not None)
        self.lines.append("node {} {} {} {}".format(kind, ",".join(ins) or "-", ",".join(outs), a).rstrip())

    def output(self, name):
        self.lines.append(f"output {name}")

    def write(self, plan_name="model.plan"):
        path = os.path.join(self.dir, plan_name)
        with open(path, "w") as f:
            f.write("\n".join(self.lines) + "\n")
        return path

    # -- lowered ops ----------------------------------------------------------
    def conv(self, x, cout, k=1, s=1, groups=1, act=ACT_SILU, bias=True, pad=None,
             weight=None, bias_val=None, res=None):
        """Conv(+BN folded)+activation, routed and folded as onnx2plan.emit_conv."""
        _, cin, H, W = self.shapes[x]
        p = k // 2 if pad is None else pad
        Ho = (H + 2 * p - k) // s + 1
        Wo = (W + 2 * p - k) // s + 1
        fan_in = cin // groups * k * k
        if weight is None:
            weight = self.rng.normal(0.0, np.sqrt(2.0 / fan_in), (cout, cin // groups, k, k))
        w = self.init(weight, "w")
        b = None
        if bias:
            if bias_val is None:
                bias_val = self.rng.normal(0.0, 0.01, cout)
            b = self.init(bias_val, "b")
        self.flops += 2 * cout * fan_in * Ho * Wo
        y = self.tensor([1, cout, Ho, Wo])
        if k == 3 and groups == 1 and s in (1, 2):
            fold = act in _FOLD_CONV3
            self.node("conv3x3", [x, w, b or "-", res or "-"], [y], stride=s, pad=p, Hout=Ho,
                      Wout=Wo, act=(act if fold and act else None),
                      cfg=(None if s == 1 else "64,8,1,32,8,2"))
        elif k == 1 and groups == 1:
            fold = act in _FOLD_1X1
            wn = w
            self.node("conv1x1", [wn, x, b or "-", res or "-"], [y], act=(act if fold and act else None))
        else:
            fold = act in _FOLD_GENERAL
            self.node("conv_general", [x, w, b or "-"], [y], K=k, S=s, P=p, G=groups, Hout=Ho,
                      Wout=Wo, act=(act if fold and act else None))
        if act and not fold:
            y = self.unary(y, _ACT_TO_UNARY[act])
        return y

    def gemm(self, x, nout, act=ACT_NONE):
        """Gemm(transB=1) lowered to conv1x1 [w, x, b] (onnx2plan.py:406-422)."""
        _, k = self.shapes[x]
        w = self.init(self.rng.normal(0.0, np.sqrt(2.0 / k), (nout, k)), "w")
        b = self.init(self.rng.normal(0.0, 0.01, nout), "b")
        self.flops += 2 * nout * k
        y = self.tensor([1, nout])
        fold = act in _FOLD_1X1
        self.node("conv1x1", [w, x, b, "-"], [y], act=(act if fold and act else None))
        if act and not fold:
            y = self.unary(y, _ACT_TO_UNARY[act])
        return y

    def unary(self, x, op):
        y = self.tensor(self.shapes[x])
        self.node("ew_unary", [x], [y], op=op, n=int(np.prod(self.shapes[x])))
        return y

    def binary(self, a, b, op, out_shape=None):
        """Add/Sub/Mul/Div with ONNX broadcasting, lowered as onnx2plan.py:244-277."""
        asha, bsha = self.shapes[a], self.shapes[b]
        if out_shape is None:
            r = max(len(asha), len(bsha))
            aa = [1] * (r - len(asha)) + asha
            bb = [1] * (r - len(bsha)) + bsha
            out_shape = [max(p, q) for p, q in zip(aa, bb)]
        y = self.tensor(out_shape)
        b_scalar = 0
        bd = None
        if list(asha) != list(out_shape) or (b in self.inits and list(bsha) != list(out_shape)):
            bd = _bdims(out_shape, asha, bsha)
        if b in self.inits and int(np.prod(bsha)) == 1 and list(asha) == list(out_shape):
            b_scalar = 1
        self.node("ew_binary", [a, b], [y], op=op, n=int(np.prod(out_shape)), b_scalar=b_scalar,
                  bdims=bd)
        return y

    def concat(self, xs, axis=1):
        shp = [list(self.shapes[x]) for x in xs]
        out = list(shp[0])
        out[axis] = sum(s[axis] for s in shp)
        outer = int(np.prod(out[:axis]))
        inner = int(np.prod(out[axis + 1:]))
        dims = [s[axis] for s in shp]
        ins = list(xs)
        assert len(ins) <= 4
        while len(ins) < 4:
            ins.append("-")
            dims.append(0)
        y = self.tensor(out)
        self.node("concat4", ins, [y], ca=dims[0], cb=dims[1], cc=dims[2], cd=dims[3],
                  outer=outer, inner=inner)
        return y

    def split(self, x, sizes, axis=1):
        xs = self.shapes[x]
        outs = []
        if axis == 1:
            c0 = 0
            for cnt in sizes:
                o = list(xs)
                o[1] = cnt
                y = self.tensor(o)
                self.node("copy_c", [x], [y], HW=int(np.prod(o[2:])), c0=c0, cnt=cnt, dst_off=0)
                c0 += cnt
                outs.append(y)
        else:
            outer = int(np.prod(xs[:axis]))
            inner = int(np.prod(xs[axis + 1:]))
            start = 0
            for ln in sizes:
                outs.append(self.slice(x, axis, start, ln))
                start += ln
        return outs

    def slice(self, x, axis, start, length):
        xs = self.shapes[x]
        o = list(xs)
        o[axis] = length
        y = self.tensor(o)
        self.node("slice_axis", [x], [y], outer=int(np.prod(xs[:axis])), axdim=xs[axis],
                  inner=int(np.prod(xs[axis + 1:])), start=start, len=length)
        return y

    def reshape(self, x, dims):
        assert int(np.prod(dims)) == int(np.prod(self.shapes[x]))
        y = self.tensor(dims)
        self.node("reshape", [x], [y])
        return y

    def maxpool(self, x, k, s, p):
        _, C, H, W = self.shapes[x]
        Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
        y = self.tensor([1, C, Ho, Wo])
        self.node("maxpool", [x], [y], C=C, H=H, W=W, Hout=Ho, Wout=Wo, K=k, S=s, P=p)
        return y

    def upsample(self, x, s=2):
        _, C, H, W = self.shapes[x]
        y = self.tensor([1, C, H * s, W * s])
        self.node("resize_nn", [x], [y], C=C, H=H, W=W, S=s)
        return y

    def permute(self, x, perm):
        xs = self.shapes[x]
        assert perm in ([0, 2, 1, 3], [0, 1, 3, 2])
        mode = 0 if perm == [0, 2, 1, 3] else 1
        y = self.tensor([xs[p] for p in perm])
        self.node("permute_0213", [x], [y], D1=xs[1], D2=xs[2], I=int(np.prod(xs[3:])), mode=mode)
        return y

    def softmax(self, x, axis):
        xs = self.shapes[x]
        y = self.tensor(xs)
        self.node("softmax_axis", [x], [y], outer=int(np.prod(xs[:axis])), axdim=xs[axis],
                  inner=int(np.prod(xs[axis + 1:])))
        return y

    def matmul(self, a, b):
        asha, bsha = self.shapes[a], self.shapes[b]
        out = list(asha[:-1]) + [bsha[-1]]
        y = self.tensor(out)
        self.flops += 2 * int(np.prod(asha)) * bsha[-1]
        self.node("bmm", [a, b], [y], B0=asha[0], B1=asha[1], M=asha[2], K=asha[3], N=bsha[3])
        return y

    def gap(self, x):
        _, C, H, W = self.shapes[x]
        y = self.tensor([1, C, 1, 1])
        self.node("gap", [x], [y], C=C, HW=H * W)
        return y

    def const(self, arr, stem="c"):
        return self.init(arr, stem)


# ---------------------------------------------------------------------- YOLOv8

def _c2f(pb, x, c2, n, shortcut):
    """ultralytics C2f: cv1 1x1 -> split(2) -> n Bottlenecks (3x3,3x3[,+]) -> concat -> cv2."""
    c = c2 // 2
    y = pb.conv(x, 2 * c, 1)
    ys = pb.split(y, [c, c])
    for _ in range(n):
        t = pb.conv(ys[-1], c, 3)
        t = pb.conv(t, c, 3)
        if shortcut:
            t = pb.binary(ys[-1], t, 0)
        ys.append(t)
    return pb.conv(pb.concat(ys), c2, 1)


def _sppf(pb, x, c2, k=5):
    c1 = pb.shapes[x][1]
    y = [pb.conv(x, c1 // 2, 1)]
    for _ in range(3):
        y.append(pb.maxpool(y[-1], k, 1, k // 2))
    return pb.conv(pb.concat(y), c2, 1)


def _anchors(sizes, strides):
    """make_anchors(grid_cell_offset=0.5): anchor points [2, A] and strides [1, A]."""
    pts, st = [], []
    for (h, w), s in zip(sizes, strides):
        sy, sx = np.meshgrid(np.arange(h) + 0.5, np.arange(w) + 0.5, indexing="ij")
        pts.append(np.stack([sx.ravel(), sy.ravel()], 0))
        st.append(np.full((1, h * w), s, np.float32))
    return np.concatenate(pts, 1).astype(np.float32), np.concatenate(st, 1)


def _pose_head(pb, feats, nc=1, nk=(17, 3), reg_max=16, dw_cls=False, legacy=False):
    """ultralytics Pose head in export form (Detect decode + Pose.kpts_decode).

    Default: the form of ultralytics 8.4 exports (requirements-export.txt pins 8.4.166), which
    is what the reference's own lowered plans hold (config/tuning.json's signatures): the box
    distributions, class scores and keypoints of the three scales are concatenated over the
    anchors separately ([4R, A], [nc, A], [3 nk, A]); the DFL distances are split into lt / rb
    by two Slice nodes (slice_axis); the output is one concat of the decoded boxes, the
    sigmoid scores and the decoded keypoints.
    legacy=True: the older export form, per scale box and class channels concatenated first,
    one [4R + nc, A] concat over the anchors split by channel copies (copy_c), the output
    built by two nested concats."""
    ch0 = pb.shapes[feats[0]][1]
    c2 = max(16, ch0 // 4, reg_max * 4)
    c3 = max(ch0, min(nc, 100))
    nkk = nk[0] * nk[1] if nk else 0
    c4 = max(ch0 // 4, nkk)
    strides = [8, 16, 32]
    sizes = [tuple(pb.shapes[f][2:]) for f in feats]
    A = sum(h * w for h, w in sizes)
    # keypoint branch: cv4[i] -> view(bs, nk, -1) -> cat(-1)
    kp = []
    for f in feats if nkk else []:
        t = pb.conv(f, c4, 3)
        t = pb.conv(t, c4, 3)
        t = pb.conv(t, nkk, 1, act=ACT_NONE)
        _, _, h, w = pb.shapes[t]
        kp.append(pb.reshape(t, [1, nkk, h * w]))
    kpt = _concat_many(pb, kp, axis=2) if kp else None
    # box / class branches
    bs, cs = [], []
    for f in feats:
        b = pb.conv(f, c2, 3)
        b = pb.conv(b, c2, 3)
        b = pb.conv(b, 4 * reg_max, 1, act=ACT_NONE)
        if dw_cls:  # YOLO11 cls branch: DWConv 3x3 + Conv 1x1, twice
            ci = pb.shapes[f][1]
            c = pb.conv(f, ci, 3, groups=ci)
            c = pb.conv(c, c3, 1)
            c = pb.conv(c, c3, 3, groups=c3)
            c = pb.conv(c, c3, 1)
        else:
            c = pb.conv(f, c3, 3)
            c = pb.conv(c, c3, 3)
        c = pb.conv(c, nc, 1, act=ACT_NONE)
        bs.append(b)
        cs.append(c)
    flat = lambda x: pb.reshape(x, [1, pb.shapes[x][1], pb.shapes[x][2] * pb.shapes[x][3]])  # noqa: E731
    if legacy:
        no = 4 * reg_max + nc
        xs = [pb.concat([b, c]) for b, c in zip(bs, cs)]
        xcat = _concat_many(pb, [pb.reshape(x, [1, no, pb.shapes[x][2] * pb.shapes[x][3]]) for x in xs], axis=2)
        box, cls = pb.split(xcat, [4 * reg_max, nc])
    else:
        box = _concat_many(pb, [flat(b) for b in bs], axis=2)   # [1, 4R, A]
        cls = _concat_many(pb, [flat(c) for c in cs], axis=2)   # [1, nc, A]
    # DFL: view(b,4,16,a).transpose(2,1).softmax(1) -> conv 16->1 (arange weights)
    d = pb.reshape(box, [1, 4, reg_max, A])
    d = pb.permute(d, [0, 2, 1, 3])
    d = pb.softmax(d, 1)
    d = pb.conv(d, 1, 1, act=ACT_NONE, bias=False,
                weight=np.arange(reg_max, dtype=np.float32).reshape(1, reg_max, 1, 1))
    d = pb.reshape(d, [1, 4, A])
    anc, strd = _anchors(sizes, strides)
    anc_c = pb.const(anc[None], "anchors")            # [1, 2, A]
    if legacy:
        lt, rb = pb.split(d, [2, 2])
    else:
        lt, rb = pb.slice(d, 1, 0, 2), pb.slice(d, 1, 2, 2)
    x1y1 = pb.binary(anc_c, lt, 1)
    x2y2 = pb.binary(anc_c, rb, 0)
    two = pb.const(np.array([2.0], np.float32), "two")
    cxy = pb.binary(pb.binary(x1y1, x2y2, 0), two, 3)
    wh = pb.binary(x2y2, x1y1, 1)
    dbox = pb.concat([cxy, wh])
    st_c = pb.const(strd, "strides")                  # [1, A]
    dbox = pb.binary(dbox, st_c, 2)
    scores = pb.unary(cls, UN_SIGMOID)
    if not nkk:
        return pb.concat([dbox, scores])
    # kpts_decode (export): view(bs,17,3,-1); (y[:,:,:2]*2 + (anchors-0.5))*strides; sigmoid vis
    y = pb.reshape(kpt, [1, nk[0], nk[1], A])
    xy = pb.slice(y, 2, 0, 2)
    xy = pb.binary(xy, pb.const(np.array([2.0], np.float32), "two"), 2)
    xy = pb.binary(xy, pb.const(anc - 0.5, "anc_m"), 0)
    xy = pb.binary(xy, st_c, 2)
    vis = pb.unary(pb.slice(y, 2, 2, 1), UN_SIGMOID)
    a = pb.concat([xy, vis], axis=2)
    a = pb.reshape(a, [1, nkk, A])
    if legacy:
        return pb.concat([pb.concat([dbox, scores]), a])
    return pb.concat([dbox, scores, a])


def _concat_many(pb, xs, axis):
    while len(xs) > 4:
        xs = [pb.concat(xs[:4], axis)] + xs[4:]
    return pb.concat(xs, axis) if len(xs) > 1 else xs[0]


def yolov8n_pose(out_dir, seed=0, imgsz=640, legacy=False):
    """YOLOv8n-pose (ultralytics yolov8-pose.yaml, depth 0.33 width 0.25), 17x3 keypoints.
    legacy=True lowers the head in the older export form (see _pose_head)."""
    pb = PlanBuilder(out_dir, seed)
    x = pb.input("images", [1, 3, imgsz, imgsz])
    x = pb.conv(x, 16, 3, 2)             # 0
    x = pb.conv(x, 32, 3, 2)             # 1
    x = _c2f(pb, x, 32, 1, True)         # 2
    x = pb.conv(x, 64, 3, 2)             # 3
    p3 = _c2f(pb, x, 64, 2, True)        # 4
    x = pb.conv(p3, 128, 3, 2)           # 5
    p4 = _c2f(pb, x, 128, 2, True)       # 6
    x = pb.conv(p4, 256, 3, 2)           # 7
    x = _c2f(pb, x, 256, 1, True)        # 8
    p5 = _sppf(pb, x, 256)               # 9
    x = pb.concat([pb.upsample(p5), p4])         # 10, 11
    n12 = _c2f(pb, x, 128, 1, False)             # 12
    x = pb.concat([pb.upsample(n12), p3])        # 13, 14
    o3 = _c2f(pb, x, 64, 1, False)               # 15
    x = pb.concat([pb.conv(o3, 64, 3, 2), n12])  # 16, 17
    o4 = _c2f(pb, x, 128, 1, False)              # 18
    x = pb.concat([pb.conv(o4, 128, 3, 2), p5])  # 19, 20
    o5 = _c2f(pb, x, 256, 1, False)              # 21
    out = _pose_head(pb, [o3, o4, o5], legacy=legacy)
    pb.output(out)
    path = pb.write()
    return path, pb.flops


# ----------------------------------------------------------------- YOLO11

def _c3k2(pb, x, c2, n, c3k, shortcut=True, e=0.5):
    """ultralytics C3k2: C2f whose blocks are Bottleneck (c3k=False) or C3k (c3k=True)."""
    c = int(c2 * e)
    y = pb.conv(x, 2 * c, 1)
    ys = pb.split(y, [c, c])
    for _ in range(n):
        src = ys[-1]
        if c3k:  # C3k(c, c, 2, shortcut): cv1/cv2 1x1 (c/2), 2 bottlenecks on cv1, concat, cv3
            h = c // 2
            a = pb.conv(src, h, 1)
            for _ in range(2):
                t = pb.conv(a, h, 3)
                t = pb.conv(t, h, 3)
                a = pb.binary(a, t, 0) if shortcut else t
            b = pb.conv(src, h, 1)
            t = pb.conv(pb.concat([a, b]), c, 1)
        else:  # Bottleneck(c, c, shortcut) with its default e=0.5 hidden width
            t = pb.conv(src, c // 2, 3)
            t = pb.conv(t, c, 3)
            if shortcut:
                t = pb.binary(src, t, 0)
        ys.append(t)
    return pb.conv(_concat_many(pb, ys, 1), c2, 1)


def _attention(pb, x, num_heads, legacy=False):
    """ultralytics Attention (attn_ratio 0.5): qkv 1x1, q^T k * scale, softmax, v attn^T, + pe(v).

    The scale multiplies q^T (a [heads, N, key_dim] tensor) before the product, as in the
    reference's lowered plans (config/tuning.json holds a scalar Mul over 2 x 32 x 400 =
    25600 elements and none over the 2 x 400 x 400 scores); legacy=True multiplies the
    scores after the product instead."""
    _, C, H, W = pb.shapes[x]
    N = H * W
    hd = C // num_heads
    kd = hd // 2
    h = C + kd * num_heads * 2
    qkv = pb.conv(x, h, 1, act=ACT_NONE)
    qkv = pb.reshape(qkv, [1, num_heads, kd * 2 + hd, N])
    q, k, v = pb.split(qkv, [kd, kd, hd], axis=2)
    qt = pb.permute(q, [0, 1, 3, 2])                  # [1, nh, N, kd]
    scale = pb.const(np.array([kd ** -0.5], np.float32), "scale")
    if legacy:
        attn = pb.binary(pb.matmul(qt, k), scale, 2)  # [1, nh, N, N]
    else:
        attn = pb.matmul(pb.binary(qt, scale, 2), k)
    attn = pb.softmax(attn, 3)
    at = pb.permute(attn, [0, 1, 3, 2])
    o = pb.matmul(v, at)                              # [1, nh, hd, N]
    o = pb.reshape(o, [1, C, H, W])
    vv = pb.reshape(v, [1, C, H, W])
    pe = pb.conv(vv, C, 3, groups=C, act=ACT_NONE)
    o = pb.binary(o, pe, 0)
    return pb.conv(o, C, 1, act=ACT_NONE)


def _c2psa(pb, x, c2, n=1, e=0.5, legacy=False):
    c = int(c2 * e)
    y = pb.conv(x, 2 * c, 1)
    a, b = pb.split(y, [c, c])
    for _ in range(n):
        b = pb.binary(b, _attention(pb, b, num_heads=c // 64, legacy=legacy), 0)
        f = pb.conv(b, c * 2, 1)
        f = pb.conv(f, c, 1, act=ACT_NONE)
        b = pb.binary(b, f, 0)
    return pb.conv(pb.concat([a, b]), c2, 1)


def yolo11n_pose(out_dir, seed=0, imgsz=640, legacy=False):
    """YOLO11n-pose (ultralytics yolo11-pose.yaml, depth 0.5 width 0.25).
    legacy=True lowers the head and the C2PSA attention scale in the older export forms
    (see _pose_head and _attention)."""
    pb = PlanBuilder(out_dir, seed)
    x = pb.input("images", [1, 3, imgsz, imgsz])
    x = pb.conv(x, 16, 3, 2)                 # 0
    x = pb.conv(x, 32, 3, 2)                 # 1
    x = _c3k2(pb, x, 64, 1, False, e=0.25)   # 2
    x = pb.conv(x, 64, 3, 2)                 # 3
    p3 = _c3k2(pb, x, 128, 1, False, e=0.25)  # 4
    x = pb.conv(p3, 128, 3, 2)               # 5
    p4 = _c3k2(pb, x, 128, 1, True)          # 6
    x = pb.conv(p4, 256, 3, 2)               # 7
    x = _c3k2(pb, x, 256, 1, True)           # 8
    x = _sppf(pb, x, 256)                    # 9
    p5 = _c2psa(pb, x, 256, legacy=legacy)   # 10
    x = pb.concat([pb.upsample(p5), p4])     # 11, 12
    n13 = _c3k2(pb, x, 128, 1, False)        # 13
    x = pb.concat([pb.upsample(n13), p3])    # 14, 15
    o3 = _c3k2(pb, x, 64, 1, False)          # 16
    x = pb.concat([pb.conv(o3, 64, 3, 2), n13])  # 17, 18
    o4 = _c3k2(pb, x, 128, 1, False)         # 19
    x = pb.concat([pb.conv(o4, 128, 3, 2), p5])  # 20, 21
    o5 = _c3k2(pb, x, 256, 1, True)          # 22
    out = _pose_head(pb, [o3, o4, o5], dw_cls=True, legacy=legacy)
    pb.output(out)
    return pb.write(), pb.flops


# ------------------------------------------------------------ MobileNetV3

def _se(pb, x, sq):
    s = pb.gap(x)
    s = pb.conv(s, sq, 1, act=ACT_RELU)
    s = pb.conv(s, pb.shapes[x][1], 1, act=ACT_HSIGMOID)
    return pb.binary(s, x, 2, out_shape=pb.shapes[x])   # torchvision: scale * input


def mobilenetv3_small(out_dir, seed=0, imgsz=224, num_classes=1000):
    """torchvision mobilenet_v3_small (BN folded), logits [1, 1000]."""
    pb = PlanBuilder(out_dir, seed)
    x = pb.input("input", [1, 3, imgsz, imgsz])
    x = pb.conv(x, 16, 3, 2, act=ACT_HSWISH)
    RE, HS = ACT_RELU, ACT_HSWISH
    cfg = [  # k, exp, out, se, act, s
        (3, 16, 16, True, RE, 2), (3, 72, 24, False, RE, 2), (3, 88, 24, False, RE, 1),
        (5, 96, 40, True, HS, 2), (5, 240, 40, True, HS, 1), (5, 240, 40, True, HS, 1),
        (5, 120, 48, True, HS, 1), (5, 144, 48, True, HS, 1), (5, 288, 96, True, HS, 2),
        (5, 576, 96, True, HS, 1), (5, 576, 96, True, HS, 1)]

    def mdiv(v, d=8):
        nv = max(d, int(v + d / 2) // d * d)
        return nv + d if nv < 0.9 * v else nv

    for k, exp, out, se, act, s in cfg:
        cin = pb.shapes[x][1]
        t = x
        if exp != cin:
            t = pb.conv(t, exp, 1, act=act)
        t = pb.conv(t, exp, k, s, groups=exp, act=act)
        if se:
            t = _se(pb, t, mdiv(exp // 4))
        t = pb.conv(t, out, 1, act=ACT_NONE)
        if s == 1 and cin == out:
            t = pb.binary(t, x, 0)
        x = t
    x = pb.conv(x, 576, 1, act=ACT_HSWISH)
    x = pb.gap(x)
    x = pb.reshape(x, [1, 576])
    x = pb.gemm(x, 1024, act=ACT_HSWISH)
    x = pb.gemm(x, num_classes)
    pb.output(x)
    return pb.write(), pb.flops


# ------------------------------------------------------------- single ops

def single_conv(out_dir, cin, cout, H, W, k=1, s=1, groups=1, act=ACT_SILU, seed=0,
                bias=True, pre_relu=False, post_relu=False):
    """One conv node (the conv sweep configs).  Returns (plan path, FLOPs/image).
    pre_relu: a ReLU between the graph input and the conv, so that the conv reads an
    internal tensor (channels-last in the HIP backend) as it does inside a model.
    post_relu: a ReLU between the conv and the graph output, so that the conv writes an
    internal tensor too (with act = 0 the ReLU folds into the conv)."""
    pb = PlanBuilder(out_dir, seed)
    x = pb.input("x", [1, cin, H, W])
    if pre_relu:
        x = pb.unary(x, UN_RELU)
    y = pb.conv(x, cout, k, s, groups=groups, act=act, bias=bias)
    if post_relu:
        y = pb.unary(y, UN_RELU)
    pb.output(y)
    return pb.write(), pb.flops


def c2psa_attention(out_dir, C=256, H=20, heads=4, seed=0, W=None, legacy=False):
    """The C2PSA attention block alone: input [1, C, H, W] (W = H by default) -> ReLU -> qkv
    1x1, per-head q^T k * scale over H*W tokens, softmax, v attn^T, + depthwise 3x3
    positional conv of v, 1x1 projection (ultralytics Attention, attn_ratio 0.5: head_dim
    C / heads, key_dim head_dim / 2).
    Returns (plan path, FLOPs/image of the attention core: q^T k and v attn^T)."""
    W = H if W is None else W
    pb = PlanBuilder(out_dir, seed=seed)
    # a ReLU first, so that the block reads an internal (channels-last) tensor as in the model
    x = pb.unary(pb.input("images", [1, C, H, W]), UN_RELU)
    pb.output(_attention(pb, x, heads, legacy=legacy))
    N, hd = H * W, C // heads
    core = 2.0 * heads * N * N * (hd // 2) + 2.0 * heads * hd * N * N
    return pb.write(), core


def gemm_plan(out_dir, M, N, K, b_dims=None, seed=0):
    """One plan-level `gemm` node, C[M][N] = A[M][K] . B[K][N] (src/PlanModel.cpp:3935-3990):
    A is an init [M, K], B the plan input with dims b_dims (numel K*N, any rank; default
    [K, N]), C a [M, N] tensor.  A and B are drawn as scripts/kernel_check.py:34-38 draws
    them (default_rng(seed).random, A first, then B, rounded to fp16).  onnx2plan never
    emits this op; a hand-written plan may.  Returns (plan path, B as fp16 [K, N])."""
    b_dims = list(b_dims) if b_dims is not None else [K, N]
    if int(np.prod(b_dims)) != K * N:
        raise ValueError("b_dims must hold K*N elements")
    rng = np.random.default_rng(seed)
    a = rng.random((M, K)).astype(np.float16)
    b = rng.random((K, N)).astype(np.float16)
    pb = PlanBuilder(out_dir, seed)
    x = pb.input("b", b_dims)
    w = pb.init(a.astype(np.float32), "a")
    y = pb.tensor([M, N])
    pb.node("gemm", [w, x], [y])
    pb.flops += 2 * M * N * K
    pb.output(y)
    return pb.write(), b


def conv1x1_config(out_dir, seed=0):
    """Single pointwise conv via the plan's conv1x1 op: Cin=64, Cout=128, 80x80, SiLU;
    X ~ U[0,1), W ~ N(0, sqrt(2/Cin)), bias ~ N(0, 0.01)."""
    return single_conv(out_dir, 64, 128, 80, 80, k=1, act=ACT_SILU, seed=seed)


CONV_SWEEP = [
    # name, cin, cout, H, W, k, s, groups, act
    ("stem3x3s2_3to16_640", 3, 16, 640, 640, 3, 2, 1, ACT_SILU),
    ("conv3x3s2_16to32_320", 16, 32, 320, 320, 3, 2, 1, ACT_SILU),
    ("conv3x3s2_32to64_160", 32, 64, 160, 160, 3, 2, 1, ACT_SILU),
    ("conv3x3s1_64to64_80", 64, 64, 80, 80, 3, 1, 1, ACT_SILU),
    ("conv3x3s1_128to128_40", 128, 128, 40, 40, 3, 1, 1, ACT_SILU),
    ("conv3x3s1_256to256_20", 256, 256, 20, 20, 3, 1, 1, ACT_SILU),
    ("dw3x3s2_16_112", 16, 16, 112, 112, 3, 2, 16, ACT_HSWISH),
    ("dw5x5s1_96_14", 96, 96, 14, 14, 5, 1, 96, ACT_HSWISH),
    ("dw5x5s2_72_28", 72, 72, 28, 28, 5, 2, 72, ACT_HSWISH),
]

MODELS = {"yolov8n-pose": yolov8n_pose, "yolo11n-pose": yolo11n_pose,
          "mobilenetv3-small": mobilenetv3_small}


def write_model(name, out_dir, seed=0):
    return MODELS[name](out_dir, seed=seed)
