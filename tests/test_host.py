"""Host-side tests (no GPU): the plan writer, the C ABI surface, the planner and its
host bounds check (dry run), and the error behaviour of the boundary."""
import os
import re

import numpy as np
import pytest

import infvino_amd as ia
from infvino_amd import planwriter as pw
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRY = ia.IVH_FLAG_DRY_RUN


def test_model_flops_match_reference_accounting(plans):
    # conv+gemm GFLOP per image as the reference reports them (docs/benchmark.md:78-80)
    assert abs(plans("yolov8n-pose")[1] / 1e9 - 9.178) < 0.005
    assert abs(plans("mobilenetv3-small")[1] / 1e9 - 0.110) < 0.005
    assert abs(plans("yolo11n-pose")[1] / 1e9 - 7.406) / 7.406 < 0.02


def test_yolov8_node_census(plans):
    p = O.Plan.load(plans("yolov8n-pose")[0])
    ops = [n.op for n in p.nodes]
    # 45 conv3x3 + 28 conv1x1 per frame, as the reference's y8 budget counts them
    assert ops.count("conv3x3") == 45 and ops.count("conv1x1") == 28
    assert p.dims[p.outputs[0]] == [1, 56, 8400]


def test_header_symbols_exported():
    hdr = open(os.path.join(ROOT, "include", "ivh.h")).read()
    declared = set(re.findall(r"^\s*(?:int|const char \*)\s+(ivh_\w+)\s*\(", hdr, re.M))
    assert declared == set(ia.SIGNATURES), declared ^ set(ia.SIGNATURES)
    L = ia.lib()
    for name in declared:
        assert hasattr(L, name), name


@pytest.mark.parametrize("name", ["yolov8n-pose", "mobilenetv3-small", "yolo11n-pose"])
def test_dry_run_plans_and_bounds(plans, name):
    path = plans(name)[0]
    m = ia.PlanModel(path, 0, 64, DRY)
    for b in (1, 5, 64):
        m.run(b)          # builds every launch and bounds-checks it on the host
    arena, weights = m.memoryInfo(64)
    assert arena > 0 and weights > 0
    kinds = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    assert kinds.count("conv_igemm") > 0
    m.close()


def test_kernel_choice_yolov8(plans):
    """Planner choices at batch 64: the stem kernel for the Cin = 3 conv, the persistent
    stride-2 kernel for the 16->32, 32->64 and 64->128 downsamples, the implicit GEMM for the
    wider ones (128->256), the
    resident-weight kernel for the stride-1 3x3 convs with 16 < Cin <= 64 (but not the
    Cin <= 32 ones with a fused residual), the wide-layer kernel for Cin >= 128 with
    64 < Cout <= 256, the DMA-pipelined kernel for the other Cin > 64 convs on the 40x40 maps
    (enough items for its persistent grid), the fused pair kernel for the three
    32-channel bottlenecks at 80x80 and the 16-channel one at 160x160 (their second conv then
    launches nothing) and the stride-1 LDS-patch kernel for the rest.  Per conv shape, so with
    the heads' sibling convs run apart (their merged launches: test_sibling_conv_merge)."""
    m = ia.PlanModel(plans("yolov8n-pose")[0], 0, 64, DRY | ia.IVH_FLAG_NO_FUSE_SIBLINGS)
    m.run(64)
    info = [m.nodeInfo(i) for i in range(m.nodeCount())]
    by = {i["desc"]: i["kernel"] for i in info}
    assert by["conv3x3 3x640x640->16x320x320 k3 s2 g1 act1"] == "conv_stem"
    assert by["conv3x3 16x320x320->32x160x160 k3 s2 g1 act1"] == "conv_s2p"
    assert by["conv3x3 32x160x160->64x80x80 k3 s2 g1 act1"] == "conv_s2p"
    assert by["conv3x3 64x80x80->128x40x40 k3 s2 g1 act1"] == "conv_s2p"
    assert by["conv3x3 128x40x40->256x20x20 k3 s2 g1 act1"] == "conv_igemm"
    s1 = [(i["kernel"], int(i["desc"].split()[1].split("x")[0]), int(i["desc"].split()[1].split("x")[1]),
           "+res" in i["desc"], int(i["desc"].split("->")[1].split("x")[0]))
          for i in info if i["op"] == "conv3x3" and " s1 " in i["desc"]]

    def want(k, cin, hw, res, cout):
        if (cin, hw) in ((32, 80), (16, 160)) and k in ("conv_pair", "(fused)"):  # bottleneck pairs, one launch
            return True
        if 16 < cin <= 64 and not (res and cin <= 32):
            return k == "conv_res"
        if cin >= 128 and cin % 32 == 0 and 64 < cout <= 256:
            return k == "conv_wide"
        return k == ("conv_pipe" if cin > 64 and hw >= 40 else "conv_halo")
    assert s1 and all(want(k, cin, hw, res, cout) for k, cin, hw, res, cout in s1)
    assert sum(k == "conv_res" for k, *_ in s1) >= 16
    # the P5 C2f bottlenecks of the backbone (with its shortcut) and of the neck: 128 -> 128
    # at 20x20, on the wide-layer kernel
    assert sum(k == "conv_wide" for k, *_ in s1) == 4
    # the heads' last 1x1 convs (box 64 and keypoint 51 planes at three scales) write the NCHW
    # head tensors through the planar-output streaming kernel; the single class plane stays on
    # the implicit GEMM
    planar = sorted(i["desc"].split()[1] for i in info if i["kernel"] == "conv_pw_planar")
    assert planar == sorted(f"{c}x{hw}x{hw}->{o}x{hw}x{hw}" for hw in (80, 40, 20) for c, o in ((51, 51), (64, 64)))
    assert sum(k == "conv_pipe" for k, *_ in s1) >= 3
    assert sum(k == "conv_pair" for k, *_ in s1) == 4 and sum(k == "(fused)" for k, *_ in s1) == 4
    m.close()


def test_kernel_choice_yolo11_pairs(plans):
    """YOLO11n-pose at batch 64: the C3k2 bottlenecks 16 -> 8 -> 16 at 160x160 and 32 -> 16 ->
    32 at 80x80 (with their shortcuts) and the two 32-channel bottlenecks at 40x40 run as
    fused pairs; with IVH_FLAG_NO_FUSE_PAIR none do."""
    m = ia.PlanModel(plans("yolo11n-pose")[0], 0, 64, DRY)
    m.run(64)
    info = [m.nodeInfo(i) for i in range(m.nodeCount())]
    m.close()
    pairs = sorted(i["desc"] for i in info if i["kernel"] == "conv_pair")
    assert pairs == sorted(["conv3x3 16x160x160->8x160x160 k3 s1 g1 act1"] +
                           ["conv3x3 32x80x80->16x80x80 k3 s1 g1 act1"] * 2 +
                           ["conv3x3 32x40x40->32x40x40 k3 s1 g1 act1"] * 2)
    fused = [i["desc"] for i in info if i["kernel"] == "(fused)" and i["op"] == "conv3x3"]
    assert "conv3x3 8x160x160->16x160x160 k3 s1 g1 act1 +res" in fused
    assert fused.count("conv3x3 16x80x80->32x80x80 k3 s1 g1 act1 +res") == 2
    m = ia.PlanModel(plans("yolo11n-pose")[0], 0, 64, DRY | ia.IVH_FLAG_NO_FUSE_PAIR)
    m.run(64)
    assert not any(m.nodeInfo(i)["kernel"] == "conv_pair" for i in range(m.nodeCount()))
    m.close()


@pytest.mark.parametrize("cin,cout,hw,pre,post,batch,want", [
    (64, 128, 80, False, False, 64, "conv_pw_planar"),   # NCHW planes in and out
    (5, 17, 48, False, False, 16, "conv_pw_planar"),     # few planes, ragged Cout
    (64, 128, 10, False, False, 2, "conv_direct"),       # 100-pixel planes: not 8-pixel pieces
    (96, 64, 40, False, False, 4, "conv_igemm"),         # Cin > 64: the implicit GEMM's planar loads
    (64, 136, 40, False, False, 4, "conv_igemm"),        # Cout > 128
    (64, 64, 40, True, False, 4, "conv_pw_planar"),      # channels-last in, NCHW planes out
    (64, 8, 40, True, False, 4, "conv_igemm"),           # a few output planes: the implicit GEMM
    (64, 64, 80, True, True, 64, "conv_pw"),             # channels-last in and out
])
def test_kernel_choice_pointwise(tmp_path, cin, cout, hw, pre, post, batch, want):
    """Which 1x1 kernel the planner picks by layout and shape (dry run): the planar-output
    streaming kernel for NCHW outputs with Cin <= 64, Cout <= 128 (Cout >= 16 from a
    channels-last input) and 8-pixel pieces, the channels-last one for channels-last
    outputs, the implicit GEMM (or the direct kernel) otherwise."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=1, act=pw.ACT_SILU, pre_relu=pre, post_relu=post)
    m = ia.PlanModel(path, 0, batch, DRY)
    m.run(batch)
    kern = next(m.nodeInfo(i)["kernel"] for i in range(m.nodeCount()) if m.nodeInfo(i)["op"].startswith("conv"))
    m.close()
    assert kern == want


def test_kernel_choice_conv1x1_config(tmp_path):
    """The plan's conv1x1 op on graph tensors (NCHW in and out, 64 -> 128 at 80x80) takes the
    planar streaming kernel at batch 1 and 64, and the implicit GEMM with IVH_FLAG_NO_PW."""
    path, _ = pw.conv1x1_config(str(tmp_path))
    for b, fl, want in ((1, 0, "conv_pw_planar"), (64, 0, "conv_pw_planar"), (64, ia.IVH_FLAG_NO_PW, "conv_igemm")):
        m = ia.PlanModel(path, 0, b, DRY | fl)
        m.run(b)
        assert m.nodeInfo(0)["kernel"] == want
        m.close()


@pytest.mark.parametrize("name,cin,cout,H,W,k,s,g,act", pw.CONV_SWEEP, ids=[c[0] for c in pw.CONV_SWEEP])
def test_kernel_choice_sweep(tmp_path, name, cin, cout, H, W, k, s, g, act):
    """Each conv sweep layer at batch 64, as it runs inside a model, gets its kernel family."""
    want = {"stem": "conv_stem", "conv3x3s2_16": "conv_s2p", "conv3x3s2_32": "conv_s2p", "conv3x3s2": "conv_igemm",
            "conv3x3s1_64": "conv_res", "conv3x3s1_128": "conv_wide", "conv3x3s1_256": "conv_wide", "dw": "dwconv"}
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=k, s=s, groups=g, act=act,
                             pre_relu=not name.startswith("stem"), post_relu=True)
    m = ia.PlanModel(path, 0, 64, DRY)
    m.run(64)
    kern = next(m.nodeInfo(i)["kernel"] for i in range(m.nodeCount()) if m.nodeInfo(i)["op"].startswith("conv"))
    m.close()
    assert kern == next(v for key, v in want.items() if name.startswith(key))


# (cin, cout, hw, k, batch) -> launch detail the planner must pick.  Batch 64 runs the wide
# 3x3 layers on LDS-patch configs 3 (32-channel chunks) and 7 (64-channel chunks); these
# small-batch shapes reach the same configs, and the 1x1 shape reaches 769..1024 output tiles
# of the 128-wide im2col tile, the case of its 128-VGPR build.
NW = ia.IVH_FLAG_NO_WIDE
TAGGED = [
    ((128, 128, 160, 3, 2), "conv_halo cfg=7", "ck=64", NW),
    ((96, 136, 96, 3, 2), "conv_halo cfg=7", "ck=64", 0),
    ((128, 128, 224, 3, 2), "conv_halo cfg=3", "ck=32", ia.IVH_FLAG_NO_PIPE | NW),
    ((128, 128, 40, 3, 64), "conv_halo cfg=3", "ck=32", ia.IVH_FLAG_NO_PIPE | NW),
    ((256, 256, 20, 3, 64), "conv_halo cfg=7", "ck=64", NW),
    ((128, 128, 160, 1, 4), "conv_igemm bn=128 bk=32 ksplit=1", "vgpr128", 0),
    ((128, 128, 40, 3, 64), "conv_pipe cfg=0", "items=438", NW),
    ((128, 64, 40, 3, 64), "conv_pipe cfg=1", "items=410", 0),
    ((64, 64, 80, 3, 2), "conv_pipe cfg=1", "items=54", ia.IVH_FLAG_PIPE_ANY),
    ((128, 128, 40, 3, 64), "conv_wide tm=13", "ranges=256", 0),
    ((256, 256, 20, 3, 64), "conv_wide tm=7", "ranges=128", 0),
    ((128, 128, 160, 3, 2), "conv_wide tm=4", "wgs=256", 0),
]


@pytest.mark.parametrize("shape,head,detail,flags", TAGGED,
                         ids=[f"{a}to{b}_{c}_k{d}_b{e}_f{f:x}" for (a, b, c, d, e), _, _, f in TAGGED])
def test_launch_tags(tmp_path, shape, head, detail, flags):
    """ivh_node_tag names the tile config the planner picked (host-only dry run)."""
    cin, cout, hw, k, b = shape
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=k, act=pw.ACT_SILU, pre_relu=True, post_relu=True)
    m = ia.PlanModel(path, 0, b, DRY | flags)
    m.run(b)
    tag = next(m.nodeTag(i) for i in range(m.nodeCount()) if m.nodeInfo(i)["op"].startswith("conv"))
    m.close()
    assert tag.startswith(head) and detail in tag.split(), tag


def test_zero_copy_views_in_c2f(plans):
    """C2f: cv1 output is split by views, the bottleneck outputs and both halves land in the
    concat buffer in place, so no copy_c/concat node launches anything."""
    path = plans("yolov8n-pose")[0]
    m = ia.PlanModel(path, 0, 1, DRY)
    m.run(1)
    info = [m.nodeInfo(i) for i in range(m.nodeCount())]
    assert all(i["kernel"] == "(view)" for i in info if i["op"] == "copy_c")
    chan_concats = [i for i in info if i["op"] == "concat4"]
    assert sum(i["kernel"] == "(view)" for i in chan_concats) >= 12
    # residual adds of the bottlenecks are folded into the conv epilogue
    assert not any(i["op"] == "ew_binary" and "+res" in i["desc"] for i in info)
    assert sum("+res" in i["desc"] for i in info) == 6
    m.close()


@pytest.mark.parametrize("flags", [ia.IVH_FLAG_NO_FUSE, ia.IVH_FLAG_NCHW_ONLY, ia.IVH_FLAG_DIRECT_ONLY,
                                   ia.IVH_FLAG_NO_REUSE])
def test_dry_run_variants(plans, flags):
    m = ia.PlanModel(plans("yolov8n-pose", imgsz=320)[0], 0, 4, DRY | flags)
    m.run(4)
    m.close()


def _write(tmp_path, text, bins=()):
    for name, n in bins:
        np.zeros(n, np.float16).tofile(tmp_path / name)
    p = tmp_path / "model.plan"
    p.write_text(text)
    return str(p)


@pytest.mark.parametrize("text,bins,msg", [
    ("tensor y 1 4\nnode ew_unary x y op=1 n=4\noutput y\n", (), "plan has no 'input' line"),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary x y op=1 n=4\n", (), "plan has no 'output' line"),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary x y op=1 n=4\noutput z\n", (), "output tensor not declared: z"),
    ("input x 1 4\ntensor y 1 4\nnode frobnicate x y\noutput y\n", (), "unknown op: frobnicate"),
    ("input x 1 4\ninit w w.bin 4 4\ntensor y 1 4\nnode conv1x1 w,x,-,- y\noutput y\n", (), "cannot open init"),
    ("input x 1 4\ninit w w.bin 4 4\ntensor y 1 4\nnode conv1x1 w,x,-,- y\noutput y\n", [("w.bin", 7)], "too short"),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary q y op=1 n=4\noutput y\n", (), "missing tensor: q"),
    ("input x 1 8 4 4\ninit w w.bin 8 8 3 3\ntensor y 1 8 4 4\nnode conv3x3 x,w,-,- y stride=1 pad=1 Hout=5 Wout=4\noutput y\n",
     [("w.bin", 576)], "Hout/Wout inconsistent"),
])
def test_malformed_plans_raise(tmp_path, text, bins, msg):
    path = _write(tmp_path, text, bins)
    with pytest.raises(RuntimeError, match=re.escape(msg)):
        m = ia.PlanModel(path, 0, 1, DRY)
        m.run(1)


def test_gemm_op_dims_dry_run(tmp_path):
    """The plan's gemm op takes M = A.dims[0], K = A.dims[1], N = numel(B) / K
    (src/PlanModel.cpp:3935-3940): a rank-4 B [1, K, H, W] plans as an M x K x H*W product
    (host bounds check included); an output whose numel is not M*N is rejected."""
    path, _ = pw.gemm_plan(str(tmp_path), 48, 20 * 24, 64, b_dims=[1, 64, 20, 24])
    m = ia.PlanModel(path, 0, 3, DRY)
    m.run(3)
    info = [m.nodeInfo(i) for i in range(m.nodeCount())]
    g = next(i for i in info if i["op"] == "gemm")
    assert g["flops"] == 2.0 * 48 * 64 * 480
    m.close()
    text = open(path).read().replace("tensor t2 48 480", "tensor t2 48 479")
    assert text != open(path).read()
    bad = tmp_path / "bad.plan"
    bad.write_text(text)
    with pytest.raises(RuntimeError, match="gemm output numel"):
        m = ia.PlanModel(str(bad), 0, 1, DRY)
        m.run(1)


def test_batch_range_checked(plans):
    m = ia.PlanModel(plans("mobilenetv3-small")[0], 0, 2, DRY)
    with pytest.raises(RuntimeError, match="out of range"):
        m.run(3)
    with pytest.raises(RuntimeError, match="out of range"):
        m.run(0)
    m.close()


def test_missing_plan_file():
    with pytest.raises(RuntimeError, match="cannot open plan"):
        ia.PlanModel("/nonexistent/model.plan", 0, 1, DRY)


def test_no_device_fails_loudly(plans):
    """Without the dry-run flag and without a GPU the boundary raises (no CPU fallback)."""
    if ia.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="HIP error"):
        ia.PlanModel(plans("mobilenetv3-small")[0], 0, 1)


def test_rel_errors_definition():
    ref = np.array([1.0, -2.0, 4.0, 0.5])
    got = ref + np.array([0.01, 0.0, -0.04, 0.0])
    mean_rel, max_rel, max_abs, scale_rel = O.rel_errors(got, ref)
    assert np.isclose(mean_rel, 0.0125 / 1.875) and np.isclose(max_rel, 0.01)
    assert np.isclose(max_abs, 0.04) and np.isclose(scale_rel, 0.0125 / 4)


def test_cpp_backend_image_slicing(tmp_path):
    """HipBackend::image: outputs of a batched inference sliced back to one image each (the
    per-image view the reference's decoders take), host code only."""
    import subprocess
    src = tmp_path / "t.cpp"
    src.write_text(r"""
#include "infvino_hip/HipBackend.hpp"
#include <cstdio>
using infvino_hip::HipBackend; using infvino_hip::Tensor;
int main() {
  Tensor a({3, 2, 4}, {}), c({3, 5}, {});
  for (int i = 0; i < 24; ++i) a.data.push_back((float)i);
  for (int i = 0; i < 15; ++i) c.data.push_back(100.0f + i);
  for (int b = 0; b < 3; ++b) {
    auto im = HipBackend::image({a, c}, b, 3);
    if (im.size() != 2 || im[0].shape != std::vector<int64_t>{1, 2, 4} || im[1].shape != std::vector<int64_t>{1, 5}) return 1;
    for (int i = 0; i < 8; ++i) if (im[0].data[i] != (float)(8 * b + i)) return 2;
    for (int i = 0; i < 5; ++i) if (im[1].data[i] != 100.0f + 5 * b + i) return 3;
  }
  try { HipBackend::image({a}, 3, 3); return 4; } catch (const std::runtime_error &) {}
  try { HipBackend::image({c}, 0, 2); return 5; } catch (const std::runtime_error &) {}
  std::puts("ok");
  return 0;
}
""")
    exe = tmp_path / "t"
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout)


def test_cpp_headers_compile(tmp_path):
    """include/infvino_hip/*.hpp compile as a C++17 translation unit against include/ivh.h."""
    import subprocess
    src = tmp_path / "t.cpp"
    src.write_text('#include "infvino_hip/HipBackend.hpp"\n'
                   'struct MI { std::string plan, device; };\n'
                   'int main() { MI m{"x.plan", "GPU.0"}; (void)sizeof(infvino_hip::HipBackend); '
                   'if (0) { infvino_hip::HipBackend b(m); infvino_hip::HipBackend c(m, true); '
                   'infvino_hip::HipBackend d(m, false, 8); } return 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # an int second argument (an older max_batch signature) does not compile
    bad = tmp_path / "bad.cpp"
    bad.write_text('#include "infvino_hip/HipBackend.hpp"\n'
                   'struct MI { std::string plan, device; };\n'
                   'int main() { MI m{"x.plan", "GPU.0"}; if (0) { infvino_hip::HipBackend b(m, 4); } return 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(bad)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "deleted" in r.stderr, r.stderr


def test_py_backend_image_slicing():
    """HipBackend.image (Python mirror): same slicing and errors as the C++ helper."""
    from infvino_amd import HipBackend, Tensor
    a = Tensor([3, 2, 4], np.arange(24, dtype=np.float32).reshape(3, 2, 4))
    c = Tensor([3, 5], 100 + np.arange(15, dtype=np.float32).reshape(3, 5))
    for b in range(3):
        ia, ic = HipBackend.image([a, c], b, 3)
        assert ia.shape == [1, 2, 4] and ic.shape == [1, 5]
        np.testing.assert_array_equal(ia.data.ravel(), np.arange(8 * b, 8 * b + 8))
        np.testing.assert_array_equal(ic.data.ravel(), 100 + np.arange(5 * b, 5 * b + 5))
    with pytest.raises(RuntimeError):
        HipBackend.image([a], 3, 3)
    with pytest.raises(RuntimeError):
        HipBackend.image([c], 0, 2)


def pool_chain_plan(d, C=16, H=20):
    """Three chained 5x5 stride-1 max pools with no concat after them: pool i reads only the
    previous pool's output, so each intermediate dies one node after it is born."""
    pb = pw.PlanBuilder(d, seed=0)
    x = pb.input("x", [1, C, H, H])
    a = pb.conv(x, C, 1)
    b = pb.maxpool(a, 5, 1, 2)
    c = pb.maxpool(b, 5, 1, 2)
    e = pb.maxpool(c, 5, 1, 2)
    pb.output(pb.conv(e, C, 1))
    return pb.write()


def test_sppf_chain_lifetimes(tmp_path):
    """The fused SPPF launch reads the chain input and writes all three pool outputs at once,
    so the memory plan must keep all four apart even where each pool output has a single
    reader (the chain input dies at the first pool node otherwise and a later pool output
    would take its bytes).  The arena therefore holds four 20x20x16 channels-last buffers."""
    m = ia.PlanModel(pool_chain_plan(str(tmp_path)), 0, 2, DRY)
    m.run(2)
    kinds = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    assert kinds.count("maxpool_sppf") == 1 and kinds.count("(fused)") == 2, kinds
    arena, _ = m.memoryInfo(1)
    assert arena >= 4 * 20 * 20 * 16 * 2, arena
    m.close()


def test_launch_plans_per_batch(plans):
    """Launch lists and their per-node ranges are kept per batch size: labelling and
    re-running alternate batch sizes sees each batch's own plan."""
    m = ia.PlanModel(plans("yolov8n-pose", imgsz=320)[0], 0, 5, DRY)
    m.run(1)
    k1 = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    m.run(5)
    m.run(3)
    m.run(1)
    k2 = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    assert k1 == k2
    m.close()


def test_labels_follow_last_batch(plans):
    """Kernel labels describe the batch of the last run: YOLOv8n-pose at 640 splits K at
    batch 1 (grids too small to fill the chip) and not at batch 64, and the pipelined 3x3
    kernel runs only at batch 64 (on the heads' 128 -> 64 / 51 convs, run apart here: merged they
    take the wide-layer kernel)."""
    m = ia.PlanModel(plans("yolov8n-pose")[0], 0, 64, DRY | ia.IVH_FLAG_NO_FUSE_SIBLINGS)
    m.run(64)
    k64 = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    t64 = [m.nodeTag(i) for i in range(m.nodeCount())]
    m.run(1)
    k1 = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    assert "conv_igemm_sk" in k1 and "conv_igemm_sk" not in k64
    assert "conv_pipe" in k64 and "conv_pipe" not in k1
    m.run(64)
    assert [m.nodeTag(i) for i in range(m.nodeCount())] == t64
    m.close()


REF_INCLUDE = "/root/reference/include"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF_INCLUDE, "infvino")), reason="reference headers absent")
def test_cpp_backend_binds_reference_types(tmp_path):
    """Built inside the reference tree (INFVINO_HIP_USE_INFVINO_TENSOR), HipBackend returns the
    reference's own infvino::Tensor and infvino::DeviceInfo (include/infvino/Tensor.hpp,
    Device.hpp), takes ClBackend's (ModelInfo, bool profiling) constructor, and serves the
    calls InferenceEngine (InferenceEngine.hpp:60), infvino_bench.cpp:89-97 and
    infvino_numtest.cpp:84-98 make on a ClBackend.  Compiled and linked against the library;
    nothing runs on a device."""
    import subprocess
    src = tmp_path / "bind.cpp"
    src.write_text(r'''
#include <cstdio>
#include <memory>
#include "infvino_hip/HipBackend.hpp"
#include "infvino/Device.hpp"
#include "infvino/Tensor.hpp"
struct ModelInfo { std::string plan, device = "AUTO"; };  // the members ClBackend reads
template <class Backend> int use(Backend & be, const std::vector<float> & buf)
{
  const infvino::DeviceInfo & dev = be.device();
  for (const auto & d : dev.available) std::printf(" %s", d.c_str());
  std::printf("%s -> %s%s (%s) %s %u %u\n", dev.requested.c_str(), dev.resolved.c_str(),
              dev.fell_back_to_cpu ? " [CPU FALLBACK]" : "", dev.full_name.c_str(), dev.opencl_version.c_str(),
              dev.eu, dev.clock_mhz);
  std::vector<infvino::Tensor> outputs = be.infer(buf.data(), buf.size());
  const std::vector<int64_t> & in = be.inputDims();
  const std::vector<std::vector<int64_t>> & shapes = be.outputShapes();
  return (int)(outputs.size() + in.size() + shapes.size() + (be.lastInferMs() > 0));
}
int main(int argc, char **)
{
  ModelInfo info{"m.plan", "GPU.0"};
  if (argc > 5) {
    infvino_hip::HipBackend be(info, false);
    auto shared = std::make_shared<infvino_hip::HipBackend>(info, true);
    return use(be, {}) + use(*shared, {});
  }
  std::printf("ok\n");
  return 0;
}
''')
    exe = tmp_path / "bind"
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-DINFVINO_HIP_USE_INFVINO_TENSOR",
                        "-I", os.path.join(ROOT, "include"), "-I", REF_INCLUDE, str(src), "-o", str(exe),
                        "-L", os.path.join(ROOT, "infvino_amd"), "-linfvino_hip",
                        "-Wl,-rpath," + os.path.join(ROOT, "infvino_amd")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)


MALFORMED = [c[:2] for c in [
    ("tensor y 1 4\nnode ew_unary x y op=1 n=4\noutput y\n", ()),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary x y op=1 n=4\n", ()),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary x y op=1 n=4\noutput z\n", ()),
    ("input x 1 4\ntensor y 1 4\nnode frobnicate x y\noutput y\n", ()),
    ("input x 1 4\ninit w w.bin 4 4\ntensor y 1 4\nnode conv1x1 w,x,-,- y\noutput y\n", ()),
    ("input x 1 4\ninit w w.bin 4 4\ntensor y 1 4\nnode conv1x1 w,x,-,- y\noutput y\n", [("w.bin", 7)]),
    ("input x 1 4\ntensor y 1 4\nnode ew_unary q y op=1 n=4\noutput y\n", ()),
    ("input x 1 8 4 4\ninit w w.bin 8 8 3 3\ntensor y 1 8 4 4\nnode conv3x3 x,w,-,- y stride=1 pad=1 Hout=5 Wout=4\n"
     "output y\n", [("w.bin", 576)]),
    ("input x 1 4\ntensor y 1 4\nnode slice_axis x y outer=1 axdim=4 inner=1 start=3 len=4\noutput y\n", ()),
    ("input x 1 4 4\ntensor y 1 4 4\nnode maxpool x y C=4 H=4 W=4 Hout=4 Wout=4 K=99 S=1 P=2\noutput y\n", ()),
    ("", ()),
]]


def test_host_sanitizers(plans, tmp_path):
    """The planner's host code built with AddressSanitizer and UndefinedBehaviorSanitizer
    (make -C infvino_amd/csrc asan; device code unchanged) runs every model as a dry run at
    batch 1 / 5 / 64 / 3 / 1 under seven flag sets -- planning, packing, the memory plan's
    overlap check and every launch's host bounds check -- and rejects malformed plans with an
    error; any invalid access or undefined behaviour aborts the run."""
    import shutil
    import subprocess
    clang = "/opt/rocm/llvm/bin/clang++"
    if not os.path.exists(clang) or not shutil.which("make"):
        pytest.skip("no clang++ / make")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "infvino_amd", "csrc"), "asan", "-j8"], check=True,
                   capture_output=True)
    out = os.path.join(ROOT, "tests", "cpp", "_build", "asan")
    exe = os.path.join(out, "dry_run_checks")
    r = subprocess.run([clang, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
                        "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cpp", "dry_run_checks.cpp"),
                        "-o", exe, "-L", out, "-linfvino_hip", "-Wl,-rpath," + out], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    good = [plans(n)[0] for n in ("yolov8n-pose", "mobilenetv3-small", "yolo11n-pose")]
    good += [pw.c2psa_attention(str(tmp_path / "attn"))[0], pool_chain_plan(str(tmp_path / "pool"))]
    bad = []
    for i, (text, bins) in enumerate(MALFORMED):
        d = tmp_path / f"bad{i}"
        d.mkdir()
        bad.append(_write(d, text, bins))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe] + good + ["--"] + bad, capture_output=True, text=True, env=env, timeout=600)
    print(r.stdout[-2000:], r.stderr[-4000:])
    assert r.returncode == 0 and "0 failures" in r.stdout


@pytest.mark.parametrize("name", ["yolov8n-pose", "yolo11n-pose"])
def test_upsample_concat_fusion(plans, name):
    """Both neck upsamples (Upsample -> Concat -> the C2f / C3k2 cv1 1x1) fold into their 1x1
    conv at every batch size; IVH_FLAG_NO_FUSE_UPSAMPLE (and IVH_FLAG_NO_REUSE, which promises
    readable intermediates) keep the resize launches."""
    path = plans(name)[0]
    for flags, fused in ((0, True), (ia.IVH_FLAG_NO_FUSE_UPSAMPLE, False), (ia.IVH_FLAG_NO_REUSE, False)):
        m = ia.PlanModel(path, 0, 64, DRY | flags)
        for b in (1, 64):
            m.run(b)
            info = [m.nodeInfo(i) for i in range(m.nodeCount())]
            tags = [m.nodeTag(i) for i in range(m.nodeCount())]
            resize = [i["kernel"] for i in info if i["op"] == "resize_nn"]
            assert len(resize) == 2
            assert resize == (["(fused)"] * 2 if fused else ["resize_nn"] * 2), resize
            up = [i["desc"] for i, t in zip(info, tags) if "upsample-concat" in t]
            want = {"yolov8n-pose": ["conv1x1 384x40x40->128x40x40", "conv1x1 192x80x80->64x80x80"],
                    "yolo11n-pose": ["conv1x1 384x40x40->128x40x40", "conv1x1 256x80x80->64x80x80"]}[name]
            assert [d.split(" k1")[0] for d in up] == (want if fused else []), up
        m.close()


def test_sibling_conv_merge(plans):
    """The Pose heads' first 3x3 convs per level (YOLOv8n: box, class and keypoint branches,
    64 + 64 + 51 channels, written as 3 x 64; YOLO11n: box and keypoint, 64 + 51 as 2 x 64, its
    class branch starting with a depthwise conv) run as one conv per level, their second convs
    as one grouped launch; IVH_FLAG_NO_FUSE_SIBLINGS runs them apart."""
    for name, per_level, groups in (("yolov8n-pose", "siblings=3 cout=192", "groups=3 cout=179"),
                                    ("yolo11n-pose", "siblings=2 cout=128", "groups=2 cout=115")):
        for flags, merged in ((0, True), (ia.IVH_FLAG_NO_FUSE_SIBLINGS, False)):
            m = ia.PlanModel(plans(name)[0], 0, 64, DRY | flags)
            for b in (1, 64):
                m.run(b)
                tags = [m.nodeTag(i) for i in range(m.nodeCount())]
                assert sum(per_level in t for t in tags) == (3 if merged else 0), (name, b, flags)
                assert not any("siblings" in t and per_level not in t for t in tags)
                if merged and b == 64:
                    # P3 (64 in): the resident-weight ping-pong kernel over the merged channel
                    # blocks; P4 / P5 (128 / 256 in): the wide-layer kernel
                    kinds = [t.split()[0] for t in tags if per_level in t]
                    assert kinds == ["conv_res", "conv_wide", "conv_wide"], kinds
                # the branches' second convs (on consecutive 64-channel views of the merged
                # root, the keypoint branch's 51 channels zero-padded) as one grouped ping-pong
                # launch per level
                grouped = [t for t in tags if groups in t]
                assert len(grouped) == (3 if merged else 0), (name, b, grouped)
                assert all(t.startswith("conv_res cfg=3") for t in grouped)
            m.close()
