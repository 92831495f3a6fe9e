"""Op-level parity on the GPU: single-node plans through the C ABI vs the CPU oracle.

Protocol of scripts/kernel_check.py (reference): seeded inputs, relative errors
mean|d|/mean|ref| and max|d|/max|ref|; contract mean_rel < 1e-2, max_rel < 5e-2 against
the reference-rounding oracle (IVO_REF, fp16 accumulation as the reference kernels do).
Against the fp32 oracle (one fp16 rounding, the HIP kernels' own semantics) the bar is
tighter: mean_rel < 2e-3, max_rel < 1e-2.  Data-movement ops must be bit-exact.
"""
import numpy as np
import pytest

import infvino_amd as ia
from infvino_amd import planwriter as pw
from oracle import oracle as O

pytestmark = pytest.mark.gpu

OP_MEAN, OP_MAX = 1e-2, 5e-2          # scripts/kernel_check.py:20-22
F32_MEAN, F32_MAX = 2e-3, 1e-2


def _run(path, batch, seed=0, lo=0.0, hi=1.0, flags=0):
    p = O.Plan.load(path)
    rng = np.random.default_rng(seed)
    x = O.f2h((lo + (hi - lo) * rng.random(p.numel(p.input_name) * batch)).astype(np.float32))
    m = ia.PlanModel(path, 0, batch, flags)
    m.setInput(x, batch)
    m.run(batch)
    got = [m.readOutput(i, batch) for i in range(m.outputCount())]
    m.close()
    return p, x, got


def _kernels(path, batch, flags=0):
    """Kernel labels the planner picks for each node at `batch` (host-only dry run)."""
    m = ia.PlanModel(path, 0, batch, flags | ia.IVH_FLAG_DRY_RUN)
    m.run(batch)
    labels = [m.nodeInfo(i)["kernel"] for i in range(m.nodeCount())]
    m.close()
    return labels


def _conv_kernel(path, batch, flags=0):
    return next(k for k in _kernels(path, batch, flags) if k.startswith(("conv", "dwconv")))


def _diagnose(g, r):
    """On a mismatch: where and how the result differs (printed with the failure)."""
    gf, rf = O.h2f(g).ravel(), O.h2f(r).ravel()
    bad = np.flatnonzero(np.abs(gf - rf) > 1e-2 * (np.abs(rf).max() + 1e-6))
    print(f"  mismatching elements {bad.size} of {gf.size}; first at {bad[:8].tolist()}")
    print(f"  got NaN {int(np.isnan(gf).sum())} zeros {int((gf == 0).sum())}; got[:8] {gf[:8]} ref[:8] {rf[:8]}")


def _check_f32(path, batch, seed=0, ref_mode=True, **kw):
    p, x, got = _run(path, batch, seed, **kw)
    ref = O.run_plan(p, x, batch)
    for g, r in zip(got, ref):
        mean_rel, max_rel, max_abs, _ = O.rel_errors(O.h2f(g), O.h2f(r.ravel()))
        print(f"{path}: vs f32 oracle mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} max_abs={max_abs:.2e}")
        if not (mean_rel < F32_MEAN and max_rel < F32_MAX):
            _diagnose(g, r)
        assert mean_rel < F32_MEAN and max_rel < F32_MAX
    if ref_mode:
        refr = O.run_plan(p, x, batch, mode=O.REF)
        for g, r in zip(got, refr):
            mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(g), O.h2f(r.ravel()))
            print(f"   vs reference-rounding oracle mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
            assert mean_rel < OP_MEAN and max_rel < OP_MAX
    return got


def test_conv1x1_config(tmp_path):
    """Single pointwise conv via the plan's conv1x1 op: 64->128 @ 80x80, SiLU."""
    path, _ = pw.conv1x1_config(str(tmp_path))
    for b in (1, 3):
        _check_f32(path, b)


SWEEP_KERNEL = {"stem": ("conv_stem",), "dw": ("dwconv",),
                "conv3x3s2": ("conv_igemm", "conv_igemm_sk", "conv_s2", "conv_s2p"),
                "conv3x3s1": ("conv_igemm", "conv_igemm_sk", "conv_halo", "conv_res", "conv_pipe")}


@pytest.mark.parametrize("name,cin,cout,H,W,k,s,g,act", pw.CONV_SWEEP, ids=[c[0] for c in pw.CONV_SWEEP])
def test_conv_sweep(tmp_path, name, cin, cout, H, W, k, s, g, act):
    """The conv sweep layers as they run inside a model: every conv but the stem reads an
    internal (channels-last) tensor."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=k, s=s, groups=g, act=act,
                             pre_relu=not name.startswith("stem"))
    assert _conv_kernel(path, 2) in next(v for k, v in SWEEP_KERNEL.items() if name.startswith(k))
    _check_f32(path, 2, ref_mode=(H * W * cin <= 160 * 160 * 32))


@pytest.mark.parametrize("cin,cout,hw,k,s,g", [(16, 32, 40, 3, 2, 1), (64, 64, 20, 3, 1, 1), (32, 64, 12, 3, 1, 4)])
def test_conv_direct_nchw(tmp_path, cin, cout, hw, k, s, g):
    """A conv reading the NCHW graph input (and grouped convs) runs the direct kernel."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=k, s=s, groups=g, act=pw.ACT_SILU)
    assert _conv_kernel(path, 2) == "conv_direct"
    _check_f32(path, 2)


@pytest.mark.parametrize("cin,cout,hw,k,s,act", [
    (48, 32, 20, 1, 1, 1),     # ragged tiles: M not a multiple of 128
    (51, 51, 20, 3, 1, 1),     # Cin not a multiple of 8 (pose keypoint branch)
    (24, 40, 9, 3, 2, 3),      # odd spatial, stride 2, HardSwish
    (16, 1, 12, 1, 1, 0),      # Cout = 1
    (256, 256, 5, 3, 1, 1),    # Cout > BN (two N tiles)
    (40, 72, 7, 5, 1, 2),      # 5x5 dense conv via conv_general
    (64, 64, 6, 3, 1, 4),      # HardSigmoid after 3x3 (unfused in the plan, folded at load)
    (3, 32, 17, 3, 1, 1),      # stem MFMA path, two 16-channel tiles, ragged pixel groups
    (3, 8, 15, 3, 2, 3),       # stem MFMA path, Cout < 16
    (2, 16, 9, 3, 1, 1),       # stem MFMA path, Cin = 2
])
def test_conv_shapes(tmp_path, cin, cout, hw, k, s, act):
    """Shape classes of the MFMA families (internal channels-last input) and of the stem
    (the graph input)."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=k, s=s, act=act, pre_relu=cin > 3)
    kern = _conv_kernel(path, 3)
    assert kern == "conv_stem" if cin <= 3 else kern in ("conv_igemm", "conv_igemm_sk", "conv_halo", "conv_res", "conv_pipe",
                                                         "conv_pw_planar")
    _check_f32(path, 3, lo=-1.0)
    if kern == "conv_pw_planar":  # the implicit GEMM on the same layer too
        assert _conv_kernel(path, 3, ia.IVH_FLAG_NO_PW) == "conv_igemm"
        _check_f32(path, 3, lo=-1.0, flags=ia.IVH_FLAG_NO_PW)


@pytest.mark.parametrize("cin,cout,H,W,batch,s", [
    (64, 64, 80, 80, 2, 1),    # the YOLOv8 80x80 bottleneck shape
    (48, 40, 33, 35, 2, 1),    # ragged 8x16 tiles on both axes
    (24, 16, 40, 24, 3, 1),    # Cin < 32: one zero-filled chunk
    (51, 51, 48, 48, 1, 1),    # Cin not a multiple of 8 (pose keypoint branch)
    (96, 136, 24, 40, 2, 1),   # Cout > 128: two N tiles, 16x8 tiles
])
def test_halo_conv3x3(tmp_path, cin, cout, H, W, batch, s):
    """3x3 stride-1 convs through the LDS-patch kernel vs the oracle and vs the im2col path."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=s, act=pw.ACT_SILU, pre_relu=True)
    nr = ia.IVH_FLAG_NO_RESIDENT | ia.IVH_FLAG_NO_SPLITK
    assert _conv_kernel(path, batch, nr) == "conv_halo"
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_HALO | ia.IVH_FLAG_NO_SPLITK) == "conv_igemm"
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False, flags=nr)
    _, _, im2col = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_HALO | ia.IVH_FLAG_NO_SPLITK)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(im2col[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (64, 64, 40, 40, 8, pw.ACT_SILU),     # BN 64 x CK 64 (the YOLO head / bottleneck class)
    (64, 64, 40, 40, 64, pw.ACT_SILU),    # two tiles per work-group (persistent loop)
    (32, 64, 40, 40, 96, pw.ACT_SILU),    # three rounds: odd and even tile counts per work-group
    (51, 51, 24, 24, 8, pw.ACT_SILU),     # Cin, Cout % 8 != 0: masked patch, padding-channel stores
    (32, 32, 40, 40, 6, pw.ACT_HSWISH),   # BN 32, 512-pixel tiles, HardSwish
    (24, 24, 64, 64, 32, pw.ACT_SILU),    # ragged CK 32, BN 32, two rounds
    (20, 64, 32, 32, 6, pw.ACT_SILU),     # ragged CK 32 with BN 64
    (24, 40, 33, 35, 6, pw.ACT_SILU),     # ragged Cin and Cout, odd H and W
    (64, 24, 40, 40, 6, pw.ACT_SILU),     # BN 32 with CK 64
    (32, 96, 24, 24, 8, pw.ACT_SILU),     # two channel blocks
])
def test_res_conv3x3(tmp_path, cin, cout, H, W, batch, act):
    """3x3 stride-1 convs with 16 < Cin <= 64 through the resident-weight kernel vs the oracle
    and vs the LDS-patch kernel (input and output channels-last, as inside a model)."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=1, act=act, pre_relu=True, post_relu=True)
    print(f"res conv {cin}->{cout} {H}x{W} batch {batch} act {act}", flush=True)
    assert _conv_kernel(path, batch) == "conv_res"
    nr = ia.IVH_FLAG_NO_RESIDENT | ia.IVH_FLAG_NO_SPLITK
    assert _conv_kernel(path, batch, nr) in ("conv_halo", "conv_igemm")
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=nr)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


def test_res_residual_chain(tmp_path):
    """Bottleneck chain of 48 channels at batch 24 (3x3 SiLU, 3x3 + residual) and a 3x3
    without activation + residual: the resident-weight kernel with the fused residual add."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, 48, 40, 40]), pw.UN_RELU)
        t = pb.conv(x, 48, 3)
        t = pb.conv(t, 48, 3)
        y = pb.binary(x, t, 0)
        u = pb.conv(y, 48, 3, act=pw.ACT_NONE)
        z = pb.binary(y, u, 0)
        return pb.unary(z, pw.UN_RELU)
    path = _small_plan(tmp_path, build)
    assert _kernels(path, 24).count("conv_res") == 3
    got = _check_f32(path, 24, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, 24, lo=-1.0, flags=ia.IVH_FLAG_NO_RESIDENT)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (64, 64, 80, 80, 64, pw.ACT_SILU),    # the 64->64 @80 layer of the YOLO heads: 6-7 tiles per work-group
    (64, 51, 80, 80, 16, pw.ACT_SILU),    # Cout 51 (the pose head): stores reach the view's padding
    (48, 64, 33, 35, 6, pw.ACT_HSWISH),   # Cin 48: two 8-channel pieces read as zeros; odd map
    (64, 96, 24, 24, 8, pw.ACT_SILU),     # two channel blocks, the second 32 channels wide
    (40, 40, 20, 20, 3, pw.ACT_RELU),     # small maps: tiles across image boundaries
    (64, 64, 40, 40, 1, pw.ACT_SILU),     # batch 1: eight work-groups of one tile each
    (56, 128, 16, 16, 2, pw.ACT_SILU),    # 16x16: one tile column, two full channel blocks
])
def test_pingpong_conv3x3(tmp_path, cin, cout, H, W, batch, act):
    """3x3 stride-1 convs with 32 < Cin <= 64, Cin % 8 == 0 and Cout > 32 through the
    ping-pong resident-weight kernel (config 3) vs the oracle, and vs the single-group kernel
    (config 0): both accumulate every 32 x 32 block over the same K slices in the same order,
    config 3 from the bias instead of zero, so the fp32 sums differ only in rounding and the
    fp16 outputs by at most two units in the last place (two where the fp32 values straddle
    a power of two)."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=1, act=act, pre_relu=True, post_relu=True)
    print(f"ping-pong conv {cin}->{cout} {H}x{W} batch {batch} act {act}", flush=True)
    tags = _conv_tags(path, batch)
    assert tags[0].startswith("conv_res cfg=3"), tags
    assert _conv_tags(path, batch, ia.IVH_FLAG_NO_PINGPONG)[0].startswith("conv_res cfg=0")
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PINGPONG)
    _assert_ulp2(got[0], other[0])


def _assert_ulp2(a, b):
    """fp16 bit patterns of non-negative outputs (the plans end in a ReLU) at most 2 apart."""
    d = np.abs(np.asarray(a).view(np.uint16).astype(np.int32) - np.asarray(b).view(np.uint16).astype(np.int32))
    print(f"   vs config 0: {int((d > 0).sum())} of {d.size} outputs differ, max {int(d.max())} ulp")
    assert d.max() <= 2 and (d > 0).mean() < 1e-2


def test_pingpong_residual_chain(tmp_path):
    """Bottleneck chain of 64 channels at batch 24 (3x3 SiLU, 3x3 + residual, 3x3 without
    activation + residual) through the ping-pong kernel's fused residual add."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, 64, 40, 40]), pw.UN_RELU)
        t = pb.conv(x, 64, 3)
        t = pb.conv(t, 64, 3)
        y = pb.binary(x, t, 0)
        u = pb.conv(y, 64, 3, act=pw.ACT_NONE)
        z = pb.binary(y, u, 0)
        return pb.unary(z, pw.UN_RELU)
    path = _small_plan(tmp_path, build)
    tags = _conv_tags(path, 24)
    assert len(tags) == 3 and all(t.startswith("conv_res cfg=3") for t in tags), tags
    got = _check_f32(path, 24, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, 24, lo=-1.0, flags=ia.IVH_FLAG_NO_PINGPONG)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (128, 128, 40, 40, 2, pw.ACT_SILU),    # BN 128 (config 0), four 32-channel chunks
    (72, 64, 33, 35, 2, pw.ACT_SILU),      # BN 64, a last chunk of 8 channels, odd H and W
    (96, 136, 24, 40, 2, pw.ACT_SILU),     # two channel blocks, the second 8 channels wide
    (64, 51, 48, 48, 1, pw.ACT_HSWISH),    # Cout 51: 8-channel stores reach the view's padding
    (256, 256, 20, 20, 2, pw.ACT_RELU),    # eight chunks, two blocks of 128 channels
    (32, 64, 80, 80, 32, pw.ACT_SILU),     # one chunk per item, 810 items: several per work-group
    (40, 24, 20, 20, 6, pw.ACT_RELU),      # two chunks (8 real channels in the second), BN 64
])
def test_pipe_conv3x3(tmp_path, cin, cout, H, W, batch, act):
    """3x3 stride-1 convs through the DMA-pipelined kernel (forced with IVH_FLAG_PIPE_ANY at
    these small sizes) vs the oracle and vs the other 3x3 kernels."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=1, act=act, pre_relu=True, post_relu=True)
    print(f"pipe conv {cin}->{cout} {H}x{W} batch {batch} act {act}", flush=True)
    assert _conv_kernel(path, batch, ia.IVH_FLAG_PIPE_ANY) == "conv_pipe"
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_PIPE) != "conv_pipe"
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False, flags=ia.IVH_FLAG_PIPE_ANY)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PIPE)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,want", [
    (128, 128, 40, 40, 64, "tm=13"),   # the 128->128 sweep layer: one pass of 13 blocks per work-group
    (256, 256, 20, 20, 64, "tm=7"),    # the 256->256 sweep layer: two channel groups, 16 chunks
    (128, 96, 40, 40, 39, "tm=10"),    # a channel block past Cout (96 of 128)
    (128, 256, 40, 40, 24, "tm=10"),
    (128, 96, 20, 20, 49, "tm=4"),     # 20x20: passes across image boundaries
    (128, 96, 20, 20, 39, "tm=2"),
    (128, 256, 20, 20, 49, "tm=7"),
    (256, 128, 20, 20, 64, ""),        # sixteen chunks, one channel group
    (128, 128, 33, 35, 40, ""),        # odd map: rows of 35, passes starting mid-row
    (192, 96, 40, 40, 16, ""),         # twelve chunks
])
def test_wide_conv3x3(tmp_path, cin, cout, H, W, batch, want):
    """3x3 stride-1 convs through the wide-layer kernel (one work-group per CU over an equal
    share of the pixels) vs the oracle and vs the kernel the planner picks without it."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=1, act=pw.ACT_SILU, pre_relu=True, post_relu=True)
    print(f"wide conv {cin}->{cout} {H}x{W} batch {batch}", flush=True)
    tags = _conv_tags(path, batch)
    assert tags[0].startswith("conv_wide " + want), tags
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_WIDE) != "conv_wide"
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_WIDE)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    print(f"   vs other kernel mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3


def _conv_tags(path, batch, flags=0):
    m = ia.PlanModel(path, 0, batch, flags | ia.IVH_FLAG_DRY_RUN)
    m.run(batch)
    tags = [m.nodeTag(i) for i in range(m.nodeCount()) if m.nodeInfo(i)["kernel"].startswith("conv")]
    m.close()
    return tags


@pytest.mark.parametrize("C,H,W,batch,want", [
    (128, 40, 40, 64, "tm=13"), (128, 40, 40, 39, "tm=10"), (128, 40, 40, 24, "tm=7"),
    (128, 20, 20, 49, "tm=4"), (128, 20, 20, 39, "tm=2"), (256, 20, 20, 49, "tm=7"),
])
def test_wide_residual_chain(tmp_path, C, H, W, batch, want):
    """Bottleneck chain (3x3 SiLU, 3x3 SiLU + residual, 3x3 SiLU + residual) through the
    wide-layer kernel with the fused residual add."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, C, H, W]), pw.UN_RELU)
        t = pb.conv(x, C, 3)
        t = pb.conv(t, C, 3)
        y = pb.binary(x, t, 0)
        u = pb.conv(y, C, 3)
        z = pb.binary(y, u, 0)
        return pb.unary(z, pw.UN_RELU)
    path = _small_plan(tmp_path, build)
    print(f"wide residual chain C {C} {H}x{W} batch {batch}", flush=True)
    tags = _conv_tags(path, batch)
    assert len(tags) == 3 and all(t.startswith("conv_wide") for t in tags), tags
    assert tags[1].startswith("conv_wide " + want) and tags[2].startswith("conv_wide " + want), tags
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_WIDE)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("C,H,W,batch,res,act1,act2", [
    (32, 80, 80, 2, True, pw.ACT_SILU, pw.ACT_SILU),     # the YOLOv8 C2f bottleneck at 80x80
    (32, 80, 80, 3, False, pw.ACT_SILU, pw.ACT_SILU),    # no shortcut (the neck's C2f)
    (32, 33, 35, 2, True, pw.ACT_HSWISH, pw.ACT_RELU),   # odd map: ragged tiles on both axes
    (32, 20, 20, 6, True, pw.ACT_SILU, pw.ACT_NONE),     # small maps: tiles across image boundaries
    (32, 40, 40, 1, False, pw.ACT_RELU, pw.ACT_SILU),    # batch 1
    (32, 80, 80, 16, True, pw.ACT_SILU, pw.ACT_SILU),    # several tiles per work-group
    (16, 160, 160, 2, True, pw.ACT_SILU, pw.ACT_SILU),   # the YOLOv8 C2f bottleneck at 160x160
    (16, 33, 35, 3, False, pw.ACT_HSWISH, pw.ACT_RELU),  # 16 channels: ragged tiles, no shortcut
    (16, 20, 20, 6, True, pw.ACT_RELU, pw.ACT_NONE),     # 16 channels: tiles across image boundaries
    (16, 160, 160, 9, True, pw.ACT_SILU, pw.ACT_SILU),   # 16 channels: several tiles per work-group
    (-16, 160, 160, 2, True, pw.ACT_SILU, pw.ACT_SILU),  # 16 -> 8 -> 16: the YOLO11 C3k2 bottleneck at 160x160
    (-16, 33, 35, 3, False, pw.ACT_HSWISH, pw.ACT_RELU), # 8-channel middle: ragged tiles, no shortcut
    (-16, 20, 20, 6, True, pw.ACT_RELU, pw.ACT_NONE),    # 8-channel middle: tiles across image boundaries
    (-32, 80, 80, 2, True, pw.ACT_SILU, pw.ACT_SILU),    # 32 -> 16 -> 32: the YOLO11 C3k2 bottleneck at 80x80
    (-32, 33, 35, 3, False, pw.ACT_HSWISH, pw.ACT_RELU), # 16-channel middle: ragged tiles, no shortcut
])
def test_conv_pair(tmp_path, C, H, W, batch, res, act1, act2):
    """A bottleneck of C = 16 or 32 channels (3x3 -> 3x3, optionally + the block input) as one
    launch of the fused pair kernel vs the oracle and vs the two convs run apart; C < 0: -C
    outer channels with a middle of half as many (16 -> 8 -> 16, 32 -> 16 -> 32)."""
    mid = -C // 2 if C < 0 else C
    C = abs(C)
    def build(pb):
        x = pb.unary(pb.input("x", [1, C, H, W]), pw.UN_RELU)
        t = pb.conv(x, mid, 3, act=act1)
        t = pb.conv(t, C, 3, act=act2)
        if res:
            t = pb.binary(x, t, 0)
        return pb.unary(t, pw.UN_RELU)
    path = _small_plan(tmp_path, build)
    print(f"conv pair C {C} mid {mid} {H}x{W} batch {batch} res {res} acts {act1} {act2}", flush=True)
    assert _kernels(path, batch).count("conv_pair") == 1
    assert "conv_pair" not in _kernels(path, batch, ia.IVH_FLAG_NO_FUSE_PAIR)
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_FUSE_PAIR)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    print(f"   vs unfused mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3


def test_pipe_residual_chain(tmp_path):
    """Bottleneck chain of 64 channels at batch 8 (3x3 SiLU, 3x3 + residual, 3x3 without
    activation + residual) through the DMA-pipelined kernel with the fused residual add."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, 64, 40, 40]), pw.UN_RELU)
        t = pb.conv(x, 64, 3)
        t = pb.conv(t, 64, 3)
        y = pb.binary(x, t, 0)
        u = pb.conv(y, 64, 3, act=pw.ACT_NONE)
        z = pb.binary(y, u, 0)
        return pb.unary(z, pw.UN_RELU)
    path = _small_plan(tmp_path, build)
    assert _kernels(path, 8, ia.IVH_FLAG_PIPE_ANY).count("conv_pipe") == 3
    got = _check_f32(path, 8, lo=-1.0, ref_mode=False, flags=ia.IVH_FLAG_PIPE_ANY)
    _, _, other = _run(path, 8, lo=-1.0, flags=ia.IVH_FLAG_NO_PIPE)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch", [
    (16, 32, 64, 64, 3),       # the YOLO 16->32 downsample shape class: 128-pixel tiles
    (16, 64, 40, 40, 2),       # 16 in, 64 out: 64-pixel tiles, two channel blocks
    (12, 40, 33, 35, 2),       # Cin % 16 != 0 (zeroed pad channels), odd H / W: bottom / right pad
    (9, 24, 9, 70, 3),         # 9 channels (one real channel in the second piece), wide and short
    (16, 8, 3, 5, 2),          # a 2 x 3 output: one mostly empty tile per image
])
def test_conv3x3_s2(tmp_path, cin, cout, H, W, batch):
    """3x3 stride-2 convs of few channels through the LDS-patch kernel of conv_s2.hip vs the
    oracle and vs the im2col path."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=2, act=pw.ACT_SILU, pre_relu=True)
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_SPLITK) == "conv_s2"
    _check_f32(path, batch, lo=-1.0, ref_mode=False, flags=ia.IVH_FLAG_NO_SPLITK)


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (32, 64, 160, 160, 8, pw.ACT_SILU),    # the YOLOv8 32->64 downsample at 160x160
    (16, 32, 320, 320, 3, pw.ACT_SILU),    # the YOLOv8 16->32 downsample at 320x320
    (28, 40, 97, 131, 8, pw.ACT_RELU),     # Cin 28 (ragged 32-channel chunk), odd map: ragged tiles
    (12, 24, 130, 70, 20, pw.ACT_HSWISH),  # Cin 12 (ragged 16-channel chunk), 8 x 16 tiles
    (32, 32, 64, 96, 48, pw.ACT_SILU),     # 32 -> 32 (one 32-channel block)
    (64, 128, 80, 80, 36, pw.ACT_SILU),    # the YOLOv8 64->128 downsample: 64 channels in, two 64-channel blocks
    (64, 64, 80, 80, 36, pw.ACT_RELU),     # the neck's 64->64 downsample
    (60, 96, 66, 90, 40, pw.ACT_HSWISH),   # Cin 60 (ragged 64-channel chunk), Cout 96 (half-empty second block)
])
def test_conv3x3_s2_persistent(tmp_path, cin, cout, H, W, batch, act):
    """3x3 stride-2 convs through the persistent resident-weight kernel of conv_s2.hip vs the
    oracle and vs the same conv with that kernel switched off."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=3, s=2, act=act, pre_relu=True, post_relu=True)
    print(f"persistent s2 conv {cin}->{cout} {H}x{W} batch {batch} act {act}", flush=True)
    assert _conv_kernel(path, batch) == "conv_s2p"
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_S2_PERSIST) != "conv_s2p"
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_S2_PERSIST)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


def test_conv3x3_s2_persistent_no_act(tmp_path):
    """The persistent stride-2 kernel without an activation (its output read by a 1x1 conv,
    so no later activation folds into it), at batch 40 (960 tiles of 4 x 16)."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, 32, 64, 96]), pw.UN_RELU)
        t = pb.conv(x, 64, 3, s=2, act=pw.ACT_NONE)
        return pb.conv(t, 32, 1)
    path = _small_plan(tmp_path, build)
    kinds = _kernels(path, 40)
    assert kinds.count("conv_s2p") == 1
    got = _check_f32(path, 40, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, 40, lo=-1.0, flags=ia.IVH_FLAG_NO_S2_PERSIST)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (32, 32, 160, 160, 2, pw.ACT_SILU),    # the YOLOv8 C2f 1x1 at 160x160
    (96, 64, 80, 80, 6, pw.ACT_SILU),      # 96 -> 64: two 64-channel K chunks (one half empty), two 32-channel blocks
    (48, 24, 97, 61, 8, pw.ACT_HSWISH),    # K 48 (a partly empty chunk), Cout 24, odd pixel count
    (512, 24, 20, 30, 64, pw.ACT_RELU),    # K 512 (eight chunks), Cout 24 (ragged 32-channel block)
    (64, 56, 80, 80, 6, pw.ACT_SILU),      # Cout 56 (ragged second 32-channel block)
    (51, 48, 80, 80, 6, pw.ACT_SILU),      # Cin 51: the last 8-channel piece masked past Cin
    (64, 64, 40, 40, 24, pw.ACT_NONE),     # no activation
    (96, 128, 80, 80, 6, pw.ACT_SILU),     # four 32-channel blocks per wave (YOLO11n C3k2 cv2 at 80x80)
    (64, 100, 80, 80, 6, pw.ACT_RELU),     # Cout 100: ragged fourth block
])
def test_conv1x1_streaming(tmp_path, cin, cout, H, W, batch, act):
    """1x1 convs through the streaming pointwise kernel of conv_pw.hip vs the oracle and vs
    the implicit GEMM."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, cin, H, W]), pw.UN_RELU)
        t = pb.conv(x, cout, 1, act=act)
        return pb.conv(t, 16, 1)  # read channels-last, so no activation folds into the first
    path = _small_plan(tmp_path, build)
    print(f"streaming 1x1 {cin}->{cout} {H}x{W} batch {batch} act {act}", flush=True)
    kinds = _kernels(path, batch)
    assert kinds.count("conv_pw") >= 1, kinds
    assert "conv_pw" not in _kernels(path, batch, ia.IVH_FLAG_NO_PW)
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PW)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("cin,cout,H,W,batch,act", [
    (64, 128, 80, 80, 6, pw.ACT_SILU),     # the plan's conv1x1 op at the reference's benchmark shape
    (48, 96, 40, 56, 16, pw.ACT_HSWISH),   # K 48 in a 64-channel step, Cout 96 (a half-empty last block)
    (24, 40, 56, 57, 11, pw.ACT_RELU),     # K 24, Cout 40; 3192-pixel planes (blocks straddle images, ragged last block)
    (5, 17, 48, 48, 16, pw.ACT_NONE),      # 5 input planes, 17 output planes, no activation
    (-51, 51, 40, 40, 4, pw.ACT_SILU),     # channels-last in (Cin 51: the last piece masked), planes out
    (-64, 64, 20, 20, 3, pw.ACT_NONE),     # the heads' box conv at 20x20 (two blocks straddle images)
    (-24, 100, 24, 16, 5, pw.ACT_HSWISH),  # channels-last K 24 in one 32-channel step, Cout 100
])
def test_conv1x1_planar(tmp_path, cin, cout, H, W, batch, act):
    """1x1 convs into NCHW planes (graph outputs) through the planar-output streaming kernel
    of conv_pw.hip, vs the oracle and vs the implicit GEMM: from NCHW planes (the graph
    input), or, with cin < 0, from a channels-last internal tensor (a ReLU first)."""
    pre = cin < 0
    cin = abs(cin)
    path, _ = pw.single_conv(str(tmp_path), cin, cout, H, W, k=1, act=act, pre_relu=pre)
    print(f"planar 1x1 {cin}->{cout} {H}x{W} batch {batch} act {act} channels-last in {pre}", flush=True)
    assert _kernels(path, batch).count("conv_pw_planar") == 1
    assert "conv_pw_planar" not in _kernels(path, batch, ia.IVH_FLAG_NO_PW)
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, other = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PW)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(other[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


def test_halo_residual_chain(tmp_path):
    """Bottleneck chain (3x3, 3x3 + residual) on 48x48: halo kernel with the fused residual."""
    def build(pb):
        x = pb.unary(pb.input("x", [1, 32, 48, 48]), pw.UN_RELU)
        t = pb.conv(x, 32, 3)
        t = pb.conv(t, 32, 3)
        return pb.binary(x, t, 0)
    path = _small_plan(tmp_path, build)
    nr = ia.IVH_FLAG_NO_RESIDENT | ia.IVH_FLAG_NO_SPLITK
    assert _kernels(path, 2, nr).count("conv_halo") == 2
    _check_f32(path, 2, lo=-1.0, flags=nr)


@pytest.mark.parametrize("cin,cout,hw,k,batch,want", [
    (128, 128, 160, 3, 2, "cfg=7"), (96, 136, 96, 3, 2, "cfg=7"), (128, 128, 224, 3, 2, "cfg=3"),
    (128, 128, 160, 1, 4, "vgpr128")])
def test_tile_configs(tmp_path, cin, cout, hw, k, batch, want):
    """The LDS-patch configs that batch 64 uses for the wide 3x3 layers (3: 32-channel chunks,
    7: 64-channel chunks, 96 -> 136 leaving a ragged last chunk and a partial output tile)
    and the 128-VGPR build of the 128-wide im2col tile, reached at small batch, against the
    oracle."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=k, act=pw.ACT_SILU, pre_relu=True)
    m = ia.PlanModel(path, 0, batch, ia.IVH_FLAG_DRY_RUN | ia.IVH_FLAG_NO_PIPE)
    m.run(batch)
    tag = next(m.nodeTag(i) for i in range(m.nodeCount()) if m.nodeInfo(i)["op"].startswith("conv"))
    m.close()
    print(tag)
    assert want in tag.split()
    _check_f32(path, batch, lo=-1.0, ref_mode=False, flags=ia.IVH_FLAG_NO_PIPE)


@pytest.mark.parametrize("cin,cout,hw,k,s,batch", [
    (256, 256, 20, 3, 1, 1),   # batch 1: 8 output tiles, 72 K tiles -> split-K
    (128, 51, 40, 3, 1, 1),
    (512, 256, 20, 1, 1, 1),
    (384, 128, 40, 1, 1, 2),
    (128, 256, 40, 3, 2, 3),
])
def test_split_k(tmp_path, cin, cout, hw, k, s, batch):
    """Small-M / long-K convs take the split-K path (partials + fixed-order reduce)."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=k, s=s, act=pw.ACT_SILU, pre_relu=True)
    assert _conv_kernel(path, batch) == "conv_igemm_sk"
    assert _conv_kernel(path, batch, ia.IVH_FLAG_NO_SPLITK) != "conv_igemm_sk"
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, nosplit = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_SPLITK)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(nosplit[0]))
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("internal,post", [(False, False), (True, False), (False, True)],
                         ids=["nchw_input", "channels_last", "nchw_in_channels_last_out"])
@pytest.mark.parametrize("c,hw,k,s,act", [(16, 112, 3, 2, 3), (96, 14, 5, 1, 3), (72, 28, 5, 2, 3),
                                          (20, 9, 3, 1, 2), (24, 10, 5, 2, 4), (64, 23, 3, 1, 1)])
def test_depthwise(tmp_path, c, hw, k, s, act, internal, post):
    """Depthwise convs on the plan's NCHW graph input (a strip of pixels of one channel plane
    per lane), on an internal channels-last tensor (8 channels x a strip of pixels per lane;
    odd widths leave partial strips), and from the NCHW input into an internal channels-last
    tensor (the planar kernel storing through the output view)."""
    path, _ = pw.single_conv(str(tmp_path), c, c, hw, hw, k=k, s=s, groups=c, act=act, pre_relu=internal,
                             post_relu=post)
    assert _conv_kernel(path, 2) == "dwconv"
    _check_f32(path, 2, lo=-1.0)


@pytest.mark.parametrize("c,h,w,k,s,p,act", [
    (64, 80, 80, 3, 1, 1, 1), (128, 40, 40, 3, 1, 1, 1), (16, 112, 112, 3, 2, 1, 0), (96, 14, 14, 5, 2, 2, 0)])
def test_depthwise_kernel_check_shapes(tmp_path, c, h, w, k, s, p, act):
    """scripts/kernel_check.py:94-99's depthwise shapes on its own data (gen_depthwise,
    :121-138: default_rng(0), x ~ N(0,1), w = 0.2 N(0,1), b ~ N(0,1), all fp16) as image 0 of
    a batch of 2, checked against kernel_check's reference (fp32 taps, act(acc + b) -> fp16)
    with its op contract; image 1 is uniform in [-1, 1).  Both images against the fp32 oracle
    and the reference-rounding oracle.  Activation codes 0 and 1 (none, SiLU) mean the same in
    the canonical and conv_general.cl numbering.  The conv reads the NCHW graph input, as
    kernel_check's kernels do."""
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal((c, h, w)).astype(np.float16)
    wt = (rng.standard_normal((c, k, k)).astype(np.float16) * 0.2).astype(np.float16)
    bt = rng.standard_normal(c).astype(np.float16)
    pb = pw.PlanBuilder(str(tmp_path), seed=0)
    y = pb.conv(pb.input("x", [1, c, h, w]), c, k, s, groups=c, act=act, pad=p,
                weight=wt.astype(np.float32).reshape(c, 1, k, k), bias_val=bt.astype(np.float32))
    pb.output(y)
    path = pb.write()
    assert _conv_kernel(path, 2) == "dwconv"
    ho, wo = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    xp = np.pad(x0.astype(np.float32), ((0, 0), (p, p), (p, p)))
    acc = np.zeros((c, ho, wo), np.float32)
    for kh in range(k):
        for kw in range(k):
            acc += xp[:, kh:kh + ho * s:s, kw:kw + wo * s:s] * wt[:, kh, kw].astype(np.float32)[:, None, None]
    acc += bt.astype(np.float32)[:, None, None]
    kc = (acc / (1.0 + np.exp(-acc)) if act == 1 else acc).astype(np.float16).astype(np.float32).ravel()
    x1 = O.f2h((2.0 * np.random.default_rng(7).random(c * h * w) - 1.0).astype(np.float32))
    x = np.concatenate([x0.view(np.uint16).ravel(), x1])
    print(f"depthwise {c}x{h}x{w} K{k} s{s} p{p} act{act} batch 2", flush=True)
    m = ia.PlanModel(path, 0, 2)
    m.setInput(x, 2)
    m.run(2)
    got = m.readOutput(0, 2).reshape(2, -1)
    m.close()
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), kc)
    print(f"   vs kernel_check reference mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < OP_MEAN and max_rel < OP_MAX
    plan = O.Plan.load(path)
    for mode, lim in ((O.F32, (F32_MEAN, F32_MAX)), (O.REF, (OP_MEAN, OP_MAX))):
        ref = O.run_plan(plan, x, 2, mode=mode)[0]
        for i in range(2):
            mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[i]), O.h2f(ref[i].ravel()))
            print(f"   image {i} vs oracle mode {mode} mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
            assert mean_rel < lim[0] and max_rel < lim[1]


@pytest.mark.parametrize("c,hw,k,s,batches", [
    (16, 112, 3, 2, (1, 6)), (64, 80, 3, 1, (1, 3)), (240, 14, 5, 1, (1, 9)), (576, 7, 5, 1, (1, 5)),
    (88, 28, 3, 1, (2, 4)), (120, 33, 5, 2, (1, 3)), (8, 61, 5, 1, (1, 2)), (40, 45, 3, 2, (3, 1)),
    (96, 56, 5, 2, (48, 1))])  # batch 48: the 5x5 stride-2 strip kernel; batch 1: tiled
def test_depthwise_tiles(tmp_path, c, hw, k, s, batches):
    """Channels-last depthwise over tile grids with ragged right and bottom edges, several
    channel tiles and sizes whose tile choice (or kernel) changes with the batch: every batch
    size agrees with the oracle, and image 0 is bit-identical across batch sizes (the
    per-pixel sum order does not depend on the tile or kernel)."""
    path, _ = pw.single_conv(str(tmp_path), c, c, hw, hw, k=k, s=s, groups=c, act=pw.ACT_HSWISH, pre_relu=True)
    outs = []
    for b in batches:
        assert _conv_kernel(path, b) == "dwconv"
        outs.append(_check_f32(path, b, lo=-1.0, ref_mode=False)[0])
    n0 = outs[0].size // batches[0]
    for o, b in zip(outs[1:], batches[1:]):
        assert np.array_equal(o[:n0], outs[0][:n0])


def _small_plan(d, build):
    pb = pw.PlanBuilder(str(d), seed=3)
    out = build(pb)
    pb.output(out)
    return pb.write()


def _sppf_pools(pb, x):
    y = [x]
    for _ in range(3):
        y.append(pb.maxpool(y[-1], 5, 1, 2))
    return pb.concat(y)


SMALL = {
    "maxpool5": lambda pb: pb.maxpool(pb.input("x", [1, 24, 13, 17]), 5, 1, 2),
    "maxpool3s2": lambda pb: pb.maxpool(pb.input("x", [1, 8, 15, 15]), 3, 2, 1),
    "resize2": lambda pb: pb.upsample(pb.input("x", [1, 40, 7, 9]), 2),
    "softmax_inner": lambda pb: pb.softmax(pb.input("x", [1, 4, 16, 300]), 2),
    "softmax_last": lambda pb: pb.softmax(pb.input("x", [1, 2, 40, 40]), 3),
    "permute0213": lambda pb: pb.permute(pb.input("x", [1, 4, 16, 50]), [0, 2, 1, 3]),
    "permute0132": lambda pb: pb.permute(pb.input("x", [1, 3, 7, 11]), [0, 1, 3, 2]),
    "slice_axis2": lambda pb: pb.slice(pb.input("x", [1, 17, 3, 40]), 2, 1, 2),
    "concat_ch": lambda pb: pb.concat([pb.input("x", [1, 5, 6, 7]),
                                       pb.unary(pb.const(np.ones((1, 3, 6, 7)), "k"), 2)]),
    "concat_axis2": lambda pb: pb.concat([pb.reshape(pb.input("x", [1, 6, 4, 5]), [1, 6, 20]),
                                          pb.const(np.arange(60).reshape(1, 6, 10) / 7.0, "k")], axis=2),
    "ew_add_bcast": lambda pb: pb.binary(pb.input("x", [1, 17, 2, 30]), pb.const(np.linspace(-1, 1, 60).reshape(2, 30), "k"), 0),
    # 8-wide broadcast kernel: vector loads of both operands, a scalar operand, a row operand
    "ew_add_bcast8": lambda pb: pb.binary(pb.input("x", [1, 17, 2, 32]), pb.const(np.linspace(-1, 1, 64).reshape(2, 32), "k"), 0),
    "ew_mul_scalar8": lambda pb: pb.binary(pb.input("x", [1, 17, 2, 40]), pb.const(np.array([2.0]), "k"), 2),
    "ew_mul_row8": lambda pb: pb.binary(pb.input("x", [1, 17, 2, 40]), pb.const(np.linspace(1, 3, 40).reshape(1, 40), "k"), 2),
    # channels-last pools (between two ReLUs both tensors are internal)
    "maxpool5_nhwc": lambda pb: pb.unary(pb.maxpool(pb.unary(pb.input("x", [1, 24, 13, 17]), 2), 5, 1, 2), 2),
    "maxpool3s2_nhwc": lambda pb: pb.unary(pb.maxpool(pb.unary(pb.input("x", [1, 16, 15, 15]), 2), 3, 2, 1), 2),
    # SPPF: three chained 5x5 pools into a channel concat, one fused launch (odd 13x19 map:
    # windows clipped on every side)
    "sppf3": lambda pb: pb.unary(_sppf_pools(pb, pb.unary(pb.input("x", [1, 24, 13, 19]), 2)), 2),
    "ew_mul_stride": lambda pb: pb.binary(pb.input("x", [1, 4, 30]), pb.const(np.linspace(1, 3, 30).reshape(1, 30), "k"), 2),
    "ew_div_scalar": lambda pb: pb.binary(pb.input("x", [1, 3, 9, 9]), pb.const(np.array([2.0]), "k"), 3),
    "ew_sub_same": lambda pb: pb.binary(pb.const(np.linspace(0, 5, 2 * 33).reshape(1, 2, 33), "k"), pb.input("x", [1, 2, 33]), 1),
    "unary_sigmoid": lambda pb: pb.unary(pb.input("x", [1, 5, 40]), 0),
    "unary_hswish": lambda pb: pb.unary(pb.input("x", [1, 6, 8, 8]), 3),
    "gap": lambda pb: pb.gap(pb.input("x", [1, 24, 11, 13])),
    "bmm": lambda pb: pb.matmul(pb.reshape(pb.input("x", [1, 2, 40, 32]), [1, 2, 40, 32]),
                                pb.const(np.random.default_rng(0).normal(0, 0.2, (1, 2, 32, 24)), "k")),
}


EXACT = {"maxpool5", "maxpool3s2", "maxpool5_nhwc", "maxpool3s2_nhwc", "resize2", "permute0213", "permute0132", "slice_axis2",
         "concat_ch", "concat_axis2", "sppf3"}


@pytest.mark.parametrize("name", sorted(SMALL))
def test_small_ops(tmp_path, name):
    path = _small_plan(tmp_path, SMALL[name])
    if name == "sppf3":
        assert _kernels(path, 3).count("maxpool_sppf") == 1
    p, x, got = _run(path, 3, lo=-3.0, hi=3.0)
    ref = O.run_plan(p, x, 3)[0].ravel()
    g = got[0]
    exact = name in EXACT
    if exact:
        assert np.array_equal(g, ref), f"{name}: data movement must be bit-exact"
    else:
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(g), O.h2f(ref))
        print(f"{name}: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
        if not (mean_rel < F32_MEAN and max_rel < F32_MAX):
            _diagnose(g, ref)
        assert mean_rel < F32_MEAN and max_rel < F32_MAX


def test_se_block_channel_broadcast(tmp_path):
    """SE: gap -> 1x1 ReLU -> 1x1 HardSigmoid -> channel-broadcast Mul on a channels-last tensor."""
    def build(pb):
        x = pb.input("x", [1, 16, 12, 12])
        t = pb.conv(x, 32, 3, 1, act=pw.ACT_HSWISH)
        t = pb.conv(t, 32, 3, 1, groups=32, act=pw.ACT_HSWISH)
        t = pw._se(pb, t, 8)
        return pb.conv(t, 16, 1, act=pw.ACT_NONE)
    path = _small_plan(tmp_path, build)
    _check_f32(path, 3, lo=-1.0)


def test_c2f_zero_copy_concat(tmp_path):
    """C2f (split views + bottleneck residual + 4-way concat written in place) and SPPF."""
    def build(pb):
        x = pb.input("x", [1, 32, 20, 20])
        y = pw._c2f(pb, x, 64, 2, True)
        return pw._sppf(pb, y, 64)
    path = _small_plan(tmp_path, build)
    _check_f32(path, 2, lo=-1.0)
    # same result with every view/fusion switched off and with NCHW everywhere
    p, x, base = _run(path, 2, lo=-1.0)
    for flags in (ia.IVH_FLAG_NO_FUSE, ia.IVH_FLAG_NCHW_ONLY | ia.IVH_FLAG_NO_REUSE, ia.IVH_FLAG_DIRECT_ONLY):
        _, _, alt = _run(path, 2, lo=-1.0, flags=flags)
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(alt[0]), O.h2f(base[0]))
        assert mean_rel < F32_MEAN and max_rel < F32_MAX, flags


def test_pool_chain_without_concat(tmp_path):
    """Three chained 5x5 max pools whose outputs each have one reader: the fused SPPF launch
    reads the chain input while writing all three outputs, which the memory plan keeps
    apart (a pool output placed over the chain input would corrupt it)."""
    from tests.test_host import pool_chain_plan
    path = pool_chain_plan(str(tmp_path))
    assert _kernels(path, 2).count("maxpool_sppf") == 1
    _check_f32(path, 2, lo=-1.0, ref_mode=False)


@pytest.mark.parametrize("cin,cout,hw,batch", [
    (64, 128, 80, 3),     # config 1 on three images
    (20, 40, 24, 2),      # Cin % 8 != 0: channels past Cin read zeros
    (384, 64, 16, 1),     # long K at batch 1 (split-K); 384 planes reach past (HW - 1) * HW
    (256, 136, 12, 5),    # Cout > 128, 8-pixel pieces crossing tiles and images
    (64, 128, 10, 2),     # 100-pixel planes: not a multiple of 8 -> direct kernel
])
def test_conv1x1_planar_input(tmp_path, cin, cout, hw, batch):
    """1x1 convs reading the plan's NCHW graph input (BASELINE config 1's shape class): the
    implicit GEMM (IVH_FLAG_NO_PW) loads 8-pixel pieces of each channel plane and transposes
    them in LDS; by default Cin <= 64, Cout <= 128 go to the planar streaming kernel."""
    path, _ = pw.single_conv(str(tmp_path), cin, cout, hw, hw, k=1, act=pw.ACT_SILU)
    kern = _conv_kernel(path, batch, ia.IVH_FLAG_NO_PW)
    assert kern == "conv_direct" if (hw * hw) % 8 else kern in ("conv_igemm", "conv_igemm_sk")
    planar = (hw * hw) % 8 == 0 and cin <= 64 and cout <= 128
    assert (_conv_kernel(path, batch) == "conv_pw_planar") == planar
    _check_f32(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PW)
    if planar:
        _check_f32(path, batch, lo=-1.0)
    if kern == "conv_igemm_sk":
        _check_f32(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_PW | ia.IVH_FLAG_NO_SPLITK)


@pytest.mark.parametrize("C,H,heads,batch,legacy", [(256, 20, 4, 3, False), (128, 20, 2, 2, False),
                                                    (256, 16, 4, 2, False), (128, 12, 2, 3, False),
                                                    (128, 8, 2, 5, False), (128, 20, 2, 2, True),
                                                    (256, 12, 4, 3, True)])
def test_attention_fused(tmp_path, C, H, heads, batch, legacy):
    """The C2PSA attention block (ultralytics Attention: qkv 1x1, q^T k * scale, softmax,
    v P^T, + depthwise positional conv, 1x1 projection) with the core as one fused kernel,
    against the oracle and against the same plan run node by node (IVH_FLAG_NO_FUSE_ATTN);
    400 / 256 / 144 / 64 tokens (13 / 8 / 5 / 2 key blocks of 32); the scale on q^T before
    the product (ultralytics 8.4 exports) and, legacy, on the scores after it."""
    print(f"attention C {C} {H}x{H} heads {heads} batch {batch} legacy {legacy}", flush=True)
    path, _ = pw.c2psa_attention(str(tmp_path), C=C, H=H, heads=heads, legacy=legacy)
    assert "attention" in _kernels(path, batch)
    assert "attention" not in _kernels(path, batch, ia.IVH_FLAG_NO_FUSE_ATTN)
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, nodes = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_FUSE_ATTN)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(nodes[0]))
    print(f"fused vs node by node: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3


@pytest.mark.parametrize("H,W,fused", [(12, 30, True), (20, 24, False)])
def test_attention_rectangular(tmp_path, H, W, fused):
    """Non-square maps: 12x30 = 360 tokens (12 key blocks, fused) and 20x24 = 480 tokens
    (more keys than the fused kernel holds: the planner keeps the four nodes), each against
    the oracle and against the node-by-node plan."""
    path, _ = pw.c2psa_attention(str(tmp_path), C=128, H=H, W=W, heads=2)
    print(f"attention {H}x{W} fused {fused}", flush=True)
    assert ("attention" in _kernels(path, 2)) == fused
    got = _check_f32(path, 2, lo=-1.0, ref_mode=False)
    _, _, nodes = _run(path, 2, lo=-1.0, flags=ia.IVH_FLAG_NO_FUSE_ATTN)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(nodes[0]))
    print(f"fused vs node by node: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3


def test_attention_large_scores(tmp_path):
    """Inputs in [-30, 30]: scores in the thousands, so exp(T - m) must take the difference
    before the exponent (an fp32 rounding of m log2e alone would exceed fp16's half ulp); the
    fused core against the node-by-node plan and the oracle."""
    path, _ = pw.c2psa_attention(str(tmp_path), C=128, H=12, heads=2)
    assert "attention" in _kernels(path, 2)
    p, x, got = _run(path, 2, lo=-30.0, hi=30.0)
    _, _, nodes = _run(path, 2, lo=-30.0, hi=30.0, flags=ia.IVH_FLAG_NO_FUSE_ATTN)
    ref = O.run_plan(p, x, 2)[0].ravel()
    g = O.h2f(got[0])
    assert np.isfinite(g).all()
    mean_rel, max_rel, _, _ = O.rel_errors(g, O.h2f(nodes[0]))
    print(f"fused vs node by node: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3
    # against the oracle at the model bar (scripts/model_check.py:25,196-201): a one-ulp
    # difference of an fp16 score in the thousands moves exp(T - m) by tens of percent
    mean_rel, max_rel, _, scale_rel = O.rel_errors(g, O.h2f(ref))
    print(f"fused vs oracle: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} scale_rel={scale_rel:.2e}")
    assert (mean_rel < 2e-2 and max_rel < 5e-2) or scale_rel < 5e-3


@pytest.mark.parametrize("M,N,K,bdims", [
    (6400, 64, 64, None),            # scripts/kernel_check.py:25-31, the reference's gemm shapes
    (1600, 128, 128, None),
    (400, 256, 256, None),
    (1024, 1024, 1024, None),
    (4096, 512, 512, None),
    (48, 480, 64, [1, 64, 20, 24]),  # B of rank 4: N = numel(B) / K = 20*24
])
def test_gemm_op(tmp_path, M, N, K, bdims):
    """The plan's gemm op, C[M][N] = A[M][K] . B[K][N] (src/PlanModel.cpp:3935-3990), at
    batch 2: image 0 is kernel_check's own B (default_rng(0), A the init), checked against
    kernel_check's reference (a.f32 @ b.f32 -> fp16) with its contract; both images against
    the fp32 oracle and, where the fp16-accumulating restatement is cheap, the
    reference-rounding oracle."""
    path, b = pw.gemm_plan(str(tmp_path), M, N, K, b_dims=bdims)
    p = O.Plan.load(path)
    a = O.h2f(next(iter(p.inits.values()))).reshape(M, K)
    x1 = O.f2h(np.random.default_rng(7).random(K * N).astype(np.float32))
    x = np.concatenate([b.view(np.uint16).ravel(), x1])
    print(f"gemm M {M} N {N} K {K} B dims {bdims or [K, N]} batch 2", flush=True)
    m = ia.PlanModel(path, 0, 2)
    m.setInput(x, 2)
    m.run(2)
    got = m.readOutput(0, 2).reshape(2, M * N)
    m.close()
    kc = (a @ b.astype(np.float32).reshape(K, N)).astype(np.float16).astype(np.float32).ravel()
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), kc)
    print(f"   vs kernel_check reference mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < OP_MEAN and max_rel < OP_MAX
    ref = O.run_plan(p, x, 2)[0]
    for i in range(2):
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[i]), O.h2f(ref[i]))
        print(f"   image {i} vs f32 oracle mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
        assert mean_rel < F32_MEAN and max_rel < F32_MAX
    if M * N * K <= 30_000_000:
        refr = O.run_plan(p, x[:K * N], 1, mode=O.REF)[0]
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(refr[0]))
        print(f"   vs reference-rounding oracle mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
        assert mean_rel < OP_MEAN and max_rel < OP_MAX


def _upcat_plan(d, ca, cb, cout, H, W, reuse_a):
    """concat(resize_nn x2 (a), b) -> 1x1 conv, as a YOLO neck's Upsample / Concat / C2f cv1;
    a (ca channels at H x W) and b (cb channels at 2H x 2W) are internal channels-last
    tensors.  reuse_a: a is read again later (the neck's second concat), so it stays live."""
    def build(pb):
        x = pb.input("x", [1, cb, 2 * H, 2 * W])
        b = pb.conv(x, cb, 1, act=pw.ACT_RELU)
        a = pb.conv(b, ca, 3, 2, act=pw.ACT_SILU)
        y = pb.conv(pb.concat([pb.upsample(a, 2), b]), cout, 1, act=pw.ACT_SILU)
        if reuse_a:
            z = pb.conv(y, ca, 3, 2, act=pw.ACT_SILU)
            y = pb.conv(pb.concat([z, a]), cout, 1, act=pw.ACT_SILU)
        return y
    return _small_plan(d, build)


@pytest.mark.parametrize("ca,cb,cout,H,W,batch,reuse_a,fused", [
    (128, 64, 64, 10, 12, 3, True, True),     # YOLOv8n P3 neck shape class (192 -> 64)
    (256, 128, 128, 5, 6, 2, False, True),    # P4 neck class (384 -> 128), split-K
    (64, 40, 48, 7, 5, 5, False, True),       # odd maps, Cout not a tile multiple
    (64, 32, 32, 20, 20, 1, True, True),      # batch 1
    (40, 24, 32, 6, 6, 2, False, False),      # 40 upsampled channels: not a whole K step
])
def test_upsample_concat_fused(tmp_path, ca, cb, cout, H, W, batch, reuse_a, fused):
    """The 1x1 conv reads the upsampled channels from the resize's input: same bits as the
    materialised concat (the same implicit GEMM, the same values in the same LDS rows)."""
    path = _upcat_plan(tmp_path, ca, cb, cout, H, W, reuse_a)
    fl = ia.IVH_FLAG_NO_PW  # both runs on the implicit GEMM, which the fused conv always uses
    tags = _conv_tags(path, batch, fl)
    assert sum("upsample-concat" in t for t in tags) == (1 if fused else 0), tags
    assert ("resize_nn" in _kernels(path, batch, fl)) == (not fused)
    assert not any("upsample-concat" in t for t in _conv_tags(path, batch, fl | ia.IVH_FLAG_NO_FUSE_UPSAMPLE))
    _, _, got = _run(path, batch, lo=-1.0, flags=fl)
    _, _, ref = _run(path, batch, lo=-1.0, flags=fl | ia.IVH_FLAG_NO_FUSE_UPSAMPLE)
    assert np.array_equal(got[0], ref[0])
    _check_f32(path, batch, lo=-1.0, ref_mode=False, flags=fl)


def _head_plan(d, cin, H, W, widths=(51, 64, 64)):
    """A Pose head level: three branches whose first 3x3 convs read the same x (here the
    keypoint branch, 51 channels, comes first in node order as in the written plans), each
    followed by its own 3x3 conv and a 1x1 conv; the three branch outputs concatenated."""
    def build(pb):
        x = pb.conv(pb.input("x", [1, cin, H, W]), cin, 1, act=pw.ACT_SILU)
        firsts = [pb.conv(x, c, 3, 1, act=pw.ACT_SILU) for c in widths]
        seconds = [pb.conv(f, c, 3, 1, act=pw.ACT_SILU) for f, c in zip(firsts, widths)]
        return pb.concat([pb.conv(t, 16, 1, act=pw.ACT_NONE) for t in seconds])
    return _small_plan(d, build)


@pytest.mark.parametrize("cin,H,W,batch,widths", [
    (64, 20, 24, 3, (51, 64, 64)),     # P3 class: the resident-weight ping-pong kernel, 3 channel blocks
    (128, 12, 10, 4, (51, 64, 64)),    # P4 class
    (256, 6, 5, 2, (51, 64, 64)),      # P5 class
    (256, 20, 20, 64, (51, 64, 64)),   # P5 at batch 64: the wide-layer kernel, 2 x 128 channels
    (128, 16, 16, 8, (51, 64)),        # YOLO11n: box and keypoint branches only
])
def test_sibling_convs_merged(tmp_path, cin, H, W, batch, widths):
    """Sibling 3x3 convs on one input run as one conv over all their output channels, each
    branch reading its channel view of the merged output: oracle bar, and the merged run
    against the branches run one by one."""
    path = _head_plan(tmp_path, cin, H, W, widths)
    tags = _conv_tags(path, batch)
    # the merge writes 64 channels per branch (the keypoint branch's 51 padded with zero rows),
    # and the branches' second convs, reading consecutive 64-channel views of it, run as one
    # grouped launch on the ping-pong kernel (the keypoint group's weights zero-padded)
    n = len(widths)
    assert sum(f"siblings={n} cout={64 * n}" in t for t in tags) == 1, tags
    assert sum(f"groups={n} cout={sum(widths)}" in t for t in tags) == 1, tags
    assert not any("siblings" in t or "groups" in t for t in _conv_tags(path, batch, ia.IVH_FLAG_NO_FUSE_SIBLINGS))
    kinds = _kernels(path, batch)
    assert kinds.count("(fused)") == 2 * (n - 1), kinds
    got = _check_f32(path, batch, lo=-1.0, ref_mode=False)
    _, _, sep = _run(path, batch, lo=-1.0, flags=ia.IVH_FLAG_NO_FUSE_SIBLINGS)
    mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(got[0]), O.h2f(sep[0]))
    print(f"   merged vs separate mean_rel={mean_rel:.2e} max_rel={max_rel:.2e}")
    assert mean_rel < 1e-3 and max_rel < 5e-3
