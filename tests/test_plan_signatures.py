"""The plan writer against the reference's own record of its lowered plans.

config/tuning.json (kept as tests/golden/tuning_signatures.txt) holds one entry per node
signature of the plans the reference lowered with onnx2plan from real ultralytics 8.4 /
torchvision exports.  Every node of the plans infvino_amd/planwriter.py writes for the same
models must have one of those signatures (oracle/signatures.py restates how the reference
computes them, after its default graph rewrites), which pins node types, shapes, attribute
values and broadcast specs that the FLOP and census checks cannot see."""
import os

import pytest

from infvino_amd import planwriter as pw
from oracle import oracle as O
from oracle import signatures as S

HERE = os.path.dirname(os.path.abspath(__file__))
MODELS = [("yolov8n-pose", 640), ("yolo11n-pose", 640), ("mobilenetv3-small", 224)]


@pytest.fixture(scope="module")
def reference_sigs():
    with open(os.path.join(HERE, "golden", "tuning_signatures.txt")) as f:
        return {line.strip() for line in f if line.strip()}


def _sigs(path):
    return S.plan_signatures(O.Plan.load(path))


@pytest.mark.parametrize("name,imgsz", MODELS)
def test_every_node_signature_is_the_reference_s(tmp_path, reference_sigs, name, imgsz):
    path, _ = pw.MODELS[name](str(tmp_path), seed=0, imgsz=imgsz)
    sigs = _sigs(path)
    missing = [(i, op, s) for i, op, s in sigs if s not in reference_sigs]
    assert not missing, missing
    assert len(sigs) > 60


def test_named_reference_nodes_present(tmp_path, reference_sigs):
    """Nodes whose shapes a plausible lowering slip would change: YOLO11's C2PSA split of q / k
    / v, its attention products and softmax, the scale on q^T; the pose decode's concats,
    slices and DFL; the fused C2f concat -> conv1x1 (conv1x1_cat4)."""
    have = set()
    for name, imgsz in MODELS:
        have |= {s for _, _, s in _sigs(pw.MODELS[name](str(tmp_path / name), seed=0, imgsz=imgsz)[0])}
    want = ["slice_axis|2,128,400,0,32_act0_f16", "slice_axis|2,128,400,32,32_act0_f16",
            "slice_axis|2,128,400,64,64_act0_f16", "bmm|1,2,400,32,400_act0_f16", "bmm|1,2,64,400,400_act0_f16",
            "softmax_axis|800,400,1_act0_f16", "ew_binary|25600,2,1_act0_f16", "permute_0213|2,32,400,1_act0_f16",
            "permute_0213|2,400,400,1_act0_f16", "concat4|1,8400,4,1,51,0_act0_f16",
            "concat4|64,1,6400,1600,400,0_act0_f16", "concat4|1,1,6400,1600,400,0_act0_f16",
            "concat4|51,1,6400,1600,400,0_act0_f16", "concat4|17,8400,2,1,0,0_act0_f16",
            "slice_axis|1,4,8400,0,2_act0_f16", "slice_axis|1,4,8400,2,2_act0_f16",
            "softmax_axis|1,16,33600_act0_f16", "permute_0213|4,16,8400,0_act0_f16"]
    for s in want:
        assert s in reference_sigs, s
        assert s in have, s
    assert any(s.startswith("conv1x1_cat4|") for s in have)


@pytest.mark.parametrize("what", ["head", "attention"])
def test_older_export_forms_are_not_the_reference_s(tmp_path, reference_sigs, what):
    """The older head form (per-scale box + class concat, copy_c splits, nested output concat)
    and the scale applied to the scores after the product are lowerings the reference's plans
    do not contain: the check tells them apart."""
    pb = pw.PlanBuilder(str(tmp_path), seed=0)
    if what == "head":
        x = pb.input("images", [1, 3, 256, 256])
        f3 = pb.conv(pb.conv(pb.conv(x, 16, 3, 2), 32, 3, 2), 64, 3, 2)
        f4 = pb.conv(f3, 128, 3, 2)
        f5 = pb.conv(f4, 256, 3, 2)
        pb.output(pw._pose_head(pb, [f3, f4, f5], legacy=True))
        path = pb.write()
        path_new = None
    else:
        path = pw.c2psa_attention(str(tmp_path / "old"), C=128, H=20, heads=2, legacy=True)[0]
        path_new = pw.c2psa_attention(str(tmp_path / "new"), C=128, H=20, heads=2)[0]
    bad = [s for _, op, s in _sigs(path) if s not in reference_sigs and op in ("concat4", "copy_c", "ew_binary")]
    assert bad
    if path_new:
        assert "ew_binary|320000,2,1_act0_f16" in bad
        assert all(s in reference_sigs for _, op, s in _sigs(path_new) if op in ("ew_binary", "bmm", "softmax_axis"))


def test_signature_format_closed_forms():
    """OpSignature::str's formats (src/Tuning.cpp:85-115) on hand-written nodes."""
    assert S._str("conv3x3", 1, W=80, H=80, s=1, p=1, Cin=64, Cout=64) == "conv3x3|W80H80s1p1_Cin64_Cout64_act1_f16"
    assert S._str("conv1x1", 1, Cout=128, N=6400, Cin=64) == "conv1x1|Cout128_N6400_Cin64_act1_f16"
    assert S._str("depthwise", 3, W=56, H=56, s=2, p=1, Cin=16, Cout=16, K=3, G=16) == \
        "depthwise|W56H56s2p1_Cin16_Cout16_K3_G16_act3_f16"
    assert S._str("gap", Cin=96, N=196) == "gap|C96_HW196_act0_f16"
    assert S._str("gemm", M=6400, N=64, K=64) == "gemm|M6400N64K64_act0_f16"
    assert S._str("maxpool", params=[128, 20, 20, 20, 20, 5, 1, 2]) == "maxpool|128,20,20,20,20,5,1,2_act0_f16"
