"""Whole-model parity on the GPU through the C ABI (scripts/model_check.py protocol):
raw head tensors vs the CPU oracle run on the same plan and inputs; pass bar
mean_rel < 2e-2 and max_rel < 5e-2, or scale_rel < 5e-3 (model_check.py:25,196-201).
Two different inputs, the second compared (README.md:153-155), batch consistency,
graph replay vs eager launches."""
import numpy as np
import pytest

import infvino_amd as ia
from infvino_amd import planwriter as pw
from oracle import oracle as O

pytestmark = pytest.mark.gpu

M_MEAN, M_MAX, M_SCALE = 2e-2, 5e-2, 5e-3


def _inputs(p, batch, seed):
    rng = np.random.default_rng(seed)
    return O.f2h(rng.random(p.numel(p.input_name) * batch).astype(np.float32))


def _model_ok(got, ref, label):
    mean_rel, max_rel, max_abs, scale_rel = O.rel_errors(O.h2f(got), O.h2f(ref))
    print(f"{label}: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} max_abs={max_abs:.2e} scale_rel={scale_rel:.2e}")
    return (mean_rel < M_MEAN and max_rel < M_MAX) or scale_rel < M_SCALE


# Pose heads [56, 8400] (src/Decoders.cpp:127-176): rows 0-3 box (cx, cy, w, h in pixels),
# row 4 person score, then 17 keypoints x (5 + 3k), y (6 + 3k), visibility (7 + 3k).  The
# global max|ref| of the head is a pixel coordinate (~640), so one relative bar over the
# whole tensor would let the [0, 1] rows drift by several units; each row group is held to
# its own max|ref|: the coordinate rows to the model bar, the score and visibility rows
# (sigmoid outputs) to the op-level bar of the fp32-accumulating kernels.
OP_MEAN, OP_MAX = 2e-3, 1e-2


def _pose_groups(nk=17):
    kx, ky, kv = 5 + 3 * np.arange(nk), 6 + 3 * np.arange(nk), 7 + 3 * np.arange(nk)
    return {"box": (np.arange(4), M_MEAN, M_MAX), "score": (np.array([4]), OP_MEAN, OP_MAX),
            "kpt_xy": (np.sort(np.concatenate([kx, ky])), M_MEAN, M_MAX), "kpt_vis": (kv, OP_MEAN, OP_MAX)}


def _pose_heads_ok(got, ref, batch, label):
    g = O.h2f(got).reshape(batch, 56, -1)
    r = O.h2f(ref).reshape(batch, 56, -1)
    ok = True
    for name, (rows, bar_mean, bar_max) in _pose_groups().items():
        mean_rel, max_rel, max_abs, _ = O.rel_errors(g[:, rows], r[:, rows])
        good = mean_rel < bar_mean and max_rel < bar_max
        print(f"{label} {name}: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} max_abs={max_abs:.2e} "
              f"(bar {bar_mean:g}/{bar_max:g}) {'ok' if good else 'FAIL'}")
        ok &= good
    return ok


@pytest.mark.parametrize("name,imgsz,batch", [("mobilenetv3-small", 224, 3), ("yolov8n-pose", 640, 2),
                                              ("yolo11n-pose", 640, 1), ("yolov8n-pose", 320, 3)])
def test_model_parity(tmp_path, name, imgsz, batch):
    path, _ = pw.MODELS[name](str(tmp_path), seed=0, imgsz=imgsz)
    p = O.Plan.load(path)
    m = ia.PlanModel(path, 0, batch)
    # frame 1: input A, frame 2: input B (staleness protocol); compare frame 2
    m.setInput(_inputs(p, batch, 1), batch)
    m.run(batch)
    xb = _inputs(p, batch, 2)
    m.setInput(xb, batch)
    m.run(batch)
    got = m.readOutput(0, batch)
    ref = O.run_plan(p, xb, batch)[0].ravel()
    if name.endswith("-pose"):
        assert _pose_heads_ok(got, ref, batch, f"{name}@{imgsz} b{batch}")
    else:
        assert _model_ok(got, ref, f"{name}@{imgsz} b{batch}")
    m.close()


@pytest.mark.parametrize("name,imgsz,batch,check", [
    ("yolov8n-pose", 640, 64, (0, 31, 63)),       # the timed configuration of the bench
    ("yolo11n-pose", 640, 64, (0, 40, 63)),
    ("mobilenetv3-small", 224, 256, (0, 128, 255)),
])
def test_timed_batch_plans(tmp_path, name, imgsz, batch, check):
    """The plans the bench times, at their batch and flags (graph replay, asynchronous runs),
    with the two-input protocol: frame 2's images `check` against the oracle (pose heads per
    row group); every image of frame 2 again, bit for bit, from a run with the batch rotated
    by 17 positions (kernels and tiles do not depend on where an image sits in the batch);
    and the checked images run alone at batch 1 on the same model, where the planner picks
    other kernels (split-K, no persistent or pipelined kernels), within fp32 summation noise."""
    path, _ = pw.MODELS[name](str(tmp_path), seed=0, imgsz=imgsz)
    p = O.Plan.load(path)
    n_in, per = p.numel(p.input_name), p.numel(p.outputs[0])
    print(f"{name}@{imgsz} batch {batch}: images {check}", flush=True)
    m = ia.PlanModel(path, 0, batch, ia.IVH_FLAG_ASYNC)
    m.setInput(_inputs(p, batch, 1), batch)
    m.run(batch)
    xb = _inputs(p, batch, 2)
    m.setInput(xb, batch)
    m.run(batch)
    got = m.readOutput(0, batch).reshape(batch, per)
    sel = np.concatenate([xb[i * n_in:(i + 1) * n_in] for i in check])
    ref = O.run_plan(p, sel, len(check))[0].reshape(len(check), per)
    for j, i in enumerate(check):
        label = f"{name}@{imgsz} b{batch} image {i}"
        if name.endswith("-pose"):
            assert _pose_heads_ok(got[i], ref[j], 1, label)
        else:
            assert _model_ok(got[i], ref[j], label)
    shift = 17
    m.setInput(np.roll(xb.reshape(batch, n_in), shift, axis=0).ravel(), batch)
    m.run(batch)
    rolled = np.roll(m.readOutput(0, batch).reshape(batch, per), -shift, axis=0)
    assert np.array_equal(rolled, got), "an image's result depends on its position in the batch"
    for i in check:
        m.setInput(xb[i * n_in:(i + 1) * n_in], 1)
        m.run(1)
        one = m.readOutput(0, 1)
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(one), O.h2f(got[i]))
        print(f"  image {i} alone vs in the batch: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} "
              f"bit-identical {np.array_equal(one, got[i])}")
        assert mean_rel < 1e-3 and max_rel < 1e-2
    m.close()


def test_batch_and_replay_consistency(tmp_path):
    """Without split-K, image i of a batch equals the same image run alone (bit-exact); with
    split-K (batch-dependent K partitioning) it agrees within fp32 summation noise and is
    bit-exact run to run.  Graph replay equals eager launches; a fresh model on input B equals
    a model that ran A first."""
    path, _ = pw.yolov8n_pose(str(tmp_path), seed=0, imgsz=256)
    p = O.Plan.load(path)
    x = _inputs(p, 3, 5)
    n = p.numel(p.input_name)

    def runs(flags):
        m = ia.PlanModel(path, 0, 3, flags)
        m.setInput(x, 3)
        m.run(3)
        full = m.readOutput(0, 3)
        per = full.size // 3
        singles = []
        for i in range(3):
            m.setInput(x[i * n:(i + 1) * n], 1)
            m.run(1)
            singles.append(m.readOutput(0, 1))
        m.setInput(x[:n], 1)
        m.run(1)
        again = m.readOutput(0, 1)
        m.close()
        return full, per, singles, again

    full, per, singles, again = runs(ia.IVH_FLAG_NO_SPLITK)
    for i in range(3):
        assert np.array_equal(singles[i], full[i * per:(i + 1) * per]), f"image {i}"
    full2, per, singles2, again2 = runs(0)
    assert np.array_equal(again2, singles2[0]), "split-K must be deterministic run to run"
    for i in range(3):
        mean_rel, max_rel, _, _ = O.rel_errors(O.h2f(singles2[i]), O.h2f(full2[i * per:(i + 1) * per]))
        assert mean_rel < 1e-3 and max_rel < 1e-2, (i, mean_rel, max_rel)
    e = ia.PlanModel(path, 0, 3, ia.IVH_FLAG_NO_GRAPH)
    e.setInput(x, 3)
    e.run(3)
    assert np.array_equal(e.readOutput(0, 3), full2)
    e.close()


def test_backend_f32_boundary(tmp_path):
    """HipBackend.infer: f32 in (reference truncation to fp16), f32 Tensors out."""
    path, _ = pw.mobilenetv3_small(str(tmp_path), seed=0)
    be = ia.HipBackend(path, max_batch=2)
    assert be.inputDims() == [1, 3, 224, 224]
    assert be.outputShapes() == [[1, 1000]]
    rng = np.random.default_rng(7)
    xf = rng.random(2 * 3 * 224 * 224).astype(np.float32)
    outs = be.infer(xf)
    assert outs[0].shape == [2, 1000]
    p = O.Plan.load(path)
    ref = O.h2f(O.run_plan(p, O.f2h_trunc(xf), 2)[0].ravel())
    assert _model_ok(O.f2h(outs[0].data.ravel()), O.f2h(ref), "backend mbv3 b2")
    with pytest.raises(RuntimeError, match="numel mismatch"):
        be.infer(xf[:100])


def test_cpp_backend_dropin(tmp_path):
    """The C++ HipBackend / HipPlanModel (include/infvino_hip/) used as ClBackend is used:
    f32 in, f32 Tensors out, batch 2, error messages; outputs vs the oracle."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "cpp", "_build", "test_backend")
    if not os.path.exists(exe):
        pytest.skip("tests/cpp/_build/test_backend not built (__graft_entry__.build())")
    path, _ = pw.mobilenetv3_small(str(tmp_path / "m"), seed=0)
    bad = tmp_path / "bad.plan"
    bad.write_text("input x 1 4\ntensor y 1 4\nnode ew_unary x y op=1 n=4\n")
    out = tmp_path / "out.bin"
    r = subprocess.run([exe, path, str(out), str(bad)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "test_backend OK" in r.stdout
    got = np.fromfile(out, np.float32)
    p = O.Plan.load(path)
    n = p.numel(p.input_name)
    i = np.arange(2 * n, dtype=np.uint64)
    xf = ((i * np.uint64(2654435761)) % np.uint64(1000)).astype(np.float32) / np.float32(1000.0)
    ref = O.h2f(O.run_plan(p, O.f2h_trunc(xf), 2)[0].ravel())
    assert _model_ok(O.f2h(got), O.f2h(ref), "C++ HipBackend mbv3 b2")


# ----------------------------------------------------------------- decode + NMS parity
# Decoded detections after the reference's PoseDecoder + NMS (restated in oracle/decode.py),
# HIP raw heads vs oracle raw heads, conf 0.25 / IoU 0.7.  Random-init heads put many
# anchors near a decision: an anchor whose fate differs between the two is accepted only
# when a near-tie explains it -- its score within EPS_S of conf or of the lowest kept score
# when max_det cut the kept set, an overlap with a kept box
# within EPS_I of the IoU threshold, or an overlapping kept box with a score within EPS_S --
# or when it overlaps such an anchor (the flip then cascades).  Matched detections must
# agree to BOX_TOL / KPT_TOL pixels (network input coordinates).
EPS_S, EPS_I, BOX_TOL, KPT_TOL = 2e-3, 2e-2, 2.0, 2.0


def _explained(dh, do, conf, thr, max_det):
    from oracle import decode as D
    A = {d.anchor: d for d in dh}
    B = {d.anchor: d for d in do}
    unmatched = {a: (A.get(a) or B.get(a)) for a in set(A) ^ set(B)}
    kept = list(A.values()) + list(B.values())
    kbox = np.array([d.box for d in kept], np.float32).reshape(-1, 4)
    ksc = np.array([d.score for d in kept], np.float32)
    # a full kept set ends at a rank cutoff: its lowest score is a decision boundary too
    cuts = [min(d.score for d in ds) for ds in (dh, do) if len(ds) >= max_det]
    seeds = set()
    for a, d in unmatched.items():
        if abs(d.score - conf) <= EPS_S or any(abs(d.score - c) <= EPS_S for c in cuts):
            seeds.add(a)
            continue
        io = D.iou_one_to_many(d.box, kbox)
        other = np.array([k.anchor != a for k in kept])
        if np.any(other & (np.abs(io - thr) <= EPS_I)) or np.any(other & (io > thr - EPS_I) & (np.abs(ksc - d.score) <= EPS_S)):
            seeds.add(a)
    done = set(seeds)
    changed = True
    while changed:
        changed = False
        for a, d in unmatched.items():
            if a in done:
                continue
            if any(D.iou(d.box, unmatched[b].box) > thr - EPS_I for b in done):
                done.add(a)
                changed = True
    return len(A.keys() & B.keys()), unmatched, done


@pytest.mark.parametrize("name,imgsz,batch", [("yolov8n-pose", 640, 2), ("yolo11n-pose", 640, 1)])
def test_pose_decode_parity(tmp_path, name, imgsz, batch):
    from oracle import decode as D
    path, _ = pw.MODELS[name](str(tmp_path), seed=0, imgsz=imgsz)
    p = O.Plan.load(path)
    x = _inputs(p, batch, 3)
    m = ia.PlanModel(path, 0, batch)
    m.setInput(x, batch)
    m.run(batch)
    got = m.readOutputF32(0, batch).reshape(batch, 56, -1)
    m.close()
    ref = O.h2f(O.run_plan(p, x, batch)[0]).reshape(batch, 56, -1)
    conf, thr = 0.25, 0.7
    # the reference's max_det (ModelInfo.hpp:34) and the whole kept set
    for b, max_det in [(b, md) for b in range(batch) for md in (300, 10 ** 6)]:
        dh = D.pose_decode(got[b], conf=conf, iou_thr=thr, max_det=max_det)
        do = D.pose_decode(ref[b], conf=conf, iou_thr=thr, max_det=max_det)
        nmatch, unmatched, explained = _explained(dh, do, conf, thr, max_det)
        A = {d.anchor: d for d in dh}
        B = {d.anchor: d for d in do}
        box_err = max([np.max(np.abs(np.subtract(A[a].box, B[a].box))) for a in A.keys() & B.keys()] or [0.0])
        kpt_err = max([np.max(np.abs(A[a].keypoints - B[a].keypoints)) for a in A.keys() & B.keys()] or [0.0])
        print(f"{name} image {b} max_det {max_det}: hip {len(dh)} oracle {len(do)} matched {nmatch} unmatched {len(unmatched)} "
              f"explained {len(explained)} box_err {box_err:.3f}px kpt_err {kpt_err:.3f}px")
        assert len(do) > 0
        assert set(unmatched) == explained, f"unexplained: {sorted(set(unmatched) - explained)[:10]}"
        assert nmatch >= 0.9 * max(len(dh), len(do))
        assert box_err <= BOX_TOL and kpt_err <= KPT_TOL


# ----------------------------------------------------------------- boundary conversions

def _write_plan(d, text):
    path = d / "io.plan"
    path.write_text(text)
    return str(path)


def test_set_input_f32_truncation_bit_exact(tmp_path):
    """ivh_set_input_f32 converts on the device with the reference's truncating f32 -> f16
    (include/infvino/Half.hpp:14-24, ClBackend.cpp:42-44): the graph input read back through
    ivh_read_tensor_f16 equals the known-answer vectors written by the reference's own
    src/Half.cpp (tests/golden/half_trunc.npz), bit for bit, in every image of a batch."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "half_trunc.npz"))
    n = g["x"].size
    path = _write_plan(tmp_path, f"input x 1 {n}\ntensor y 1 {n}\nnode ew_unary x y op=2 n={n}\noutput y\n")
    m = ia.PlanModel(path, 0, 2)
    x2 = np.concatenate([g["x"], g["x"][::-1]])
    m.setInputF32(x2, 2)
    back = m.readTensor("x", 2)
    m.close()
    assert np.array_equal(back[:n], g["h"])
    assert np.array_equal(back[n:], g["h"][::-1])


def test_read_output_f32_exact_every_half(tmp_path):
    """ivh_read_output_f32 (ClBackend.cpp:53-61's readOutput + f16_to_f32) is the exact
    f16 -> f32 conversion for all 65536 half patterns, NaN payloads included; the f16
    readback returns the bits that the (bit-exact) slice wrote."""
    path = _write_plan(tmp_path, "input x 1 4 16384\ntensor y 1 4 16384\n"
                                 "node slice_axis x y outer=1 axdim=4 inner=16384 start=0 len=4\noutput y\n")
    m = ia.PlanModel(path, 0, 1)
    h = np.arange(65536, dtype=np.uint16)
    m.setInput(h, 1)
    m.run(1)
    f16 = m.readOutput(0, 1)
    f32 = m.readOutputF32(0, 1)
    m.close()
    assert np.array_equal(f16, h)
    assert np.array_equal(f32.view(np.uint32), O.h2f(h).view(np.uint32))
    nan = ((h >> 10) & 0x1F) == 31
    nan &= (h & 0x3FF) != 0
    assert np.isnan(f32[nan]).all()
    ref = h[~nan].view(np.float16).astype(np.float32)
    assert np.array_equal(f32[~nan].view(np.uint32), ref.view(np.uint32))


def test_profiling_mode_accumulates(tmp_path):
    """IVH_FLAG_PROFILE (ClBackend / PlanModel profiling=true): every run adds each node's
    device time; outputs equal those of graph replay; clearProfile resets the totals."""
    import ctypes as C
    path, _ = pw.yolov8n_pose(str(tmp_path), seed=0, imgsz=256)
    p = O.Plan.load(path)
    x = _inputs(p, 2, 4)
    ref = ia.PlanModel(path, 0, 2)
    ref.setInput(x, 2)
    ref.run(2)
    want = ref.readOutput(0, 2)
    ref.close()
    m = ia.PlanModel(path, 0, 2, ia.IVH_FLAG_PROFILE)
    m.setInput(x, 2)
    for _ in range(3):
        m.run(2)
    assert np.array_equal(m.readOutput(0, 2), want)
    n = m.nodeCount()
    ms, calls = (C.c_double * n)(), (C.c_int * n)()
    assert ia.lib().ivh_node_times(m._h, ms, calls, n) == 0
    launching = [i for i in range(n) if m.nodeInfo(i)["kernel"] not in ("(view)", "(fused)")]
    assert all(calls[i] == 3 and ms[i] > 0 for i in launching)
    assert all(calls[i] == 0 for i in range(n) if i not in launching)
    assert ia.lib().ivh_clear_profile(m._h) == 0
    assert ia.lib().ivh_node_times(m._h, ms, calls, n) == 0
    assert sum(calls) == 0
    m.close()
