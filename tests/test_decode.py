"""Pinning the pose decode / NMS restatement (oracle/decode.py) on the CPU.

The reference holds no golden detections for this path, so each rule of
src/Nms.cpp and src/Decoders.cpp is checked against a closed form or a brute-force
evaluation that a plausible slip (a non-strict threshold, an unstable order, a swapped
letterbox term, a dropped class split) would fail.
"""
import numpy as np
import pytest

from oracle import decode as D


def test_iou_closed_forms():
    assert D.iou((0, 0, 2, 2), (0, 0, 2, 2)) == pytest.approx(1.0)
    assert D.iou((0, 0, 1, 1), (2, 2, 1, 1)) == 0.0
    # 2x1 boxes overlapping in a 1x1 square: 1 / (2 + 2 - 1)
    assert D.iou((0, 0, 2, 1), (1, 0, 2, 1)) == pytest.approx(1 / 3)
    # a box inside another: area ratio
    assert D.iou((0, 0, 4, 4), (1, 1, 2, 2)) == pytest.approx(4 / 16)
    # degenerate union -> 0 (Nms.cpp:25)
    assert D.iou((0, 0, 0, 0), (0, 0, 0, 0)) == 0.0
    # negative extents count as zero area (Nms.cpp:21-22)
    assert D.iou((0, 0, -1, 2), (0, 0, 1, 1)) == 0.0


def test_iou_vectorised_matches_scalar():
    rng = np.random.default_rng(0)
    boxes = np.concatenate([rng.random((200, 2)) * 100, rng.random((200, 2)) * 30], 1).astype(np.float32)
    v = D.iou_one_to_many(boxes[0], boxes)
    for k in range(len(boxes)):
        assert v[k] == pytest.approx(D.iou(boxes[0], boxes[k]), abs=1e-7)


def test_nms_strict_threshold_and_order():
    # A suppresses B (IoU 0.8 > 0.7); C overlaps A at 0.5 and survives
    a, b, c = (0, 0, 10, 10), (0, 0, 10, 8), (0, 0, 10, 5)
    assert D.iou(a, b) == pytest.approx(0.8)
    assert D.iou(a, c) == pytest.approx(0.5)
    keep = D.nms(np.array([b, c, a], np.float32), np.array([0.8, 0.7, 0.9], np.float32), 0.7)
    assert keep == [2, 1]
    # IoU exactly at the threshold does not suppress (">" in Nms.cpp:49)
    keep = D.nms(np.array([a, b], np.float32), np.array([0.9, 0.8], np.float32), 0.8)
    assert keep == [0, 1]
    # equal scores: stable order, the lower index wins
    keep = D.nms(np.array([b, a], np.float32), np.array([0.5, 0.5], np.float32), 0.7)
    assert keep == [0]


def test_nms_matches_brute_force():
    rng = np.random.default_rng(1)
    n = 300
    xy = rng.random((n, 2)) * 60
    wh = 5 + rng.random((n, 2)) * 20
    boxes = np.concatenate([xy, wh], 1).astype(np.float32)
    scores = rng.random(n).astype(np.float32)
    # naive O(n^2) greedy NMS with the scalar iou
    order = sorted(range(n), key=lambda i: -scores[i])
    alive, ref = set(order), []
    for i in order:
        if i not in alive:
            continue
        ref.append(i)
        for j in order:
            if j in alive and j != i and order.index(j) > order.index(i) and D.iou(boxes[i], boxes[j]) > 0.45:
                alive.discard(j)
    assert D.nms(boxes, scores, 0.45) == ref


def test_nms_per_class_and_max_det():
    dets = [D.Detection(box=(0, 0, 10, 10), score=0.9, class_id=1),
            D.Detection(box=(0, 0, 10, 10), score=0.8, class_id=0),   # other class: kept
            D.Detection(box=(0, 0, 10, 9), score=0.7, class_id=1),    # suppressed by the first
            D.Detection(box=(50, 50, 5, 5), score=0.95, class_id=0)]
    out = D.nms_per_class(dets, 0.5, 300)
    assert [d.score for d in out] == [0.95, 0.9, 0.8]
    assert [d.score for d in D.nms_per_class(dets, 0.5, 2)] == [0.95, 0.9]


def test_pose_decode_threshold_and_letterbox():
    nk = 17
    raw = np.zeros((5 + 3 * nk, 3), np.float32)
    raw[:4, 0] = [110, 120, 40, 20]          # cx cy w h
    raw[4] = [0.25, 0.2499, 0.6]             # score == conf is kept, below is dropped
    raw[5, 0], raw[6, 0] = 30, 40            # keypoint 0
    raw[:4, 2] = [500, 500, 10, 10]
    lb = D.Letterbox(scale=0.5, pad_left=10, pad_top=20)
    dets = D.pose_decode(raw, conf=0.25, iou_thr=0.7, lb=lb)
    assert [d.anchor for d in dets] == [2, 0]
    d0 = dets[1]
    # Preprocess.hpp:30-35: x = (cx - pad_left)/scale - w/scale/2, w = w/scale
    assert d0.box == pytest.approx((160.0, 180.0, 80.0, 40.0))
    assert d0.keypoints[0] == pytest.approx((40.0, 40.0))
    assert d0.keypoints.shape == (nk, 2)
