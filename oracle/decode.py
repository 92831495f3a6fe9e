"""CPU restatement of the reference's pose post-processing -- TEST INFRASTRUCTURE ONLY.

The product path never decodes: the reference's own PoseDecoder / nms run unchanged on the
f32 host tensors the HIP backend returns.  This module restates them so the tests can check
that the HIP path's raw head tensors lead to the same detections as the oracle's after
decode + NMS (the parity protocol for YOLOv8n-pose / YOLO11n-pose).

Restated from the reference (file:line):
  iou            src/Nms.cpp:10-26      (inter / union, 0 when union <= 1e-9)
  nms            src/Nms.cpp:28-55      (stable sort by score desc; suppress IoU > thr)
  nms_per_class  src/Decoders.cpp:33-63 (per class id, then sort by score desc, max_det)
  pose_decode    src/Decoders.cpp:127-176 (score = channel 4, skip score < conf; box and
                 keypoints mapped back through the letterbox)
  Letterbox      include/infvino/Preprocess.hpp:25-35 (toImage / rectToImage)
Every detection also carries the anchor index it came from, so two decodes can be matched
anchor by anchor.  The reference's final sort is std::sort (unspecified order for equal
scores); here it is stable (anchor order among equal scores).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Letterbox:
    """Preprocess.hpp:18-36: scale and padding of the letterboxed network input."""
    scale: float = 1.0
    pad_left: float = 0.0
    pad_top: float = 0.0

    def to_image(self, x, y):
        return (x - np.float32(self.pad_left)) / np.float32(self.scale), \
               (y - np.float32(self.pad_top)) / np.float32(self.scale)

    def rect_to_image(self, cx, cy, w, h):
        s = np.float32(self.scale)
        x = (cx - np.float32(self.pad_left)) / s
        y = (cy - np.float32(self.pad_top)) / s
        return x - w / s / np.float32(2.0), y - h / s / np.float32(2.0), w / s, h / s


@dataclass
class Detection:
    box: tuple            # x, y, width, height (image coordinates)
    score: float
    class_id: int = 0
    keypoints: np.ndarray = field(default_factory=lambda: np.zeros((0, 2), np.float32))
    anchor: int = -1      # index of the anchor the detection came from


def iou(a, b) -> float:
    """Nms.cpp:10-26 in float32."""
    f = np.float32
    x1, y1 = max(f(a[0]), f(b[0])), max(f(a[1]), f(b[1]))
    x2 = min(f(a[0]) + f(a[2]), f(b[0]) + f(b[2]))
    y2 = min(f(a[1]) + f(a[3]), f(b[1]) + f(b[3]))
    inter = max(f(0), x2 - x1) * max(f(0), y2 - y1)
    area_a = max(f(0), f(a[2])) * max(f(0), f(a[3]))
    area_b = max(f(0), f(b[2])) * max(f(0), f(b[3]))
    uni = area_a + area_b - inter
    return float(inter / uni) if uni > f(1e-9) else 0.0


def iou_one_to_many(box, boxes: np.ndarray) -> np.ndarray:
    """iou(box, boxes[k]) for every k, the same float32 arithmetic vectorised."""
    f = np.float32
    b = boxes.astype(np.float32)
    x1 = np.maximum(f(box[0]), b[:, 0])
    y1 = np.maximum(f(box[1]), b[:, 1])
    x2 = np.minimum(f(box[0]) + f(box[2]), b[:, 0] + b[:, 2])
    y2 = np.minimum(f(box[1]) + f(box[3]), b[:, 1] + b[:, 3])
    inter = np.maximum(f(0), x2 - x1) * np.maximum(f(0), y2 - y1)
    area_a = max(f(0), f(box[2])) * max(f(0), f(box[3]))
    area_b = np.maximum(f(0), b[:, 2]) * np.maximum(f(0), b[:, 3])
    uni = area_a + area_b - inter
    out = np.zeros(len(b), np.float32)
    ok = uni > f(1e-9)
    out[ok] = inter[ok] / uni[ok]
    return out


def nms(boxes: np.ndarray, scores: np.ndarray, iou_threshold: float) -> list[int]:
    """Nms.cpp:28-55: greedy NMS in stable descending-score order; returns kept indices."""
    order = sorted(range(len(scores)), key=lambda i: -float(scores[i]))  # Python sort is stable
    removed = np.zeros(len(scores), bool)
    keep = []
    boxes = np.asarray(boxes, np.float32).reshape(-1, 4)
    order = np.asarray(order, np.int64)
    for pos, idx in enumerate(order):
        if removed[idx]:
            continue
        keep.append(int(idx))
        rest = order[pos + 1:]
        rest = rest[~removed[rest]]
        if len(rest):
            over = iou_one_to_many(boxes[idx], boxes[rest]) > np.float32(iou_threshold)
            removed[rest[over]] = True
    return keep


def nms_per_class(dets: list[Detection], iou_thr: float, max_det: int) -> list[Detection]:
    """Decoders.cpp:33-63."""
    if not dets:
        return dets
    out = []
    for cid in sorted({d.class_id for d in dets}):
        idx = [i for i, d in enumerate(dets) if d.class_id == cid]
        boxes = np.array([dets[i].box for i in idx], np.float32)
        scores = np.array([dets[i].score for i in idx], np.float32)
        for k in nms(boxes, scores, iou_thr):
            out.append(dets[idx[k]])
    out.sort(key=lambda d: -d.score)
    return out[:max_det]


def pose_decode(raw: np.ndarray, conf: float = 0.25, iou_thr: float = 0.7, max_det: int = 300,
                nkpt: int = 17, kdims: int = 3, lb: Letterbox | None = None) -> list[Detection]:
    """Decoders.cpp:127-176 for one image: raw is [C, N] (channel-major, C = 5 + nkpt*kdims)
    float32; channels 0-3 cx cy w h, 4 the score, then the keypoints (x, y, visibility)."""
    lb = lb or Letterbox()
    raw = np.asarray(raw, np.float32)
    assert raw.ndim == 2 and raw.shape[0] == 5 + nkpt * kdims, raw.shape
    dets = []
    for a in np.nonzero(~(raw[4] < np.float32(conf)))[0]:
        x, y, w, h = lb.rect_to_image(raw[0, a], raw[1, a], raw[2, a], raw[3, a])
        kx, ky = lb.to_image(raw[5 + np.arange(nkpt) * kdims, a], raw[6 + np.arange(nkpt) * kdims, a])
        dets.append(Detection(box=(float(x), float(y), float(w), float(h)), score=float(raw[4, a]),
                              class_id=0, keypoints=np.stack([kx, ky], 1).astype(np.float32), anchor=int(a)))
    return nms_per_class(dets, iou_thr, max_det)
