"""Writes tests/golden/tuning_signatures.txt: the keys of the reference's config/tuning.json,
one per line.  Each key is the OpSignature::str() of one node of the plans the reference
lowered from real exports (src/Tuning.cpp:85-115; small ops via smallSig,
src/PlanModel.cpp:2595-2679), so the list is the reference's own record of the node types,
shapes and attributes its YOLOv8n-pose / YOLO11n-pose / MobileNetV3-small plans contain.
The fixture keeps that data where the reference tree is absent; only the keys are kept
(the tuned kernel options and timings of the Intel GPU are not)."""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/config/tuning.json"


def main():
    with open(SRC) as f:
        entries = json.load(f)["entries"]
    keys = sorted(entries)
    with open(os.path.join(HERE, "tuning_signatures.txt"), "w") as f:
        f.write("\n".join(keys) + "\n")
    print("wrote", len(keys), "signatures")


if __name__ == "__main__":
    main()
