"""Benchmark: YOLOv8n-pose 3x640x640 fp16 on one MI355X through the HIP backend.

One step = one pass of the plan over one batch of 64 synthetic images already resident in
HBM (the captured HIP graph of the whole plan).  Prints ONE JSON line on stdout; a per-node
table goes to stderr.

  value          images/s at batch 64 (whole job, one GPU)
  latency_b1_ms  wall time of one synchronous batch-1 inference (graph replay)
  roofline       dominant kernel (largest device time per batch-64 step): algorithmic FLOPs
                 (or bytes) per launch / its mean launch time, HIP events on the model stream
  conv_mfma_frac all conv FLOPs of a step / conv device time / dense fp16 MFMA peak
  roofline_step  the whole step against its roofline: sum over nodes of the node's ideal time
                 (max of algorithmic FLOPs / MFMA peak and bytes / HBM peak) over the sum of
                 the nodes' measured times -- the time-weighted mean of the per-node fractions
  config1        the single pointwise conv (64->128 at 80x80, SiLU) at batch 1 and 64, with
                 its roofline (HBM bound)
  conv_sweep     the conv operator sweep (stem, strided / stride-1 3x3, depthwise) at batch
                 64 and batch 1, and the depthwise layers at batch 256: per layer time,
                 TFLOP/s, GB/s and fraction of its binding roof (MFMA, HBM, or for depthwise
                 the fp32 VALU)
  attention      the C2PSA attention block at 256 channels, 4 heads, head_dim 64, 400 tokens
                 (q^T k, softmax, v attn^T) at batch 64 and 1, with its roofline
  other_models   YOLOv8n-pose 640 (batch 16 / 64), MobileNetV3-small 224 (batch 1 / 32 / 256)
                 and YOLO11n-pose 640 (batch 1 / 64): images/s of graph replays and batch-1
                 latency
  mfma_roof_probe  the fp16 MFMA rate of the conv kernels' inner-loop shape with no global
                 traffic (infvino_amd/tools/mfma_roof), for zero and for random operands: the
                 matrix cores draw more power on random data and the clock drops
  vendor_gemm_probe  torch.matmul fp16 on random 8192^3 operands (the ROCm BLAS GEMM) on
                 the box: conv_sweep rows of MFMA-bound layers carry frac_practical against
                 it (a fraction above 1 against any probe is not reported: that probe is no
                 roof there)
  hbm_stream_probe  plain torch fill / copy / broadcast-copy rates on the box: the practical
                 HBM roof of a streaming kernel's traffic pattern; config1's batch-64 line
                 carries frac_practical against the broadcast copy (1 read : 2 writes), the
                 dominant kernel's roofline against the copy past the Infinity Cache, the
                 HBM-bound conv_sweep rows against the copy on their side of it (256 MB)
  cpu_baseline   the CPU oracle (oracle/, C + OpenMP) on a bounded sample of the same
                 workload on this host's cores -- a reported baseline, not a target; it
                 records the probe for a CPU OpenCL runtime that could run the reference's own
                 kernels instead
"""
import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# Vector fp32 FMA without packed fp32 (which this build does not use): one FMA per lane per
# cycle, 256 CUs x 64 lanes x 2 FLOPs x 2.4 GHz.  The roof of the depthwise convs, which run
# on the VALU (v_fma_mix_f32) rather than on MFMA.
PEAK_VALU_FP32_TFLOPS = 78.6


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def calibrate(ia, pw):
    """A plain streaming kernel of known size: ReLU over 8 images x 8 x 1024 x 1024 fp16
    (128 MiB read, 128 MiB written per launch).  Its FETCH_SIZE / WRITE_SIZE per dispatch,
    over the known byte counts, give the counter-to-bytes factors."""
    with tempfile.TemporaryDirectory() as d:
        pb = pw.PlanBuilder(d, seed=0)
        y = pb.unary(pb.input("x", [1, 8, 1024, 1024]), pw.UN_RELU)
        pb.output(y)
        m = ia.PlanModel(pb.write(), 0, 8, ia.IVH_FLAG_NO_GRAPH)
        m.setInput(np.zeros(8 * 8 * 1024 * 1024, np.uint16), 8)
        for _ in range(5):
            m.run(8)
        m.close()
    log("[bench] calibration pass: 5 x (128 MiB read + 128 MiB write)")


# Other layers of the YOLOv8n-pose step whose kernels the planner picks (profiled one at a
# time): name, cin, cout, H, W, k, s.  "pair<C>_<H>" is a C2f bottleneck (two 3x3 convs C -> C
# with the block input added), which runs as one fused launch.
MODEL_LAYERS = [
    ("conv3x3s1_128to64_40", 128, 64, 40, 40, 3, 1),
    ("conv3x3s2_64to128_80", 64, 128, 80, 80, 3, 2),
    ("conv3x3s2_128to256_40", 128, 256, 40, 40, 3, 2),
    ("conv1x1_32to32_160", 32, 32, 160, 160, 1, 1),
    ("pair16_160", 16, 16, 160, 160, 3, 1),
    ("pair32_80", 32, 32, 80, 80, 3, 1),
    ("conv3x3s1_64to64_40", 64, 64, 40, 40, 3, 1),
    ("conv3x3s1_128to128_20", 128, 128, 20, 20, 3, 1),
    ("conv3x3s1_256to64_20", 256, 64, 20, 20, 3, 1),
    ("conv3x3s2_64to64_80", 64, 64, 80, 80, 3, 2),
    ("conv3x3s2_128to128_40", 128, 128, 40, 40, 3, 2),
    ("conv1x1_384to128_40", 384, 128, 40, 40, 1, 1),
    ("conv1x1_128to64_80", 128, 64, 80, 80, 1, 1),
    # a Pose head level: the box / class / keypoint branches' first 3x3 convs (64 + 64 + 51
    # channels from one input), which run as one merged conv
    ("heads_64_80", 64, 179, 80, 80, 3, 1),
    ("heads_128_40", 128, 179, 40, 40, 3, 1),
    ("heads_256_20", 256, 179, 20, 20, 3, 1),
    # the same with each branch's second 3x3 conv, which run as one grouped launch
    ("heads2_64_80", 64, 179, 80, 80, 3, 1),
]


def sweep_plan(pw, d, name):
    """Plan of one conv sweep layer in the layout it has inside a model: the stem reads the
    NCHW graph input, every other conv sits between two ReLUs (channels-last tensors).
    "config1": the plan's conv1x1 op on graph tensors (64->128 at 80x80, NCHW in and out);
    "attention": the C2PSA attention block (256 channels, 4 heads, 400 tokens); the
    MODEL_LAYERS names: those layers between two ReLUs."""
    if name == "config1":
        return pw.conv1x1_config(d)[0]
    if name == "attention":
        return pw.c2psa_attention(d)[0]
    extra = next((c for c in MODEL_LAYERS if c[0] == name), None)
    if extra:
        _, cin, cout, H, W, k, s = extra
        pb = pw.PlanBuilder(d, seed=0)
        x = pb.unary(pb.input("x", [1, cin, H, W]), pw.UN_RELU)
        if name.startswith("pair"):
            t = pb.conv(x, cout, 3, 1)
            y = pb.conv(t, cout, 3, 1, res=x)
        elif name.startswith("heads2"):
            # first and second 3x3 convs of each branch, then a 1x1 conv
            y = pb.concat([pb.conv(pb.conv(pb.conv(x, c, 3, 1), c, 3, 1), 16, 1) for c in (51, 64, 64)])
        elif name.startswith("heads"):
            # keypoint branch first, as in the written plans; each branch output read by a conv
            y = pb.concat([pb.conv(pb.conv(x, c, 3, 1), 16, 1) for c in (51, 64, 64)])
        else:
            y = pb.conv(x, cout, k, s)
        pb.output(pb.unary(y, pw.UN_RELU))
        return pb.write()
    _, cin, cout, H, W, k, s, g, act = next(c for c in pw.CONV_SWEEP if c[0] == name)
    pb = pw.PlanBuilder(d, seed=0)
    x = pb.input("x", [1, cin, H, W])
    if not name.startswith("stem"):
        x = pb.unary(x, pw.UN_RELU)
    y = pb.unary(pb.conv(x, cout, k, s, groups=g, act=act), pw.UN_RELU)
    pb.output(y)
    return pb.write()


def layer_runs(ia, pw, name, batch, iters, flags=0):
    """One sweep layer's plan, `iters` eager passes (for counter collection on that conv)."""
    with tempfile.TemporaryDirectory() as d:
        m = ia.PlanModel(sweep_plan(pw, d, name), 0, batch, ia.IVH_FLAG_NO_GRAPH | flags)
        x0 = np.random.default_rng(0).random(m.inputNumel() * batch, dtype=np.float32)
        m.setInput(x0.astype(np.float16).view(np.uint16), batch)
        for _ in range(iters):
            m.run(batch)
        m.close()
    log(f"[bench] layer {name} batch {batch}: {iters} passes")


def conv_sweep(ia, pw, batch, iters, only=None):
    """The conv operator sweep (stem, strided and stride-1 3x3, depthwise) at `batch`, each
    conv measured in the layout it has inside a model: the stem reads the NCHW graph input,
    every other conv sits between two ReLUs so its input and output are internal
    (channels-last) tensors.  Per layer: HIP-event time of the conv node, algorithmic
    TFLOP/s and GB/s, and the fraction of the roof that binds it: for the MFMA convs MFMA
    when the arithmetic intensity is above the ridge, HBM otherwise; for the depthwise convs
    (vector FMAs) the larger of the HBM time and the fp32 VALU time.  `only`: a prefix of the
    layer names to keep."""
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    rows = []
    for name, cin, cout, H, W, k, s, g, act in pw.CONV_SWEEP:
        if only and not name.startswith(only):
            continue
        with tempfile.TemporaryDirectory() as d:
            m = ia.PlanModel(sweep_plan(pw, d, name), 0, batch, ia.IVH_FLAG_NO_GRAPH)
            x0 = np.random.default_rng(0).random(m.inputNumel() * batch, dtype=np.float32)
            m.setInput(x0.astype(np.float16).view(np.uint16), batch)
            m.run(batch)
            ci = next(i for i in range(m.nodeCount()) if m.nodeInfo(i)["op"].startswith("conv"))
            inf = m.nodeInfo(ci)
            t = float(m.profileNodes(batch, iters)[ci]) * 1e-3
            m.close()
        fl, by = inf["flops"] * batch, inf["bytes"] * batch
        tf, gbs = fl / t / 1e12, by / t / 1e9
        if inf["kernel"] == "dwconv":
            t_valu, t_hbm = fl / (PEAK_VALU_FP32_TFLOPS * 1e12), by / (PEAK_HBM_GBS * 1e9)
            bound = "valu" if t_valu > t_hbm else "hbm"
            frac = max(t_valu, t_hbm) / t
        else:
            bound = "mfma" if fl / by >= ridge else "hbm"
            frac = tf / PEAK_FP16_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS
        rows.append({"layer": name, "kernel": inf["kernel"], "us": round(t * 1e6, 2),
                     "tflops": round(tf, 1), "gbs": round(gbs, 1), "bound": bound, "frac": round(frac, 4)})
        log(f"[sweep] {name:24s} b{batch} {inf['kernel']:12s} {t * 1e6:8.2f} us {tf:7.1f} TFLOP/s "
            f"{gbs:7.1f} GB/s -> {bound} {frac * 100:.1f}%")
    return rows


def roof_of(flops, nbytes, t_s):
    """Achieved rate of one launch against the roof that binds it (MFMA when its arithmetic
    intensity is above the ridge, HBM otherwise)."""
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if flops > 0 and flops / max(nbytes, 1) >= ridge:
        a = flops / t_s / 1e12
        return {"bound": "mfma", "achieved": round(a, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(a / PEAK_FP16_TFLOPS, 4)}
    a = nbytes / t_s / 1e9
    return {"bound": "hbm", "achieved": round(a, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(a / PEAK_HBM_GBS, 4)}


def ideal_s(flops, nbytes):
    return max(flops / (PEAK_FP16_TFLOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9))


def config1(ia, pw, iters):
    """The single pointwise conv of the plan's conv1x1 op, 64->128 at 80x80 with SiLU, at
    batch 1 and 64 (HIP-event time of the conv node, eager launches)."""
    out = {}
    for b in (1, 64):
        with tempfile.TemporaryDirectory() as d:
            path, _ = pw.conv1x1_config(d)
            m = ia.PlanModel(path, 0, b, ia.IVH_FLAG_NO_GRAPH)
            x0 = np.random.default_rng(0).random(m.inputNumel() * b, dtype=np.float32)
            m.setInput(x0.astype(np.float16).view(np.uint16), b)
            m.run(b)
            inf = m.nodeInfo(0)
            t = float(m.profileNodes(b, iters)[0]) * 1e-3
            m.close()
        fl, by = inf["flops"] * b, inf["bytes"] * b
        row = {"batch": b, "kernel": inf["kernel"], "us": round(t * 1e6, 2), "gflop": round(fl / 1e9, 4),
               "mbytes": round(by / 1e6, 3), "roofline": roof_of(fl, by, t)}
        out[f"b{b}"] = row
        log(f"[config1] conv1x1 64->128 @80x80 SiLU batch {b}: {row['us']} us, {row['roofline']}")
    return out


def attention(ia, pw, iters):
    """The C2PSA attention block (256 channels, 4 heads, head_dim 64, 20x20 = 400 tokens) at
    batch 64 and 1: time of the attention core -- q^T k, scale, softmax, v P^T, as one fused
    kernel (the default) and node by node (IVH_FLAG_NO_FUSE_ATTN) -- and of the whole block,
    each node timed with HIP events."""
    out = {}
    for b in (64, 1):
        row = {"batch": b}
        for label, flags in (("fused", 0), ("node_by_node", ia.IVH_FLAG_NO_FUSE_ATTN)):
            with tempfile.TemporaryDirectory() as d:
                path, core_flops = pw.c2psa_attention(d)
                m = ia.PlanModel(path, 0, b, ia.IVH_FLAG_NO_GRAPH | flags)
                x0 = np.random.default_rng(0).random(m.inputNumel() * b, dtype=np.float32)
                m.setInput(x0.astype(np.float16).view(np.uint16), b)
                m.run(b)
                prof = m.profileNodes(b, iters)
                infos = [m.nodeInfo(i) for i in range(m.nodeCount())]
                m.close()
            core = [i for i, inf in enumerate(infos) if inf["op"] == "attention"]
            if not core:  # q's permute and scale (when the scale is on q^T) through the last bmm
                first = next(i for i, inf in enumerate(infos) if inf["op"] in ("bmm", "permute_0213"))
                last = max(i for i, inf in enumerate(infos) if inf["op"] == "bmm")
                core = list(range(first, last + 1))
            t_core = float(sum(prof[i] for i in core)) * 1e-3
            by_core = sum(infos[i]["bytes"] for i in core) * b
            t_block = float(sum(prof[i] for i in range(1, len(infos)))) * 1e-3  # all but the leading ReLU
            row[label] = {"core_us": round(t_core * 1e6, 2), "block_us": round(t_block * 1e6, 2),
                          "core_mbytes": round(by_core / 1e6, 2),
                          "core_tflops": round(core_flops * b / t_core / 1e12, 2),
                          "roofline": roof_of(core_flops * b, by_core, t_core),
                          "nodes": {infos[i]["desc"]: round(float(prof[i]) * 1e3, 2) for i in core}}
        row["core_gflop"] = round(core_flops * b / 1e9, 3)
        out[f"b{b}"] = row
        f, n = row["fused"], row["node_by_node"]
        log(f"[attention] C2PSA 256ch 4 heads 400 tokens batch {b}: core fused {f['core_us']} us "
            f"({f['core_tflops']} TFLOP/s, {f['roofline']['bound']} {f['roofline']['frac'] * 100:.1f}%) vs node by node "
            f"{n['core_us']} us; block {f['block_us']} vs {n['block_us']} us")
    return out


def opencl_probe():
    """Whether this host can run the reference's own OpenCL kernels on its CPU cores: the ICD
    files present and, through the OpenCL loader, every platform and its CPU devices."""
    import ctypes as C
    import glob
    icds = sorted(os.path.basename(f) for f in glob.glob("/etc/OpenCL/vendors/*.icd"))
    res = {"icd_files": icds, "platforms": [], "cpu_devices": 0}
    try:
        cl = C.CDLL("libOpenCL.so.1")
    except OSError as e:
        res["loader"] = f"absent ({e})"
        return res
    res["loader"] = "libOpenCL.so.1"
    n = C.c_uint(0)
    if cl.clGetPlatformIDs(0, None, C.byref(n)) != 0 or n.value == 0:
        return res
    plats = (C.c_void_p * n.value)()
    cl.clGetPlatformIDs(n.value, plats, None)
    for pf in plats:
        name = C.create_string_buffer(256)
        cl.clGetPlatformInfo(C.c_void_p(pf), C.c_uint(0x0902), C.c_size_t(256), name, None)  # CL_PLATFORM_NAME
        nd = C.c_uint(0)
        rc = cl.clGetDeviceIDs(C.c_void_p(pf), C.c_ulong(1 << 1), 0, None, C.byref(nd))  # CL_DEVICE_TYPE_CPU
        ndev = nd.value if rc == 0 else 0
        res["platforms"].append({"name": name.value.decode(errors="replace"), "cpu_devices": ndev})
        res["cpu_devices"] += ndev
    return res


def mfma_roof_probe():
    """Runs infvino_amd/tools/mfma_roof (a child process) and returns its JSON line, or a
    note when the probe binary is absent or fails."""
    import subprocess
    exe = os.path.join(ROOT, "infvino_amd", "tools", "mfma_roof")
    if not os.path.exists(exe):
        return {"note": "probe not built (make -C infvino_amd/csrc tools)"}
    try:
        r = subprocess.run([exe, "2000"], capture_output=True, text=True, timeout=120)
    except subprocess.TimeoutExpired:
        return {"note": "probe timed out"}
    if r.returncode != 0:
        return {"note": f"probe failed: {r.stderr.strip()[-200:]}"}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"[bench] MFMA roof probe: zeros {res['zeros_tflops']} TFLOP/s, random {res['random_tflops']} TFLOP/s")
    return res


def hbm_stream_probe():
    """Runs `bench.py --phase hbm` as a child process (torch initialises its own HIP context
    there, away from the library's) and returns its JSON line, or a note."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--phase", "hbm"], capture_output=True,
                           text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return {"note": "probe timed out"}
    if r.returncode != 0:
        return {"note": f"probe failed: {r.stderr.strip()[-200:]}"}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"[bench] HBM stream probe: {res}")
    return res


def hbm_stream_rates():
    """Plain torch kernels with the traffic patterns of the streaming convs, timed with
    events: a fill of 104.9 MB (writes only), a 52.4 MB copy (1:1) and a broadcast copy of
    52.4 MB into 104.9 MB (1 read : 2 writes, the pattern of the conv1x1 config 64 -> 128) and
    a 157 MB copy (314 MB moved, more than the Infinity Cache holds, like the stem's 367 MB).
    What they reach on this box is the practical HBM roof of such a stream (below the 8 TB/s
    peak); footprints under 256 MB are partly served by the Infinity Cache between passes."""
    import torch
    n = 52428800 // 2
    x = torch.randn(n, device="cuda:0", dtype=torch.float16)
    y = torch.empty(2 * n, device="cuda:0", dtype=torch.float16)
    z = torch.empty(n, device="cuda:0", dtype=torch.float16)

    def rate(fn, nbytes, iters=50):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(nbytes / (e0.elapsed_time(e1) / iters * 1e-3) / 1e9, 1)

    y2 = y.view(2, n)
    res = {"fill_gbs": rate(lambda: y.fill_(1.0), 4 * n),
           "copy_gbs": rate(lambda: z.copy_(x), 4 * n),
           "broadcast_1r2w_gbs": rate(lambda: y2.copy_(x.unsqueeze(0).expand(2, n)), 6 * n)}
    del x, y, z, y2
    big = torch.empty(3 * n + 512, device="cuda:0", dtype=torch.float16).normal_()
    big2 = torch.empty_like(big)
    res["copy_large_gbs"] = rate(lambda: big2.copy_(big), 4 * big.numel(), iters=20)  # 157 + 157 MB
    res.update({"unit": "GB/s of algorithmic bytes", "source": "torch fill_ / copy_ kernels",
                "copy_large_bytes": 4 * big.numel()})
    return res


def vendor_gemm_rate():
    """torch.matmul (the ROCm BLAS libraries' fp16 GEMM) on random 8192 x 8192 x 8192
    operands, timed with events: what a vendor GEMM sustains on this box on random data
    (the matrix cores draw more power on random operands and the clock drops), the roof the
    MFMA-bound conv layers are rated against."""
    import torch
    n = 8192
    g = torch.Generator(device="cuda:0").manual_seed(0)
    a = torch.rand(n, n, device="cuda:0", dtype=torch.float16, generator=g) - 0.5
    b = torch.rand(n, n, device="cuda:0", dtype=torch.float16, generator=g) - 0.5
    c = torch.empty(n, n, device="cuda:0", dtype=torch.float16)
    for _ in range(3):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    iters = 20
    e0.record()
    for _ in range(iters):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / iters
    tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    return {"gemm_f16_tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_FP16_TFLOPS, 4), "ms": round(ms, 4),
            "shape": [n, n, n], "operands": "uniform [-0.5, 0.5) fp16, fp32 accumulate (torch.matmul)",
            "torch": torch.__version__}


def vendor_gemm_probe():
    """Runs `bench.py --phase gemm` as a child process and returns its JSON line, or a note."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--phase", "gemm"], capture_output=True,
                           text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return {"note": "probe timed out"}
    if r.returncode != 0:
        return {"note": f"probe failed: {r.stderr.strip()[-200:]}"}
    res = json.loads(r.stdout.strip().splitlines()[-1])
    log(f"[bench] vendor GEMM probe: {res}")
    return res


def model_lines(ia, pw, specs, steps, warmup):
    """The other model configurations: images/s of graph replays at each batch (inputs
    resident in HBM) and the synchronous batch-1 latency."""
    out = {}
    for name, imgsz, batches in specs:
        tmp = tempfile.TemporaryDirectory()
        path, flops = pw.MODELS[name](tmp.name, seed=0, imgsz=imgsz)
        row = {"imgsz": imgsz, "gflop_per_image": round(flops / 1e9, 3)}
        bmax = max(batches)
        x = np.random.default_rng(0).random(3 * imgsz * imgsz * bmax, dtype=np.float32).astype(np.float16)
        m = ia.PlanModel(path, 0, bmax, ia.IVH_FLAG_ASYNC)
        m.setInput(x.view(np.uint16), bmax)
        for b in batches:
            for _ in range(warmup):
                m.run(b)
            m.sync()
            t0 = time.perf_counter()
            for _ in range(steps):
                m.run(b)
            m.sync()
            row[f"images_per_s_b{b}"] = round(b * steps / (time.perf_counter() - t0), 1)
        m.close()
        m1 = ia.PlanModel(path, 0, 1, 0)
        m1.setInput(x.view(np.uint16)[:3 * imgsz * imgsz], 1)
        for _ in range(warmup):
            m1.run(1)
        lat = []
        for _ in range(steps):
            t = time.perf_counter()
            m1.run(1)
            lat.append(time.perf_counter() - t)
        m1.close()
        row["latency_b1_ms"] = round(float(np.mean(lat)) * 1e3, 4)
        out[name] = row
        log(f"[models] {name}@{imgsz}: " + ", ".join(f"{k}={v}" for k, v in row.items()))
        tmp.cleanup()
    return out


def measured_traffic(node_desc, batch):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc
    summary (profiles/traffic_dominant_kernel.md: node / batch / hbm_bytes_per_launch
    records), when it was measured on this node at this batch."""
    path = os.path.join(ROOT, "profiles", "traffic_dominant_kernel.md")
    if not os.path.exists(path):
        return None
    node = b = None
    for line in open(path):
        if line.startswith("node:"):
            node, b = line.split(":", 1)[1].strip(), None
        elif line.startswith("batch:"):
            b = int(line.split(":", 1)[1])
        elif line.startswith("hbm_bytes_per_launch:") and node == node_desc and b == batch:
            return float(line.split(":", 1)[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--imgsz", type=int, default=640)
    ap.add_argument("--model", default="yolov8n-pose")
    ap.add_argument("--profile-iters", type=int, default=5)
    ap.add_argument("--cpu-images", type=int, default=-1, help="oracle sample size (-1: ~15 s worth)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the per-layer conv sweep")
    ap.add_argument("--no-models", action="store_true", help="skip the MobileNetV3 / YOLO11n lines")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch node by node instead of replaying the captured HIP graph")
    ap.add_argument("--layer", default="conv3x3s2_16to32_320", help="sweep layer (or config1) for --phase layer")
    ap.add_argument("--flags", type=lambda v: int(v, 0), default=0,
                    help="extra ivh_create flags for --phase layer and --phase throughput (e.g. 0x200: no "
                         "resident-weight kernel, 0x300000: no upsample-concat / sibling-conv fusion)")
    ap.add_argument("--phase", default="all", choices=["all", "throughput", "calib", "sweep", "layer", "hbm", "gemm",
                                                       "attention"],
                    help="throughput: only the batch-64 timed steps (for counter runs); calib: a known-size "
                         "128 MiB-in/128 MiB-out elementwise pass to scale FETCH_SIZE/WRITE_SIZE; "
                         "sweep: the conv sweep only; layer: --steps passes of one sweep layer (--layer); "
                         "hbm: the torch HBM stream probe alone (one JSON line); "
                         "gemm: the torch fp16 GEMM probe alone (one JSON line); "
                         "attention: the C2PSA attention measurement alone (one JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the batch axis would shard as independent replicas, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    if args.phase == "hbm":  # before the library touches the GPU
        print(json.dumps(hbm_stream_rates()))
        return
    if args.phase == "gemm":
        print(json.dumps(vendor_gemm_rate()))
        return
    import infvino_amd as ia
    from infvino_amd import planwriter as pw

    if args.phase == "attention":
        print(json.dumps(attention(ia, pw, max(args.profile_iters, 10))))
        return
    if args.phase == "calib":
        calibrate(ia, pw)
        return
    if args.phase == "sweep":
        conv_sweep(ia, pw, args.batch, max(args.profile_iters, 10))
        return
    if args.phase == "layer":
        layer_runs(ia, pw, args.layer, args.batch, args.steps, args.flags)
        return
    tmp = tempfile.TemporaryDirectory()
    path, flops_img = pw.MODELS[args.model](tmp.name, seed=0, imgsz=args.imgsz)
    B = args.batch
    rng = np.random.default_rng(0)
    n_in = 3 * args.imgsz * args.imgsz
    x = rng.random(n_in * B, dtype=np.float32).astype(np.float16).view(np.uint16)

    # ---- throughput: K graph replays queued back to back, synchronised at both ends
    gflag = ia.IVH_FLAG_NO_GRAPH if args.no_graph else 0
    m = ia.PlanModel(path, 0, B, ia.IVH_FLAG_ASYNC | gflag | (args.flags if args.phase == "throughput" else 0))
    m.setInput(x, B)
    for _ in range(args.warmup):
        m.run(B)
    m.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.run(B)
    m.sync()
    dt = time.perf_counter() - t0
    ms_step = dt * 1e3 / args.steps
    ips = B * args.steps / dt
    log(f"[bench] {args.model}@{args.imgsz} batch {B}: {ms_step:.3f} ms/step, {ips:.0f} images/s")

    if args.phase == "throughput":
        m.close()
        log(json.dumps({"phase": "throughput", "images_per_s": round(ips, 1), "ms_per_step": round(ms_step, 4)}))
        return
    # ---- per-node device time at batch B (HIP events on the model stream)
    prof = m.profileNodes(B, args.profile_iters)
    infos = [m.nodeInfo(i) for i in range(m.nodeCount())]
    conv_t = sum(t for t, inf in zip(prof, infos) if inf["op"].startswith("conv"))
    conv_f = sum(inf["flops"] * B for inf in infos if inf["op"].startswith("conv"))
    order = np.argsort(-prof)
    log(f"[bench] per-node device time, batch {B} (sum {prof.sum():.3f} ms; graph step {ms_step:.3f} ms)")
    for i in order[:25]:
        inf = infos[i]
        t = prof[i]
        tf = inf["flops"] * B / (t * 1e-3) / 1e12 if t > 0 else 0
        gbs = inf["bytes"] * B / (t * 1e-3) / 1e9 if t > 0 else 0
        log(f"  {t:8.4f} ms  {tf:7.1f} TFLOP/s  {gbs:7.1f} GB/s  {inf['kernel']:12s} {inf['desc']}")
    dom = int(order[0])
    d = infos[dom]
    t_dom = prof[dom] * 1e-3
    ai = d["flops"] / d["bytes"] if d["bytes"] else float("inf")
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    if d["flops"] > 0 and ai >= ridge:
        achieved = d["flops"] * B / t_dom / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP16_TFLOPS, 4)}
    else:
        achieved = d["bytes"] * B / t_dom / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4)}
    traffic = measured_traffic(d["desc"], B)
    roof.update({"traffic": traffic,
                 "traffic_source": ("rocprofv3 FETCH_SIZE + WRITE_SIZE of this node, scaled by a calibration "
                                    "kernel: profiles/traffic_dominant_kernel.md (committed, not measured in "
                                    "this run)") if traffic else None,
                 "kernel": d["kernel"], "node": d["desc"],
                 "launch_ms": round(t_dom * 1e3, 4),
                 "flops_per_launch": d["flops"] * B, "bytes_per_launch": d["bytes"] * B})
    conv_frac = conv_f / (conv_t * 1e-3) / 1e12 / PEAK_FP16_TFLOPS if conv_t > 0 else 0.0
    # the whole step against its roofline: every launching node's ideal time (its binding
    # roof at the published peaks) over its measured time, weighted by the measured time
    t_meas = float(prof.sum()) * 1e-3
    t_ideal = sum(ideal_s(inf["flops"] * B, inf["bytes"] * B) for t, inf in zip(prof, infos) if t > 0)
    roof_step = {"frac": round(t_ideal / t_meas, 4), "ideal_ms": round(t_ideal * 1e3, 4),
                 "node_sum_ms": round(t_meas * 1e3, 4),
                 "definition": "sum over launching nodes of max(FLOPs / 2500 TFLOP/s, bytes / 8000 GB/s) "
                               "over the sum of their HIP-event times, batch 64"}
    log(f"[bench] step roofline: ideal {t_ideal * 1e3:.3f} ms of {t_meas * 1e3:.3f} ms node time "
        f"-> {roof_step['frac'] * 100:.1f}%")
    m.close()

    # ---- batch-1 latency: synchronous runs (graph replay), mean wall time
    m1 = ia.PlanModel(path, 0, 1, gflag)
    m1.setInput(x[:n_in], 1)
    for _ in range(max(args.warmup, 5)):
        m1.run(1)
    lat = []
    for _ in range(max(args.steps, 20)):
        t = time.perf_counter()
        m1.run(1)
        lat.append(time.perf_counter() - t)
    lat_ms = float(np.mean(lat) * 1e3)
    log(f"[bench] batch 1 latency: mean {lat_ms:.3f} ms, p50 {np.median(lat) * 1e3:.3f} ms")
    prof1 = m1.profileNodes(1, args.profile_iters)
    inf1 = [m1.nodeInfo(i) for i in range(m1.nodeCount())]
    launched = sum(1 for i in inf1 if i["kernel"] != "(view)")
    log(f"[bench] per-node device time, batch 1 (sum {prof1.sum():.3f} ms over {launched} launching nodes)")
    for i in np.argsort(-prof1)[:15]:
        log(f"  {prof1[i]:8.4f} ms  {inf1[i]['kernel']:12s} {inf1[i]['desc']}")
    m1.close()

    c1 = None if args.no_sweep else config1(ia, pw, max(args.profile_iters, 10))
    hbm_probe = hbm_stream_probe()

    def practical(achieved, ref):
        # a fraction of what a plain library kernel reaches on the box; a kernel that beats
        # the probe shows the probe is no roof there, so no fraction is reported
        f = achieved / ref
        return round(f, 4) if f <= 1.0 else None

    if c1 and hbm_probe.get("broadcast_1r2w_gbs"):
        c1["b64"]["roofline"]["frac_practical"] = practical(c1["b64"]["roofline"]["achieved"],
                                                            hbm_probe["broadcast_1r2w_gbs"])
    if roof["bound"] == "hbm" and hbm_probe.get("copy_large_gbs"):
        # against a plain copy of a footprint past the Infinity Cache, as the step's largest
        # node (367 MB) is
        roof["practical_peak"] = hbm_probe["copy_large_gbs"]
        roof["frac_practical"] = practical(roof["achieved"], hbm_probe["copy_large_gbs"])
    probe = mfma_roof_probe()
    gemm = vendor_gemm_probe()
    sweep = None
    if not args.no_sweep:
        sweep = {f"b{b}": conv_sweep(ia, pw, b, max(args.profile_iters, 10)) for b in (B, 1)}
        sweep["dw_b256"] = conv_sweep(ia, pw, 256, max(args.profile_iters, 10), only="dw")
        for rows in sweep.values():
            for r in rows:
                if r["bound"] == "mfma" and gemm.get("gemm_f16_tflops"):
                    # against the vendor GEMM on random operands on this box
                    r["frac_practical"] = practical(r["tflops"], gemm["gemm_f16_tflops"])
                elif r["bound"] == "hbm" and hbm_probe.get("copy_gbs") and hbm_probe.get("copy_large_gbs"):
                    # a copy of the same side of the 256 MB Infinity Cache as the layer's bytes
                    nbytes = r["gbs"] * 1e9 * r["us"] * 1e-6
                    ref = hbm_probe["copy_large_gbs"] if nbytes > 256e6 else hbm_probe["copy_gbs"]
                    r["frac_practical"] = practical(r["gbs"], ref)
    attn = None if args.no_sweep else attention(ia, pw, max(args.profile_iters, 10))
    others = None if args.no_models else model_lines(
        ia, pw, [("yolov8n-pose", 640, (16, 64)), ("mobilenetv3-small", 224, (1, 32, 256)),
                 ("yolo11n-pose", 640, (1, 64))], 20, 5)

    # ---- CPU baseline: the oracle on a bounded sample of the same workload
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        p = O.Plan.load(path)
        cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        t = time.perf_counter()
        O.run_plan(p, x[:n_in], 1)
        one = time.perf_counter() - t
        k = args.cpu_images if args.cpu_images > 0 else max(1, min(64, int(15.0 / max(one, 1e-3))))
        t = time.perf_counter()
        O.run_plan(p, x[:n_in * k], k)
        el = time.perf_counter() - t
        ocl = opencl_probe()
        cpu = {"value": round(k / el, 3), "unit": "images/s", "cores": cores, "kind": "port",
               "sample": f"{k} images of {args.model} 3x{args.imgsz}x{args.imgsz} through the C oracle "
                         f"(fp32 accumulate, OpenMP over output channels), {el:.1f} s",
               "reference_kernels": ("unavailable: no OpenCL CPU device on this host (the reference's .cl "
                                     "kernels need one; see opencl_probe)") if ocl["cpu_devices"] == 0 else
                                    "an OpenCL CPU device exists (opencl_probe); not used by this bench",
               "opencl_probe": ocl}
        log(f"[bench] cpu oracle: {k / el:.3f} images/s on {cores} threads")

    out = {
        "metric": "images/sec at batch 1 & 64 (yolov8n-pose 640, fp16); conv MFMA % peak",
        "value": round(ips, 1),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (uniform[0,1) frames, random-init He-normal weights, BN folded)",
        "config": {"workload": f"{args.model} 3x{args.imgsz}x{args.imgsz} batch {B}, one plan pass per step",
                   "batch": B, "imgsz": args.imgsz, "gflop_per_image": round(flops_img / 1e9, 3)},
        "latency_b1_ms": round(lat_ms, 4),
        "launch": "eager" if args.no_graph else "hip_graph",
        "conv_mfma_frac": round(conv_frac, 4),
        "tflops_effective": round(flops_img * ips / 1e12, 2),
        "roofline": roof,
        "roofline_step": roof_step,
        "mfma_roof_probe": probe,
        "vendor_gemm_probe": gemm,
        "hbm_stream_probe": hbm_probe,
        "config1": c1,
        "conv_sweep": sweep,
        "attention": attn,
        "other_models": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    tmp.cleanup()


if __name__ == "__main__":
    main()
