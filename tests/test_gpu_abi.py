"""Single-op C ABI (include/ivh.h, ivh_conv2d_f16 ... ivh_bmm_f16) on the GPU: each entry
point runs one operation on caller-owned device buffers (torch allocations here) and is
compared with the CPU oracle on the same seeded inputs, with the op-level bar of the plan
tests (fp32 oracle: mean_rel < 2e-3, max_rel < 1e-2; data movement bit-exact).  The
padding channels of channels-last activations hold NaN bit patterns, so a kernel that lets
them reach an output fails."""
import numpy as np
import pytest
import torch

import infvino_amd.ops as ops
from oracle import oracle as O

pytestmark = pytest.mark.gpu

F32_MEAN, F32_MAX = 2e-3, 1e-2
NAN16 = 0x7E00


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16).copy()).to("cuda")


def _host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def _nhwc(x: np.ndarray, B, C, H, W, fill=NAN16) -> np.ndarray:
    cs = (C + 7) // 8 * 8
    out = np.full((B, H, W, cs), fill, np.uint16)
    out[..., :C] = x.reshape(B, C, H, W).transpose(0, 2, 3, 1)
    return out


def _from_nhwc(y: np.ndarray, B, C, H, W) -> np.ndarray:
    cs = (C + 7) // 8 * 8
    return y.reshape(B, H, W, cs)[..., :C].transpose(0, 3, 1, 2).reshape(B, -1)


def _ok(got, ref, label):
    mean_rel, max_rel, max_abs, _ = O.rel_errors(O.h2f(got.ravel()), O.h2f(ref.ravel()))
    print(f"{label}: mean_rel={mean_rel:.2e} max_rel={max_rel:.2e} max_abs={max_abs:.2e}")
    return mean_rel < F32_MEAN and max_rel < F32_MAX


def _pack(d, w, b):
    packed = torch.empty(ops.conv_packed_bytes(d), dtype=torch.uint8, device="cuda")
    ops.pack_conv_weights(d, w, b, packed.data_ptr())
    return packed


CONVS = [
    # cin, cout, h, w, k, s, p, g, act, channels_last, residual
    (64, 128, 20, 20, 1, 1, 0, 1, ops.ACT_SILU, 1, False),     # 1x1 implicit GEMM
    (24, 40, 17, 19, 3, 1, 1, 1, ops.ACT_HSWISH, 1, True),     # 3x3 s1 LDS patch, ragged, residual
    (21, 32, 15, 15, 3, 2, 1, 1, ops.ACT_SILU, 1, False),      # 3x3 s2 im2col, Cin % 8 != 0
    (8, 20, 9, 11, 5, 1, 2, 1, ops.ACT_SIGMOID, 1, True),      # 5x5, 8 channels a piece, residual
    (13, 48, 17, 14, 3, 2, 1, 1, ops.ACT_SILU, 1, True),       # 3x3 s2 LDS patch, pad channels, residual
    (128, 256, 10, 10, 3, 1, 1, 1, ops.ACT_RELU, 1, False),    # wide, K step 64
    (3, 16, 64, 64, 3, 2, 1, 1, ops.ACT_SILU, 0, False),       # stem, planar in and out
    (16, 1, 4, 64, 1, 1, 0, 1, ops.ACT_NONE, 0, False),        # planar 1x1, one output channel
    (32, 64, 10, 10, 3, 1, 1, 4, ops.ACT_RELU, 1, False),      # grouped, direct kernel
    (48, 48, 14, 14, 5, 2, 2, 48, ops.ACT_HSWISH, 1, True),    # depthwise 5x5 s2, residual
]


@pytest.mark.parametrize("cin,cout,h,w,k,s,p,g,act,cl,res", CONVS,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}x{c[3]}-k{c[4]}s{c[5]}g{c[7]}-cl{c[9]}" for c in CONVS])
def test_abi_conv2d(cin, cout, h, w, k, s, p, g, act, cl, res):
    B = 3
    rng = np.random.default_rng(cin * 1000 + cout)
    d = ops.conv_desc(cin, cout, h, w, k, s, p, g, act, True, cl)
    ho, wo = ops.conv_out_dims(d)
    assert (ho, wo) == ((h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1)
    x = O.f2h(rng.random(B * cin * h * w).astype(np.float32))
    wt = O.f2h((rng.standard_normal(cout * (cin // g) * k * k) * np.sqrt(2.0 / (cin // g * k * k))).astype(np.float32))
    bias = O.f2h((rng.standard_normal(cout) * 0.01).astype(np.float32))
    r = O.f2h(rng.random(B * cout * ho * wo).astype(np.float32)) if res else None
    packed = _pack(d, wt, bias)
    conv = ops.dwconv if g == cin == cout and k in (3, 5) else ops.conv2d
    if cl:
        xd = _dev(_nhwc(x, B, cin, h, w))
        yd = _dev(np.full(B * ho * wo * ((cout + 7) // 8 * 8), NAN16, np.uint16))
        rd = _dev(_nhwc(r, B, cout, ho, wo)) if res else None
    else:
        xd, yd = _dev(x), _dev(np.full(B * cout * ho * wo, NAN16, np.uint16))
        rd = _dev(r) if res else None
    conv(d, xd.data_ptr(), packed.data_ptr(), rd.data_ptr() if rd is not None else None, yd.data_ptr(), B)
    y = _host(yd)
    got = _from_nhwc(y, B, cout, ho, wo) if cl else y.reshape(B, -1)
    for b in range(B):
        ref = O.conv2d(x[b * cin * h * w:(b + 1) * cin * h * w], wt, bias,
                       None if r is None else r[b * cout * ho * wo:(b + 1) * cout * ho * wo],
                       cin, h, w, cout, k, s, p, g, ho, wo, act, O.F32, 2)
        assert _ok(got[b], ref, f"conv {cin}->{cout} {h}x{w} k{k} s{s} g{g} cl{cl} image {b}")


def test_abi_dwconv_rejects_dense():
    d = ops.conv_desc(16, 16, 8, 8, 3, 1, 1, 1)
    with pytest.raises(RuntimeError, match="depthwise"):
        ops.dwconv(d, 16, 16, None, 16, 1)   # rejected before any pointer is used


@pytest.mark.parametrize("n_in,n_out,act", [(576, 1024, ops.ACT_HSWISH), (100, 37, ops.ACT_SIGMOID)])
def test_abi_gemv(n_in, n_out, act):
    B = 5
    rng = np.random.default_rng(n_in)
    d = ops.conv_desc(n_in, n_out, 1, 1, act=act, has_bias=True, channels_last=False)
    x = O.f2h(rng.random(B * n_in).astype(np.float32))
    wt = O.f2h((rng.standard_normal(n_out * n_in) * np.sqrt(2.0 / n_in)).astype(np.float32))
    bias = O.f2h((rng.standard_normal(n_out) * 0.01).astype(np.float32))
    packed = _pack(d, wt, bias)
    xd, yd = _dev(x), _dev(np.zeros(B * n_out, np.uint16))
    ops.gemv(d, xd.data_ptr(), packed.data_ptr(), yd.data_ptr(), B)
    y = _host(yd).reshape(B, n_out)
    for b in range(B):
        ref = O.conv2d(x[b * n_in:(b + 1) * n_in], wt, bias, None, n_in, 1, 1, n_out, 1, 1, 0, 1, 1, 1, act, O.F32, 1)
        assert _ok(y[b], ref, f"gemv {n_in}->{n_out} image {b}")


def test_abi_eltwise():
    B, n = 2, 4000
    rng = np.random.default_rng(7)
    a = O.f2h((rng.random(B * n) * 4 - 2).astype(np.float32))
    bv = O.f2h((rng.random(B * n) + 0.5).astype(np.float32))
    L = O.lib()
    ad, bd, yd = _dev(a), _dev(bv), _dev(np.zeros(B * n, np.uint16))
    for op in range(4):
        ops.eltwise(op, ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), n, B)
        ref = np.empty(B * n, np.uint16)
        L.ivo_ew_binary(a, bv, ref, B * n, op, 0)
        assert np.array_equal(_host(yd), ref), f"binary op {op}"
    ops.eltwise(2, ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), n, B, b_scalar=True)
    ref = O.f2h(O.h2f(a) * O.h2f(bv[:1]))
    assert np.array_equal(_host(yd), ref), "scalar multiply"
    # unary: canonical activation codes, against the formulas in fp32 with one rounding
    af = O.h2f(a).astype(np.float32)
    forms = {ops.ACT_SILU: af / (1 + np.exp(-af)), ops.ACT_RELU: np.maximum(af, 0),
             ops.ACT_HSWISH: af * np.clip(af + 3, 0, 6) / 6, ops.ACT_HSIGMOID: np.clip(af + 3, 0, 6) / 6,
             ops.ACT_SIGMOID: 1 / (1 + np.exp(-af))}
    for act, f in forms.items():
        ops.eltwise(act, ad.data_ptr(), None, yd.data_ptr(), n, B)
        got = O.h2f(_host(yd))
        ref = O.h2f(O.f2h(f.astype(np.float32)))
        assert np.max(np.abs(got - ref)) <= 2e-3 * max(1.0, float(np.max(np.abs(ref)))), f"unary {act}"


def test_abi_pool_softmax_bmm():
    rng = np.random.default_rng(9)
    L = O.lib()
    B, C, H, W = 2, 16, 20, 20
    x = O.f2h((rng.random(B * C * H * W) * 2 - 1).astype(np.float32))
    xd = _dev(x)
    # maxpool 5/1/2 (SPPF) and 3/2/1: bit-exact
    for k, s, p in [(5, 1, 2), (3, 2, 1)]:
        ho, wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
        yd = _dev(np.zeros(B * C * ho * wo, np.uint16))
        ops.pool(ops.POOL_MAX, xd.data_ptr(), yd.data_ptr(), C, H, W, k, s, p, B)
        y = _host(yd).reshape(B, -1)
        for b in range(B):
            ref = np.empty(C * ho * wo, np.uint16)
            L.ivo_maxpool(x[b * C * H * W:(b + 1) * C * H * W], ref, C, H, W, ho, wo, k, s, p)
            assert np.array_equal(y[b], ref), f"maxpool {k}/{s}/{p}"
    yd = _dev(np.zeros(B * C * H * W * 4, np.uint16))
    ops.pool(ops.POOL_RESIZE, xd.data_ptr(), yd.data_ptr(), C, H, W, 0, 2, 0, B)
    y = _host(yd).reshape(B, -1)
    for b in range(B):
        ref = np.empty(C * H * W * 4, np.uint16)
        L.ivo_resize_nn(x[b * C * H * W:(b + 1) * C * H * W], ref, C, H, W, 2)
        assert np.array_equal(y[b], ref), "resize x2"
    # softmax over a strided axis (vector path) and over the last axis
    for outer, axis, inner in [(4, 16, 8400 // 4), (3, 10, 1), (2, 24, 20)]:
        n = outer * axis * inner
        s = O.f2h((rng.standard_normal(B * n) * 3).astype(np.float32))
        sd, od = _dev(s), _dev(np.zeros(B * n, np.uint16))
        ops.softmax(sd.data_ptr(), od.data_ptr(), outer, axis, inner, B)
        got = _host(od).reshape(B, -1)
        for b in range(B):
            ref = np.empty(n, np.uint16)
            L.ivo_softmax_axis(s[b * n:(b + 1) * n], ref, outer, axis, inner)
            assert _ok(got[b], ref, f"softmax {outer}x{axis}x{inner}")
    # batched matmul (the C2PSA attention shapes, scaled down)
    bb, m, k, n = 2, 40, 32, 48
    a = O.f2h((rng.standard_normal(B * bb * m * k) * 0.5).astype(np.float32))
    bm = O.f2h((rng.standard_normal(B * bb * k * n) * 0.5).astype(np.float32))
    ad, bd, yd = _dev(a), _dev(bm), _dev(np.zeros(B * bb * m * n, np.uint16))
    ops.bmm(ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), bb, m, k, n, B)
    got = _host(yd).reshape(B, -1)
    for b in range(B):
        ref = np.empty(bb * m * n, np.uint16)
        L.ivo_bmm(a[b * bb * m * k:(b + 1) * bb * m * k], bm[b * bb * k * n:(b + 1) * bb * k * n], ref, bb, m, k, n)
        assert _ok(got[b], ref, "bmm")
