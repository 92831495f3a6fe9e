// Convolution operands: family choice, packing and launch resolution (see conv_pack.hpp).
// Packings restate the reference's weight layouts for this backend's kernels:
//   implicit GEMM  fp16 [round_up(Cout,128)][kpad], k = (ky*K + kx)*cin8 + ci
//   LDS patch      fp16 [round_up(Cout,128)][chunk][tap][ck] (3x3 stride 1 pad 1)
//   stem           fp16 [ceil(Cout/16)*16][32], k = ci*9 + tap; and [16][64], k = tap*4 + ci
//   direct         fp32 [G][Cin/G][K][K][Cout/G]
//   depthwise      fp32 [K][K][C]
// (the reference packs per kernel too: PlanModel.cpp:232-334).
#include "conv_pack.hpp"

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/ivh.h"
#include "kernels.hpp"

namespace ivh {

namespace {

long rup(long v, long m) { return (v + m - 1) / m * m; }

float h2f_bits(uint16_t h)
{
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  uint32_t u;
  if (e == 0) {
    if (m == 0) u = s;
    else {  // subnormal
      int ee = -1;
      uint32_t mm = m;
      do { ++ee; mm <<= 1; } while (!(mm & 0x400));
      u = s | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 0x3ff) << 13);
    }
  } else if (e == 31) u = s | 0x7f800000u | (m << 13);
  else u = s | ((e + 112) << 23) | (m << 13);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

int halo_index(int ck) { return ck == 16 ? 0 : (ck == 32 ? 1 : 2); }

}  // namespace

ConvPacking conv_packing(const ConvSpec & s)
{
  if (s.Cin < 1 || s.Cout < 1 || s.G < 1 || s.Cin % s.G || s.Cout % s.G || s.K < 1 || s.S < 1 || s.P < 0)
    throw std::runtime_error("conv geometry");
  ConvPacking pk;
  const int cin_g = s.Cin / s.G;
  const bool dw = s.G > 1 && s.G == s.Cin && s.Cout == s.Cin && (s.K == 3 || s.K == 5);
  if (dw) pk.family = kFamDw;
  else if (s.G == 1 && (s.x_nhwc || s.x_vec1 || (s.x_planes8 && s.K == 1 && s.S == 1 && s.P == 0)))
    pk.family = kFamIgemm;
  else pk.family = kFamDirect;
  if (s.flags & IVH_FLAG_DIRECT_ONLY) pk.family = dw ? kFamDw : kFamDirect;

  size_t off = 0;
  auto seg = [&](size_t bytes) {
    const size_t o = off;
    off = rup((long)(off + bytes), 256);
    return o;
  };
  if (s.has_bias) pk.bias = seg((size_t)(rup(s.Cout, kIgemmRowPad) + 16) * 4);
  if (pk.family == kFamIgemm) {
    const int rows = (int)rup(s.Cout, kIgemmRowPad);
    pk.cin8 = (int)rup(cin_g, 8);
    pk.kpad = igemm_kpad(s.Cout, s.K * s.K * pk.cin8);
    pk.w = seg((size_t)rows * pk.kpad * 2);
    if (s.K == 3 && s.S == 1 && s.P == 1 && s.x_nhwc && !(s.flags & IVH_FLAG_NO_HALO)) {
      for (int cfg : {0, 7}) {  // every chunk size some tile config may use for this Cin
        const int ck = halo_cfg_ck(cfg, cin_g), hi = halo_index(ck);
        if (pk.halo[hi] != kNoSeg) continue;
        pk.kpad_halo[hi] = (cin_g + ck - 1) / ck * halo_taps(ck) * ck;
        pk.halo[hi] = seg((size_t)rows * pk.kpad_halo[hi] * 2);
      }
      if (cin_g % 32 == 0 && cin_g >= 128 && s.Cout > 64 && s.Cout <= 256 && !(s.flags & IVH_FLAG_NO_WIDE)) {
        pk.wide_bn = 128;
        pk.wide = seg((size_t)rup(s.Cout, pk.wide_bn) * 9 * cin_g * 2);
      }
      // 16 input channels: also one 32-channel chunk (zero past 16), the packing of the
      // second conv of a 32 -> 16 -> 32 bottleneck run as a fused pair of 32 channels
      if (cin_g == 16 && s.Cout == 32 && pk.halo[1] == kNoSeg) {
        pk.kpad_halo[1] = halo_taps(32) * 32;
        pk.halo[1] = seg((size_t)rows * pk.kpad_halo[1] * 2);
      }
    }
  } else if (pk.family == kFamDirect && s.G == 1 && cin_g <= 3 && s.K == 3 && s.Cout <= 32) {
    const int rows = (s.Cout + 15) / 16 * 16;
    pk.stem = true;
    pk.w = seg(((size_t)rows * 32 + 16 * 64) * 2);
    if (s.Cout <= 16) pk.stem_w2 = pk.w + (size_t)rows * 32 * 2;
  } else if (pk.family == kFamDirect) {
    pk.w = seg(((size_t)s.G * cin_g * s.K * s.K * (s.Cout / s.G) + 32) * 4);
  } else {
    pk.w = seg(((size_t)s.K * s.K * s.Cout + 8) * 4);
    pk.dw_w16 = seg(((size_t)s.K * s.K * s.Cout + 8) * 2);
  }
  pk.bytes = off;
  return pk;
}

void conv_pack(const ConvSpec & s, const ConvPacking & pk, const uint16_t * W, const uint16_t * B,
               std::vector<uint8_t> & blob)
{
  blob.assign(pk.bytes, 0);
  const int Cout = s.Cout, K = s.K, G = s.G, cin_g = s.Cin / s.G;
  auto at = [&](int co, int ci, int t) { return W[((size_t)co * cin_g + ci) * K * K + t]; };
  if (pk.bias != kNoSeg) {
    float * bf = reinterpret_cast<float *>(blob.data() + pk.bias);
    for (int c = 0; c < Cout; ++c) bf[c] = B ? h2f_bits(B[c]) : 0.0f;
  }
  if (pk.family == kFamIgemm) {
    uint16_t * P = reinterpret_cast<uint16_t *>(blob.data() + pk.w);
    for (int co = 0; co < Cout; ++co)
      for (int ci = 0; ci < cin_g; ++ci)
        for (int t = 0; t < K * K; ++t) P[(size_t)co * pk.kpad + t * pk.cin8 + ci] = at(co, ci, t);
    for (int hi = 0; hi < 3; ++hi) {
      if (pk.halo[hi] == kNoSeg) continue;
      const int ck = hi == 0 ? 16 : (hi == 1 ? 32 : 64), taps = halo_taps(ck), kh = pk.kpad_halo[hi];
      uint16_t * Q = reinterpret_cast<uint16_t *>(blob.data() + pk.halo[hi]);
      for (int co = 0; co < Cout; ++co)
        for (int ci = 0; ci < cin_g; ++ci)
          for (int t = 0; t < 9; ++t) Q[(size_t)co * kh + ((ci / ck) * taps + t) * ck + (ci % ck)] = at(co, ci, t);
    }
    if (pk.wide != kNoSeg) {
      uint16_t * Q = reinterpret_cast<uint16_t *>(blob.data() + pk.wide);
      const int bn = pk.wide_bn, ncb = bn / 32, nch = cin_g / 16, ncg = (Cout + bn - 1) / bn;
      size_t o = 0;
      for (int cg = 0; cg < ncg; ++cg)
        for (int c16 = 0; c16 < nch; ++c16)
          for (int t = 0; t < 9; ++t)
            for (int cb = 0; cb < ncb; ++cb)
              for (int l = 0; l < 64; ++l)
                for (int e = 0; e < 8; ++e, ++o) {
                  const int co = cg * bn + cb * 32 + (l & 31), ci = c16 * 16 + (l >> 5) * 8 + e;
                  Q[o] = co < Cout ? at(co, ci, t) : 0;
                }
    }
  } else if (pk.stem) {
    uint16_t * P = reinterpret_cast<uint16_t *>(blob.data() + pk.w);
    for (int co = 0; co < Cout; ++co)
      for (int k = 0; k < cin_g * 9; ++k) P[(size_t)co * 32 + k] = W[(size_t)co * cin_g * 9 + k];
    if (pk.stem_w2 != kNoSeg) {
      uint16_t * P2 = reinterpret_cast<uint16_t *>(blob.data() + pk.stem_w2);
      for (int co = 0; co < Cout; ++co)
        for (int ci = 0; ci < cin_g; ++ci)
          for (int t = 0; t < 9; ++t) P2[co * 64 + t * 4 + ci] = at(co, ci, t);
    }
  } else if (pk.family == kFamDirect) {
    float * P = reinterpret_cast<float *>(blob.data() + pk.w);
    const int cout_g = Cout / G;
    for (int co = 0; co < Cout; ++co) {
      const int g = co / cout_g, cl = co % cout_g;
      for (int ci = 0; ci < cin_g; ++ci)
        for (int t = 0; t < K * K; ++t)
          P[(((size_t)g * cin_g + ci) * K * K + t) * cout_g + cl] = h2f_bits(at(co, ci, t));
    }
  } else {
    float * P = reinterpret_cast<float *>(blob.data() + pk.w);
    uint16_t * P16 = reinterpret_cast<uint16_t *>(blob.data() + pk.dw_w16);
    for (int c = 0; c < Cout; ++c)
      for (int t = 0; t < K * K; ++t) {
        P[(size_t)t * Cout + c] = h2f_bits(W[(size_t)c * K * K + t]);
        P16[(size_t)t * Cout + c] = W[(size_t)c * K * K + t];
      }
  }
}

int conv_resolve(const ConvSpec & s, const ConvPacking & pk, const void * dev_blob, int batch, float * ws,
                 ConvParams & p)
{
  const char * base = static_cast<const char *>(dev_blob);
  p.bias = pk.bias != kNoSeg ? reinterpret_cast<const float *>(base + pk.bias) : nullptr;
  p.w = reinterpret_cast<const __half *>(base + pk.w);
  if (pk.family == kFamDw) {
    p.w2 = reinterpret_cast<const __half *>(base + pk.dw_w16);
    return kLaunchDw;
  }
  if (pk.family == kFamDirect) {
    p.stem_mfma = pk.stem ? 1 : 0;
    if (pk.stem && pk.stem_w2 != kNoSeg) p.w2 = reinterpret_cast<const __half *>(base + pk.stem_w2);
    return kLaunchDirect;
  }
  p.cin8 = pk.cin8;
  p.kpad = pk.kpad;
  p.bk = igemm_bk(p.Cout, p.K * p.K * p.cin8);
  p.ksplit = 1;
  p.ws = nullptr;
  if (ws) {
    p.ksplit = igemm_ksplit((long)batch * p.Ho * p.Wo, p.Cout, p.kpad);
    if (p.ksplit > 1) p.ws = ws;
  }
  if (!s.x_nhwc && !s.x_vec1) {  // 1x1 on NCHW planes (x_planes8): no other kernel applies
    if (p.x.layout != kNCHW || p.x.cs != p.H * p.W || (p.x.cs % 8) || (p.x.img % 8) ||
        (reinterpret_cast<uintptr_t>(p.x.ptr) % 16) || p.K != 1 || p.S != 1 || p.P != 0)
      throw std::runtime_error("implicit-GEMM input view: NCHW planes of 8-pixel pieces expected");
    p.xt = 1;
    // the streaming pointwise kernel with planar output when y is NCHW planes too (the plan's
    // conv1x1 op on graph tensors, Cin <= 64, Cout <= 128).  Measured against the implicit
    // GEMM on MI355X (SiLU, kernel time): 64->128 at 80x80 57.3 -> 32.4 us at batch 64 (2.7 ->
    // 4.9 TB/s), 9.5 -> 5.5 us at batch 1; 64->64 at 80x80 38.8 -> 23.0 us; faster on every
    // shape tried from batch 1 to 64 but 32->64 at 160x160 batch 64 (114 vs 108 us, where both
    // fall to ~2.8 TB/s on a 315 MB footprint).
    if (!(s.flags & IVH_FLAG_NO_PW) && pwt_plan(p)) {
      p.pw = 2;
      p.ksplit = 1;
      p.ws = nullptr;
    }
    return kLaunchIgemm;
  }
  // a 1x1 conv reading a fused 2x upsample (the executor's upsample-concat fusion): the
  // implicit GEMM, the one family with that input
  if (p.cu) {
    if (!upcat_ok(p)) throw std::runtime_error("upsample-concat input geometry");
    return kLaunchIgemm;
  }
  // 1x1 stride 1 with Cout <= 128 on channels-last views: the streaming pointwise kernel of
  // conv_pw.hip when its 32-pixel blocks fill the persistent grid several times over, and
  // where it was measured faster than the implicit GEMM (MI355X, batch 64, kernel trace):
  // every Cout <= 32 (32->32 at 160x160: 37.5 vs 46.4 us, 48->32: 49.2 vs 53.0), Cout <= 64
  // with K <= 96 (64->64 at 80x80: 24.2 vs 25.9, 96->64: 28.8 vs 31.8) or K = 128 at 80x80
  // and up (33.4 vs 35.0).  The implicit GEMM stays faster for 48->64 at 160x160 (99.7 vs
  // 104.0), 192->64 at 80x80 (44.8 vs 47.3) and 128->64 at 40x40 (12.0 vs 13.3).  With
  // 64 < Cout <= 128 (four 32-channel blocks per wave) only for K <= 96: 96->128 at 80x80
  // 53.6 -> 50.6 us, while 128->128 and 192->128 at 40x40 are slower (20.2 -> 23.3, 21.1 ->
  // 23.7 us).
  // 1x1 from channels-last x to NCHW planes (the heads' last convs, whose outputs are graph
  // tensors): the planar-output streaming kernel, measured against the implicit GEMM on
  // MI355X (YOLOv8n-pose heads, batch 64 / 1): 51->51 at 80x80 22.5 -> 18.5 / 5.8 -> 4.6 us,
  // 64->64 at 80x80 23.9 -> 21.9 / 5.4 -> 4.6 us, at 20x20 6.1 -> 5.2 / 6.4 -> 4.0 us.  Not
  // for a single class plane (64->1 at 80x80: 13.4 vs 14.5 us at batch 64), where its 64
  // computed channels are mostly padding.
  if (p.K == 1 && !(s.flags & IVH_FLAG_NO_PW) && p.y.layout == kNCHW && p.Cout >= 16 && pwt_plan(p)) {
    p.pw = 2;
    p.ksplit = 1;
    p.ws = nullptr;
    return kLaunchIgemm;
  }
  const bool pw_wins = p.Cout <= 32 || (p.cin8 <= 96 && p.cin8 != 48) ||
                       (p.Cout <= 64 && p.cin8 > 96 && p.cin8 <= 128 && pw_blocks(p) >= 8192);
  if (p.K == 1 && !(s.flags & IVH_FLAG_NO_PW) && pw_plan(p) && pw_blocks(p) >= kPwMinBlocks && pw_wins) {
    p.pw = 1;
    p.ksplit = 1;
    p.ws = nullptr;
    return kLaunchIgemm;
  }
  // 3x3 stride 1 with Cin % 8 == 0, 64 < Cin, Cout <= 256: the DMA-pipelined persistent
  // kernel on the 32-channel-chunk packing, when its items fill the persistent grid.
  // Measured on MI355X at batch 64 against the LDS-patch kernel: 128->128 at 40x40 46.5 ->
  // 43.0 us, 128->51 / 128->64 at 40x40 28.2 / 27.6 -> 26.1 / 27.1 us; with Cin <= 64 the
  // resident-weight kernel below stays faster (64->64 at 80x80: 44 vs 51 us).
  int hc, th, tw;
  // 3x3 stride 1 with Cin % 32 == 0, Cin >= 128, 64 < Cout <= 256 and SiLU: the wide-layer
  // kernel (one persistent work-group per CU over an equal share of the pixels) on the
  // fragment-ordered packing, when every work-group gets at least two 32-pixel blocks.
  if (p.K == 3 && p.S == 1 && p.P == 1 && !(s.flags & IVH_FLAG_NO_WIDE) && pipe_views_ok(p) &&
      wide_plan(p.Cin, p.Cout, p.H, p.W, batch, p.act, &th, &tw)) {
    const long nblk = (((long)batch * (p.H + 1) - 1) * p.W + 31) / 32;
    if (pk.wide != kNoSeg && pk.wide_bn == 128 && nblk >= 2L * tw) {
      p.wide = 1;
      p.th = th;
      p.tw = tw;
      p.ck = 16;
      p.ksplit = 1;
      p.ws = nullptr;
      p.w = reinterpret_cast<const __half *>(base + pk.wide);
      p.kpad = 9 * p.Cin;
      return kLaunchIgemm;
    }
  }
  const bool pipe_any = (s.flags & IVH_FLAG_PIPE_ANY) != 0;
  if (p.K == 3 && p.S == 1 && p.P == 1 && !(s.flags & IVH_FLAG_NO_PIPE) && (p.Cin > 64 || pipe_any) && p.Cout <= 256 &&
      pipe_views_ok(p) &&
      pipe_plan(p.Cin, p.Cout, p.H, p.W, batch, p.act, &hc, &th, &tw)) {
    const int hi = halo_index(32);
    if (pk.halo[hi] != kNoSeg && pk.kpad_halo[hi] == (p.Cin + 31) / 32 * 9 * 32) {
      ConvParams q = p;
      q.th = th;
      q.tw = tw;
      q.pipe = hc + 1;
      if (pipe_any || pipe_items(q) >= kPipeMinItems) {
        p.pipe = hc + 1;
        p.th = th;
        p.tw = tw;
        p.ck = 32;
        p.ksplit = 1;
        p.ws = nullptr;
        p.w = reinterpret_cast<const __half *>(base + pk.halo[hi]);
        p.kpad = pk.kpad_halo[hi];
        return kLaunchIgemm;
      }
    }
  }
  // 3x3 stride 1 with 16 < Cin <= 64: weights resident in LDS, persistent over pixel tiles.
  // Measured on MI355X at batch 64 against the LDS-patch kernel: faster for every such layer
  // of the YOLO models except a fused residual with Cin <= 32 (32->32 at 80x80 + residual:
  // 35 vs 30 us); with Cin <= 16 the two are even (16->16 at 160x160: 49 vs 51 us).
  if (p.K == 3 && p.S == 1 && p.P == 1 && !(s.flags & IVH_FLAG_NO_RESIDENT) && p.Cin > 16 &&
      !(p.r.ptr && p.Cin <= 32) && res_views_ok(p) &&
      res_plan(p.Cin, p.Cout, p.H, p.W, batch, p.act, !(s.flags & IVH_FLAG_NO_PINGPONG), &hc, &th, &tw)) {
    const int ck = res_ck(p.Cin), hi = halo_index(ck);
    if (pk.halo[hi] != kNoSeg && pk.kpad_halo[hi] == halo_taps(ck) * ck) {
      ConvParams q = p;
      q.th = th;
      q.tw = tw;
      if (res_tiles(q) >= kResMinTiles) {
        p.res = hc + 1;
        p.th = th;
        p.tw = tw;
        p.ck = ck;
        p.ksplit = 1;
        p.ws = nullptr;
        p.w = reinterpret_cast<const __half *>(base + pk.halo[hi]);
        p.kpad = pk.kpad_halo[hi];
        if (p.x.layout != kNHWC || (p.x.cs % 8) || (p.x.img % 8) || (reinterpret_cast<uintptr_t>(p.x.ptr) % 16))
          throw std::runtime_error("implicit-GEMM input view not 16-byte aligned NHWC");
        return kLaunchIgemm;
      }
    }
  }
  // LDS-patch kernel when its grid fills the chip; otherwise im2col (+ split-K)
  if (p.K == 3 && p.S == 1 && p.P == 1 && halo_plan(p.Cin, p.Cout, p.H, p.W, batch, &hc, &th, &tw)) {
    const int ck = halo_cfg_ck(hc, p.Cin), hi = halo_index(ck);
    if (pk.halo[hi] != kNoSeg) {
      ConvParams q = p;
      q.th = th;
      q.tw = tw;
      const long wgs = halo_grid_x(q) * ((p.Cout + halo_bn(hc) - 1) / halo_bn(hc));
      if (wgs >= 160 || p.ksplit == 1) {
        p.halo = hc + 1;
        p.th = th;
        p.tw = tw;
        p.ck = ck;
        p.ksplit = 1;
        p.ws = nullptr;
        p.w = reinterpret_cast<const __half *>(base + pk.halo[hi]);
        p.kpad = pk.kpad_halo[hi];
      }
    }
  }
  // 3x3 stride 2 with 16 or 32 (padded) input channels and Cout <= 64, or 64 input channels
  // and Cout <= 128 (64-channel blocks on the grid's y), no residual: the persistent
  // resident-weight kernel of conv_s2.hip on the implicit-GEMM packing, when its tiles fill
  // the persistent grid several times over.
  const bool act_ok = p.act == kActNone || p.act == kActSiLU || p.act == kActReLU || p.act == kActHSwish;
  if (!p.halo && p.K == 3 && p.S == 2 && p.P == 1 && !(s.flags & IVH_FLAG_NO_S2_PERSIST) && act_ok &&
      (((pk.cin8 == 16 || pk.cin8 == 32) && p.Cout <= 64) || (pk.cin8 == 64 && p.Cout <= 128)) &&
      pk.kpad >= 9 * pk.cin8 && p.Ho == (p.H - 1) / 2 + 1 && p.Wo == (p.W - 1) / 2 + 1 && s2pk_views_ok(p)) {
    const int cfg = pk.cin8 == 64 ? 6 : (pk.cin8 == 16 ? 2 : 4) + (p.Cout > 32 ? 1 : 0);
    ConvParams q = p;
    q.s2 = cfg + 1;
    if (s2pk_tiles(q) >= kS2PkMinTiles) {
      p.s2 = cfg + 1;
      p.th = s2pk_th(cfg);
      p.tw = 16;
      p.ksplit = 1;
      p.ws = nullptr;
      if (p.x.layout != kNHWC || (p.x.cs % 8) || (p.x.img % 8) || (reinterpret_cast<uintptr_t>(p.x.ptr) % 16))
        throw std::runtime_error("implicit-GEMM input view not 16-byte aligned NHWC");
      return kLaunchIgemm;
    }
  }
  // small-channel stride-2 convs: the LDS-patch kernel of conv_s2.hip on the same packing
  int sc;
  if (!p.halo && p.K == 3 && p.S == 2 && p.P == 1 && s2_plan(p.Cin, p.Cout, p.Ho, p.Wo, &sc, &th, &tw) &&
      s2_cfg_ck(sc) == pk.cin8) {
    ConvParams q = p;
    q.th = th;
    q.tw = tw;
    if (s2_grid(q) >= 160 || p.ksplit == 1) {
      p.s2 = sc + 1;
      p.th = th;
      p.tw = tw;
      p.ksplit = 1;
      p.ws = nullptr;
    }
  }
  if (p.x.layout != kNHWC || (p.x.cs % 8) || (p.x.img % 8) || (reinterpret_cast<uintptr_t>(p.x.ptr) % 16))
    throw std::runtime_error("implicit-GEMM input view not 16-byte aligned NHWC");
  if (p.kpad < p.K * p.K * p.cin8 || p.cin8 < p.Cin) throw std::runtime_error("packed weight geometry");
  (void)s;
  return kLaunchIgemm;
}

size_t conv_splitk_floats(const ConvSpec & s, const ConvPacking & pk, int max_batch)
{
  if (pk.family != kFamIgemm) return 0;
  const long hwo = (long)s.Ho() * s.Wo();
  const int bn = igemm_bn(s.Cout);
  const long npad = (long)(s.Cout + bn - 1) / bn * bn;
  size_t need = 0;
  for (int b = 1; b <= max_batch; ++b) {
    const int ks = igemm_ksplit((long)b * hwo, s.Cout, pk.kpad);
    if (ks > 1) need = std::max(need, (size_t)ks * npad * b * hwo);
  }
  return need;
}

}  // namespace ivh
