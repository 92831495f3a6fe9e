// Convolution operands on the host side: kernel family choice, weight packing and launch
// resolution, shared by the plan executor and the single-op C ABI.
//
// One conv's packed operands are one blob (bias as fp32, then the weight packings of its
// kernel family) whose layout is a function of the conv's geometry only, so a caller that
// packed a blob can launch on it from the geometry alone.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "ivh_internal.hpp"

namespace ivh {

enum ConvFamily : int { kFamIgemm = 0, kFamDirect = 1, kFamDw = 2 };

// One convolution, per image (the reference's conv1x1 / conv3x3 / conv_general nodes).
struct ConvSpec {
  int Cin = 0, Cout = 0, H = 0, W = 0;
  int K = 1, S = 1, P = 0, G = 1;
  int act = 0;
  bool has_bias = false;
  bool x_nhwc = false;  // input channels-last with 16-byte aligned pixels (MFMA families)
  bool x_vec1 = false;  // single-pixel NCHW input (an FC / GEMV): the MFMA family reads it too
  bool x_planes8 = false;  // 1x1 conv on NCHW input whose planes hold a multiple of 8 pixels:
                           // the MFMA family reads it, transposing pixel pieces in LDS
  uint32_t flags = 0;   // IVH_FLAG_DIRECT_ONLY / IVH_FLAG_NO_HALO
  int Ho() const { return (H + 2 * P - K) / S + 1; }
  int Wo() const { return (W + 2 * P - K) / S + 1; }
};

constexpr size_t kNoSeg = ~(size_t)0;

// Byte offsets of the segments of a packed blob (kNoSeg: absent).
struct ConvPacking {
  int family = kFamDirect;
  size_t bias = kNoSeg;              // fp32 [round_up(Cout, 128) + 16]
  size_t w = kNoSeg;                 // the family's main packing
  int cin8 = 0, kpad = 0;            // implicit GEMM: fp16 [round_up(Cout,128)][kpad]
  size_t halo[3] = {kNoSeg, kNoSeg, kNoSeg};  // 3x3 s1 p1: fp16 [rows][chunk][tap][ck], ck 16/32/64
  int kpad_halo[3] = {0, 0, 0};
  // 3x3 s1 p1 with Cin % 32 == 0, 64 <= Cin, Cout <= 256 (the wide-layer kernel): fp16
  // [Cout / wide_bn groups][Cin / 16][tap][wide_bn / 32][64 lanes][8], every 32 x 16 MFMA A
  // fragment (lane l: output channel l % 32 of its block, input channels 8 (l / 32) ..) as
  // 1 KB in lane order, so the kernel's copies of a chunk read one contiguous range
  size_t wide = kNoSeg;
  int wide_bn = 0;
  bool stem = false;                 // Cin <= 3 3x3: fp16 [ceil(Cout/16)*16][32] ...
  size_t stem_w2 = kNoSeg;           // ... then (Cout <= 16) fp16 [16][64], k = tap*4 + ci
  size_t dw_w16 = kNoSeg;            // depthwise: the same [K][K][C] weights as fp16
  size_t bytes = 0;
};

// Kernel family and blob layout of a conv.
ConvPacking conv_packing(const ConvSpec & s);
// Packs plan-order weights w[Cout][Cin/G][K][K] and bias[Cout] (fp16 bits; bias may be
// null) into a host blob of packing.bytes bytes.
void conv_pack(const ConvSpec & s, const ConvPacking & pk, const uint16_t * w, const uint16_t * bias,
               std::vector<uint8_t> & blob);

enum ConvLaunch : int { kLaunchIgemm = 0, kLaunchDirect = 1, kLaunchDw = 2 };
// Completes p for a launch at `batch` from a device copy of the blob: weights, bias, the
// MFMA kernel and tile choice (LDS-patch kernel, split-K when ws is given and the grid is
// small).  p's views, geometry, act and batch are set by the caller.  Returns the launcher.
int conv_resolve(const ConvSpec & s, const ConvPacking & pk, const void * dev_blob, int batch, float * ws,
                 ConvParams & p);

// Largest split-K workspace (floats) a conv needs at batch sizes 1..max_batch.
size_t conv_splitk_floats(const ConvSpec & s, const ConvPacking & pk, int max_batch);

}  // namespace ivh
