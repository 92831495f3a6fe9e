// Internal types shared by the host executor and the gfx950 kernels.
//
// Activation storage model (one GPU, batch B as the outer axis):
//   Every activation tensor of the plan describes ONE image (src/PlanModel.cpp:3561-3564
//   read C,H,W from the last three dims and ignore dim 0).  On the device a tensor is a
//   *view* into a root buffer that holds B images back to back:
//     element (b, c, p)  with p = h*W + w  lives at
//        base + b*img + (layout == NHWC ? p*cs + c : c*cs + p)
//   NHWC (channels-last) is the layout the MFMA implicit-GEMM convs read and write: the
//   GEMM K axis (input channels) is contiguous, so operand fragments are 16-byte loads.
//   A channel range of a root (concat write-offset, split) is the same root with base
//   moved by the channel offset; nothing is copied.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>

namespace ivh {

enum Layout : int { kNCHW = 0, kNHWC = 1 };

// Canonical activation codes (include/infvino/KernelFamily.hpp:70-73).
enum Act : int { kActNone = 0, kActSiLU = 1, kActReLU = 2, kActHSwish = 3, kActHSigmoid = 4, kActSigmoid = 5 };

struct View {
  __half * ptr = nullptr;  // image 0, channel 0 of this view
  long img = 0;            // elements between consecutive images (0 = shared by all images)
  int layout = kNCHW;
  int cs = 0;              // NCHW: elements between channels; NHWC: elements between pixels
};

// One convolution launch.  Output pixels of all images form the GEMM M axis.
// Division of unsigned 32-bit n by a run-time invariant d >= 1 through a multiply-high
// (Granlund & Montgomery, "Division by invariant integers using multiplication", 1994,
// round-up variant): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> l for every n < 2^32 (the sum taken in 64 bits).
struct FastDiv {
  unsigned m = 1;
  int l = 0;
};
inline FastDiv fastdiv_make(unsigned d)
{
  FastDiv f;
  while ((1ull << f.l) < d) ++f.l;
  f.m = (unsigned)(((1ull << 32) * ((1ull << f.l) - d)) / d + 1);
  return f;
}

struct ConvParams {
  View x, y, r;              // input, output, residual (r.ptr == nullptr: none)
  const __half * w = nullptr;  // packed weights (layout depends on the kernel family)
  // fp32 bias; for the MFMA families it holds round_up(Cout, 128) entries, zero past Cout,
  // which the epilogues read in 16-byte pieces without a bound check
  const float * bias = nullptr;
  int batch = 1;
  int Cin = 0, H = 0, W = 0;
  int Cout = 0, Ho = 0, Wo = 0;
  int K = 1, S = 1, P = 0, G = 1;  // square kernel, stride, pad, groups
  int act = 0;
  int cin8 = 0;   // input channels rounded up to 8 (im2col K chunking)
  int kpad = 0;   // packed K per output channel, multiple of the K tile
  int bk = 32;    // implicit-GEMM K step (32 / 64); kpad is a multiple of it
  // split-K (implicit GEMM): ksplit > 1 writes fp32 partials [ksplit][Npad][M] to ws and a
  // second kernel reduces them in fixed order and applies the epilogue
  int ksplit = 1;
  float * ws = nullptr;
  // stem MFMA path: w holds fp16 [ceil(Cout/16)*16][32] (k = ci*9 + ky*3 + kx, zero padded);
  // w2 (Cout <= 16) the row-tiled kernel's fp16 [16][64] (k = tap*4 + ci, zero padded)
  int stem_mfma = 0;
  const __half * w2 = nullptr;
  // 3x3 stride-1 pad-1 LDS-patch kernel (conv_halo.hip): halo = tile config + 1 (0: not
  // used), th x tw = output tile of the tall batch image; w is then packed
  // [co][chunk][tap][ck] with ck = halo_cfg_ck(cfg, Cin) and halo_taps(ck) taps per chunk
  int halo = 0;
  int th = 0, tw = 0;
  int ck = 0;  // input-channel chunk of the halo weight packing (16 / 32 / 64)
  // 3x3 stride-1 pad-1 resident-weight kernel (conv_res.hip, Cin <= ck): config + 1 (0: not
  // used); th x tw and ck as for the halo kernel, w the single-chunk halo packing
  int res = 0;
  // 3x3 stride-1 pad-1 DMA-pipelined kernel (conv_pipe.hip, Cin % 8 == 0, Cin >= 32): config
  // + 1 (0: not used); th x tw as for the halo kernel, w the 32-channel-chunk halo packing
  int pipe = 0;
  // 3x3 stride-1 pad-1 wide-layer kernel (conv_wide.hip, Cin % 32 == 0, Cin >= 128): 1 when
  // used; th = 32-pixel blocks per wave and pass, tw = pixel ranges (work-groups per
  // 128-channel group); w the fragment-ordered packing (ConvPacking::wide)
  int wide = 0;
  // channels after the output view's last one that belong to no tensor (the padding of a
  // channels-last root whose last channel range this view is); a kernel may write there
  int ypad = 0;
  // 3x3 stride-2 small-channel kernel (conv_s2.hip): config + 1 (0: not used); th x tw is
  // then the output tile of one image and w the implicit-GEMM packing
  int s2 = 0;
  // 1x1 stride-1 streaming kernel (conv_pw.hip, Cout <= 64, channels-last views): 1 when
  // used; w is then the implicit-GEMM packing
  int pw = 0;
  // implicit GEMM of a 1x1 conv reading NCHW channel planes (x.cs = pixels per plane, a
  // multiple of 8): each thread loads 8 consecutive pixels of one channel and writes them
  // transposed into the tile's pixel rows in LDS (0: channels-last input)
  int xt = 0;
  // implicit GEMM of a 1x1 conv over a channel concat whose first cu channels are a 2x
  // nearest upsample (0: none): those channels are read from xu, channels-last at
  // (H / 2) x (W / 2), at pixel (oy / 2, ox / 2); channels cu.. from x as usual
  View xu;
  int cu = 0;
  // grouped launch (the resident-weight ping-pong kernel): output channel block y (64
  // channels) reads input channels y * xg .. y * xg + Cin - 1 of x (0: every block reads 0..)
  int xg = 0;
  // divisions by Ho * Wo and by Wo (set by the implicit-GEMM launcher)
  FastDiv dv_hwo, dv_wo;
};

// Generic small-op descriptor (elementwise / pooling / data movement).
struct SmallParams {
  View a, b, y;
  View c;                      // a third output (kMaxPoolSppf)
  int batch = 1;
  int C = 0, H = 0, W = 0;     // per-image geometry of the iteration space
  int Ho = 0, Wo = 0;
  int K = 0, S = 1, P = 0;
  int op = 0;
  long n = 0;                  // per-image element count (flat ops)
  int i0 = 0, i1 = 0, i2 = 0, i3 = 0, i4 = 0;  // op-specific integers
  int rank = 0;
  int dims[18] = {0};          // ew_binary broadcast spec (rank <= 6)
};

// Fused attention core (q^T k, * scale, softmax, v P^T) of one node per head batch: q, k
// [heads][kAttnKD][n], v, y [heads][kAttnHD][n] per image, NCHW views with cs = one head's
// block; scale is the plan's fp16 scalar as fp32.
constexpr int kAttnKD = 32, kAttnHD = 64, kAttnMaxN = 512;
struct AttnParams {
  View q, k, v, y;
  int batch = 1, heads = 1, n = 0;
  float scale = 1.0f;
  int scale_q = 0;  // 1: the scale multiplies q (rounded to fp16) before q^T k; 0: the scores
};

// Fused Detect / Pose head decode: per-scale head tensors in, [4 + nc + 3 nk][A] out per image
// (the plan's decode tail, matched by the executor).  Anchor a of scale s is pixel a - off[s]
// of that scale's tensors.
struct DecodeParams {
  View x[4];                      // per scale: box distributions (4R ch)
  View c[4];                      // per scale: class scores (nc ch; may be x's channels 4R..)
  View k[4];                      // per scale: keypoints (3 nk ch; unused when nk == 0)
  View y;                         // [4 + nc + 3 nk][A], channel stride A
  const __half * dflw = nullptr;  // R bin weights of the DFL projection
  const __half * anc = nullptr;   // anchor centres [2][A]
  const __half * st = nullptr;    // strides [A]
  const __half * ancm = nullptr;  // keypoint offsets [2][A] (anchors - 0.5)
  const __half * cbox = nullptr;  // scalar: centre = (x1y1 + x2y2) / cbox (box_div) or * cbox
  const __half * ckpt = nullptr;  // scalar: keypoint xy multiplier
  int off[4] = {0, 0, 0, 0};      // first anchor of each scale
  int nscale = 0, batch = 1, A = 0, R = 0, nc = 0, nk = 0, box_div = 1;
  int nchw = 0;                   // every x / k view is NCHW (the compile-time-count kernels)
};

}  // namespace ivh
