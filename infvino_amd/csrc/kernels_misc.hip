// Bandwidth-bound gfx950 kernels: direct conv (stem Cin<8, grouped, NCHW-input convs),
// depthwise conv, the small ops of kernels/ops.cl, and the boundary conversions.
// None of these use MFMA; they are written for coalesced HBM access with batch B as an
// outer grid axis.  Element addressing goes through ivh::View (NCHW or NHWC, strided).
#include "conv_common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <type_traits>
#include <initializer_list>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>

namespace ivh {

__device__ __forceinline__ long vidx(const View & v, int b, int c, long p)
{
  return (long)b * v.img + (v.layout == kNHWC ? p * v.cs + c : (long)c * v.cs + p);
}
__device__ __forceinline__ float vld(const View & v, int b, int c, long p)
{
  return (float)reinterpret_cast<const _Float16 *>(v.ptr)[vidx(v, b, c, p)];
}
__device__ __forceinline__ void vst(const View & v, int b, int c, long p, float x)
{
  reinterpret_cast<_Float16 *>(v.ptr)[vidx(v, b, c, p)] = (_Float16)x;
}

static inline unsigned nblk(long n, int t) { return (unsigned)((n + t - 1) / t); }

// ------------------------------------------------------------------ direct conv
// Restates conv_general (kernels/conv_general.cl:7-48) / conv3x3_cin3 (conv_cin3.cl:67-118):
// one lane = one output pixel x COB output channels of one group, fp32 accumulation.
// Weights packed fp32 [G][cin_g][K][K][cout_g] so every lane of a wave reads the same
// weight addresses (uniform, scalar-cache friendly).
template <int COB>
__global__ void __launch_bounds__(256) conv_direct_kernel(const ConvParams p)
{
  const int HWo = p.Ho * p.Wo;
  const long Mt = (long)p.batch * HWo;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int cout_g = p.Cout / p.G, cin_g = p.Cin / p.G;
  const int ncb = (cout_g + COB - 1) / COB;
  if (idx >= Mt * ncb * p.G) return;
  const long pix = idx % Mt;
  const int cbg = (int)(idx / Mt);
  const int g = cbg / ncb, cb = cbg % ncb;
  const int b = (int)(pix / HWo), hw = (int)(pix % HWo);
  const int oy = hw / p.Wo, ox = hw % p.Wo;
  const int col = cb * COB;  // first channel within the group
  const float * W = reinterpret_cast<const float *>(p.w);
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = 0.0f;
  for (int cl = 0; cl < cin_g; ++cl) {
    const int c = g * cin_g + cl;
    for (int ky = 0; ky < p.K; ++ky) {
      const int iy = oy * p.S - p.P + ky;
      if ((unsigned)iy >= (unsigned)p.H) continue;
      for (int kx = 0; kx < p.K; ++kx) {
        const int ix = ox * p.S - p.P + kx;
        if ((unsigned)ix >= (unsigned)p.W) continue;
        const float xv = vld(p.x, b, c, (long)iy * p.W + ix);
        const float * wp = W + (((long)(g * cin_g + cl) * p.K + ky) * p.K + kx) * cout_g + col;
#pragma unroll
        for (int j = 0; j < COB; ++j) acc[j] += xv * wp[j];
      }
    }
  }
  float out[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) {
    const int co = g * cout_g + col + j;
    float v = acc[j] + ((p.bias && col + j < cout_g) ? p.bias[co] : 0.0f);
    v = act_f(v, p.act);
    if (p.r.ptr && col + j < cout_g) v += vld(p.r, b, co, hw);
    out[j] = v;
  }
  const int co0 = g * cout_g + col;
  _Float16 * yb = reinterpret_cast<_Float16 *>(p.y.ptr);
  if (COB % 8 == 0 && p.y.layout == kNHWC && col + COB <= cout_g &&
      (((p.y.cs | (int)p.y.img | co0 | (int)(reinterpret_cast<uintptr_t>(yb) >> 1)) & 7) == 0)) {
#pragma unroll
    for (int j = 0; j < COB; j += 8) {
      h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (_Float16)out[j + e];
      *reinterpret_cast<h8 *>(yb + (long)b * p.y.img + (long)hw * p.y.cs + co0 + j) = v;
    }
  } else {
#pragma unroll
    for (int j = 0; j < COB; ++j)
      if (col + j < cout_g) vst(p.y, b, co0 + j, hw, out[j]);
  }
}


// Stem convolution with few input channels (conv3x3_cin3, kernels/conv_cin3.cl:67-118) on
// fp16 MFMA: K = Cin*9 taps padded to 32, one v_mfma_f32_16x16x32_f16 per 16 output pixels
// and 16 output channels.  Operand A (weights, [co][k], k = ci*9 + ky*3 + kx exactly the
// plan's [Cout][Cin][3][3] order) is loaded once per lane; operand B is gathered straight
// from the input (im2col in registers).  D layout: lane holds pixel lane%16 and channels
// 4*(lane/16) + 0..3, so a wave stores 16 pixels x 32 bytes contiguously (channels-last).
typedef _Float16 h8s __attribute__((ext_vector_type(8)));
typedef float f4s __attribute__((ext_vector_type(4)));
typedef _Float16 h4s __attribute__((ext_vector_type(4)));

template <int NT, bool NCHW_IN>
__global__ void __launch_bounds__(256) conv_stem_mfma_kernel(const ConvParams p)
{
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int HWo = p.Ho * p.Wo;
  const int taps = p.Cin * 9;
  const _Float16 * W = reinterpret_cast<const _Float16 *>(p.w);  // [NT*16][32]
  h8s afrag[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    afrag[t] = *reinterpret_cast<const h8s *>(W + (t * 16 + (lane & 15)) * 32 + (lane >> 4) * 8);
  const _Float16 * xb = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img;
  _Float16 * yb = reinterpret_cast<_Float16 *>(p.y.ptr);
  const bool vec = p.y.layout == kNHWC && ((p.y.cs | (int)p.y.img | (int)(reinterpret_cast<uintptr_t>(yb) >> 1)) & 3) == 0;
  // this wave: 4 groups of 16 consecutive output pixels
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int pix = (blockIdx.x * 4 + wave) * 64 + g * 16 + (lane & 15);
    const bool pvalid = pix < HWo;
    const int oy = pix / p.Wo, ox = pix - oy * p.Wo;
    const int iy0 = oy * p.S - p.P, ix0 = ox * p.S - p.P;
    h8s bfrag;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = (lane >> 4) * 8 + e;
      float v = 0.0f;
      if (pvalid && k < taps) {
        const int ci = k / 9, r = k - ci * 9, ky = r / 3, kx = r - ky * 3;
        const int iy = iy0 + ky, ix = ix0 + kx;
        if ((unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W) {
          const int q = iy * p.W + ix;
          v = (float)xb[NCHW_IN ? (long)ci * p.x.cs + q : (long)q * p.x.cs + ci];
        }
      }
      bfrag[e] = (_Float16)v;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f4s acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag[t], bfrag, acc, 0, 0, 0);
      if (!pvalid) continue;
      const int co0 = t * 16 + (lane >> 4) * 4;
      float o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int co = co0 + v;
        float x = acc[v] + (co < p.Cout && p.bias ? p.bias[co] : 0.0f);
        x = act_f(x, p.act);
        if (p.r.ptr && co < p.Cout) x += vld(p.r, b, co, pix);
        o[v] = x;
      }
      if (vec && co0 + 4 <= p.Cout) {
        h4s hv;
#pragma unroll
        for (int v = 0; v < 4; ++v) hv[v] = (_Float16)o[v];
        *reinterpret_cast<h4s *>(yb + (long)b * p.y.img + (long)pix * p.y.cs + co0) = hv;
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (co0 + v < p.Cout) vst(p.y, b, co0 + v, pix, o[v]);
      }
    }
  }
}

// 1x1 conv with few output channels on planar (NCHW) input and output -- the DFL
// projection of the pose head (16 bins -> 1), conv_general.cl:7-48 semantics: one lane =
// 8 consecutive pixels x all Cout (<= 8), 16-byte loads per input channel, fp32 weights
// [Cin][Cout] read uniformly, fp32 accumulation.
template <int COUT>
__global__ void __launch_bounds__(256) conv1x1_nchw8_kernel(const ConvParams p)
{
  const int HW = p.H * p.W, P8 = HW >> 3;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (t >= P8) return;
  const int p0 = t * 8;
  const float * W = reinterpret_cast<const float *>(p.w);
  float acc[COUT][8];
#pragma unroll
  for (int c = 0; c < COUT; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[c][e] = 0.0f;
  const _Float16 * xb = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img + p0;
  for (int ci = 0; ci < p.Cin; ++ci) {
    const h8 xv = *reinterpret_cast<const h8 *>(xb + (long)ci * p.x.cs);
#pragma unroll
    for (int c = 0; c < COUT; ++c) {
      const float w = c < p.Cout ? W[ci * p.Cout + c] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[c][e] += w * (float)xv[e];
    }
  }
#pragma unroll
  for (int c = 0; c < COUT; ++c) {
    if (c >= p.Cout) break;
    const float bv = p.bias ? p.bias[c] : 0.0f;
    h8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (_Float16)act_f(acc[c][e] + bv, p.act);
    if (p.r.ptr) {
      const h8 rv = *reinterpret_cast<const h8 *>(reinterpret_cast<const _Float16 *>(p.r.ptr) + (long)b * p.r.img +
                                                  (long)c * p.r.cs + p0);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)rv[e]);
    }
    *reinterpret_cast<h8 *>(reinterpret_cast<_Float16 *>(p.y.ptr) + (long)b * p.y.img + (long)c * p.y.cs + p0) = v;
  }
}

bool conv1x1_nchw8_ok(const ConvParams & p)
{
  auto a8 = [](const View & v) {
    return v.layout == kNCHW && ((v.cs | v.img | (long)(reinterpret_cast<uintptr_t>(v.ptr) >> 1)) & 7) == 0;
  };
  return p.K == 1 && p.S == 1 && p.P == 0 && p.G == 1 && p.Cout <= 8 && p.H == p.Ho && p.W == p.Wo &&
         ((long)p.H * p.W) % 8 == 0 && a8(p.x) && a8(p.y) && (!p.r.ptr || a8(p.r));
}

// Row-tiled stem for the common case (kernels/conv_cin3.cl:67-118 semantics): 3x3 stride 2
// pad 1, Cin <= 3, Cout <= 16, planar NCHW input, channels-last output, no residual.  A
// work-group owns TR output rows of one image.  It stages the 2*TR+1 input rows it needs in
// LDS as [row][col][4] (channels interleaved, 4th slot zero; two zero columns on each side
// for the padding), loading each channel plane with 16-byte coalesced loads.  Each wave then
// takes 16-pixel blocks: K = 9 taps x 4 channel slots (36, two 16x16x32 MFMAs: taps 0-7 and
// tap 8), B fragments are two 8-byte LDS reads per lane, weights ([16][64], k = tap*4 + ci)
// stay in registers, and the D layout gives each lane 4 consecutive channels of one pixel,
// so a block is 16 pixels x 32 bytes written contiguously.
template <int TR, int UIT, int ACT>
__global__ void __launch_bounds__(256) conv_stem_rows_kernel(const ConvParams p)
{
  extern __shared__ __attribute__((aligned(16))) _Float16 srow[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD-aware order over (row tile, image): consecutive row tiles share an input row
  const int lin = xcd_tile(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
  const int b = lin / gridDim.x, oy0 = (lin % gridDim.x) * TR;
  const int W = p.W, LW = W + 4;               // LDS row: 2 pad columns each side
  const int G = W >> 3;                        // 8-pixel column groups per input row
  const float inv_g = __builtin_amdgcn_rcpf((float)G);
  const _Float16 * xb = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img;
  // zero the pad columns of every staged row
  for (int e = tid; e < (2 * TR + 1) * 4; e += 256) {
    const int lr = e >> 2, c = e & 3;
    const int col = c < 2 ? c : W + c;
    *reinterpret_cast<h4s *>(srow + ((long)lr * LW + col) * 4) = h4s{};
  }
  // every load of this thread is issued before the first LDS store (UIT units of three
  // 16-byte channel loads; the host keeps (2*TR+1)*W/8 <= 256*UIT)
  h8s c[UIT][3];
  int dsto[UIT];
#pragma unroll
  for (int i = 0; i < UIT; ++i) {
    const int u = tid + 256 * i;
    const int lr = idiv_small(u, G, inv_g), g = u - lr * G;
    const int iy = 2 * oy0 - 1 + lr;
    dsto[i] = u < (2 * TR + 1) * G ? (lr * LW + 8 * g + 2) * 4 : -1;
    const bool ok = dsto[i] >= 0 && iy >= 0 && iy < p.H;
#pragma unroll
    for (int ci = 0; ci < 3; ++ci)
      c[i][ci] = (ok && ci < p.Cin) ? *reinterpret_cast<const h8s *>(xb + (long)ci * p.x.cs + (long)iy * W + 8 * g) : h8s{};
  }
#pragma unroll
  for (int i = 0; i < UIT; ++i) {
    if (dsto[i] < 0) continue;
    _Float16 * dst = srow + dsto[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h8s v;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v[4 * h + 0] = c[i][0][2 * j + h];
        v[4 * h + 1] = c[i][1][2 * j + h];
        v[4 * h + 2] = c[i][2][2 * j + h];
        v[4 * h + 3] = (_Float16)0.0f;
      }
      *reinterpret_cast<h8s *>(dst + 8 * j) = v;
    }
  }
  __syncthreads();

  // lane: output pixel (lane & 15) of a 16-pixel block, K group q = lane >> 4 (taps 2q and
  // 2q + 1 of the first MFMA; q == 0 also feeds tap 8 to the second); D gives it channels
  // 4q .. 4q+3 of its pixel
  const int co = lane & 15, q = lane >> 4;
  const _Float16 * W4 = reinterpret_cast<const _Float16 *>(p.w2);
  const h8s a1 = *reinterpret_cast<const h8s *>(W4 + co * 64 + 8 * q);
  const h8s a2 = *reinterpret_cast<const h8s *>(W4 + co * 64 + 32 + 8 * q);
  float bias[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) bias[v] = (p.bias && 4 * q + v < p.Cout) ? p.bias[4 * q + v] : 0.0f;
  // LDS offsets (halves) of the lane's taps relative to its pixel's window corner
  const int ta = 2 * q, tb = 2 * q + 1;
  const int off0 = ((ta / 3) * LW + ta % 3) * 4, off1 = ((tb / 3) * LW + tb % 3) * 4;
  const int off8 = (2 * LW + 2) * 4;
  const int CB = (p.Wo + 15) >> 4;
  const int px = lane & 15;
  _Float16 * const yb = reinterpret_cast<_Float16 *>(p.y.ptr) + (long)b * p.y.img + 4 * q;
  const bool full = 4 * q + 4 <= p.Cout;
  // blocks (output row r, 16-pixel column block cb); wave w takes cb = w, w + 4, ... four
  // blocks per pass: all LDS fragment reads first, then the MFMAs and the stores
  for (int r = 0; r < TR; ++r) {
    const int oy = oy0 + r;
    if (oy >= p.Ho) break;
    const _Float16 * const rbase = srow + (2 * r * LW + 1) * 4;
    _Float16 * const yrow = yb + (long)oy * p.Wo * p.y.cs;
    for (int cb0 = wave; cb0 < CB; cb0 += 16) {
      h8s b1[4], b2[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int cb = cb0 + 4 * k < CB ? cb0 + 4 * k : cb0;
        const int ox = cb * 16 + px;
        const _Float16 * src = rbase + 8 * (ox < p.Wo ? ox : p.Wo - 1);
        const h4s t0 = *reinterpret_cast<const h4s *>(src + off0);
        const h4s t1 = *reinterpret_cast<const h4s *>(src + off1);
        const h4s t8 = q == 0 ? *reinterpret_cast<const h4s *>(src + off8) : h4s{};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          b1[k][e] = t0[e];
          b1[k][4 + e] = t1[e];
          b2[k][e] = t8[e];
          b2[k][4 + e] = (_Float16)0.0f;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f4s acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1[k], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b2[k], acc, 0, 0, 0);
        const int ox = (cb0 + 4 * k) * 16 + px;
        if (cb0 + 4 * k >= CB || ox >= p.Wo) continue;
        _Float16 * yp = yrow + (long)ox * p.y.cs;
        if (full) {
          h4s hv;
#pragma unroll
          for (int v = 0; v < 4; ++v) hv[v] = (_Float16)act_fast<ACT>(acc[v] + bias[v]);
          *reinterpret_cast<h4s *>(yp) = hv;
        } else {
          for (int v = 0; v < 4 && 4 * q + v < p.Cout; ++v) yp[v] = (_Float16)act_fast<ACT>(acc[v] + bias[v]);
        }
      }
    }
  }
}

constexpr int kStemTR = 2, kStemUIT = 2;

// LDS bytes of the row-tiled stem for an input width
static long stem_rows_lds(int W) { return (long)(2 * kStemTR + 1) * (W + 4) * 8; }

bool stem_rows_supported(const ConvParams & p)
{
  auto al = [](const void * ptr, int bytes) { return (reinterpret_cast<uintptr_t>(ptr) % bytes) == 0; };
  return p.stem_mfma && p.w2 && p.K == 3 && p.S == 2 && p.P == 1 && p.G == 1 && p.Cin >= 1 && p.Cin <= 3 &&
         p.Cout <= 16 && !p.r.ptr && p.x.layout == kNCHW && p.y.layout == kNHWC && (p.W % 8) == 0 &&
         (p.x.cs % 8) == 0 && (p.x.img % 8) == 0 && al(p.x.ptr, 16) && (p.y.cs % 4) == 0 && (p.y.img % 4) == 0 &&
         al(p.y.ptr, 8) && p.Ho == (p.H - 1) / 2 + 1 && p.Wo == (p.W - 1) / 2 + 1 && stem_rows_lds(p.W) <= 65536 &&
         (2 * kStemTR + 1) * (p.W / 8) <= 256 * kStemUIT;
}

bool stem_supported(const ConvParams & p)
{
  return p.K == 3 && p.G == 1 && p.Cin >= 1 && p.Cin <= 3 && p.Cout <= 32 && p.stem_mfma;
}

void launch_conv_direct(const ConvParams & p, hipStream_t s)
{
  if (stem_rows_supported(p)) {
    const dim3 grid((unsigned)((p.Ho + kStemTR - 1) / kStemTR), (unsigned)p.batch);
    const size_t lds = (size_t)stem_rows_lds(p.W);
    switch (p.act) {
    case kActSiLU: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActSiLU>), grid, dim3(256), lds, s, p); break;
    case kActReLU: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActReLU>), grid, dim3(256), lds, s, p); break;
    case kActHSwish: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActHSwish>), grid, dim3(256), lds, s, p); break;
    case kActHSigmoid: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActHSigmoid>), grid, dim3(256), lds, s, p); break;
    case kActSigmoid: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActSigmoid>), grid, dim3(256), lds, s, p); break;
    default: hipLaunchKernelGGL((conv_stem_rows_kernel<kStemTR, kStemUIT, kActNone>), grid, dim3(256), lds, s, p); break;
    }
    return;
  }
  if (stem_supported(p)) {
    const dim3 grid(nblk((long)p.Ho * p.Wo, 256), (unsigned)p.batch);
    const bool nchw = p.x.layout == kNCHW;
    if (p.Cout <= 16) {
      if (nchw) hipLaunchKernelGGL((conv_stem_mfma_kernel<1, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((conv_stem_mfma_kernel<1, false>), grid, dim3(256), 0, s, p);
    } else {
      if (nchw) hipLaunchKernelGGL((conv_stem_mfma_kernel<2, true>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((conv_stem_mfma_kernel<2, false>), grid, dim3(256), 0, s, p);
    }
    return;
  }
  if (conv1x1_nchw8_ok(p)) {
    const dim3 grid(nblk((long)p.H * p.W / 8, 256), (unsigned)p.batch);
    if (p.Cout <= 1) hipLaunchKernelGGL(conv1x1_nchw8_kernel<1>, grid, dim3(256), 0, s, p);
    else if (p.Cout <= 4) hipLaunchKernelGGL(conv1x1_nchw8_kernel<4>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(conv1x1_nchw8_kernel<8>, grid, dim3(256), 0, s, p);
    return;
  }
  const int cout_g = p.Cout / p.G;
  const long Mt = (long)p.batch * p.Ho * p.Wo;
  if (cout_g < 4) {
    const long n = Mt * cout_g * p.G;
    hipLaunchKernelGGL(conv_direct_kernel<1>, dim3(nblk(n, 256)), dim3(256), 0, s, p);
  } else if (cout_g % 16 == 0 || (p.G == 1 && cout_g > 8)) {
    const long n = Mt * ((cout_g + 15) / 16) * p.G;
    hipLaunchKernelGGL(conv_direct_kernel<16>, dim3(nblk(n, 256)), dim3(256), 0, s, p);
  } else if (cout_g % 8 == 0 || p.G == 1) {
    const long n = Mt * ((cout_g + 7) / 8) * p.G;
    hipLaunchKernelGGL(conv_direct_kernel<8>, dim3(nblk(n, 256)), dim3(256), 0, s, p);
  } else {
    const long n = Mt * cout_g * p.G;
    hipLaunchKernelGGL(conv_direct_kernel<1>, dim3(nblk(n, 256)), dim3(256), 0, s, p);
  }
}

// ------------------------------------------------------------------- depthwise
// Restates depthwise_f16 / depthwise_v / depthwise_blk (kernels/conv_general.cl:85-187,
// depthwise_blk.cl:118-228): y[c] = act(sum_k x[c]*w[c] + b[c]), K in {3,5}, S in {1,2}.
//
// Channels-last tiled kernel.  A tile is TOH x TOW output pixels x 8G channels of one
// image; its input window with the halo, ((TOH-1)S+K) x ((TOW-1)S+K) pixels x 8G channels,
// is loaded into LDS with 16-byte buffer loads (consecutive lanes read consecutive 16-byte
// pieces of the NHWC rows; pixels outside the image are loads past the buffer's range,
// which return zeros, so the taps need no bound checks), together with the tile's
// [K][K][8G] fp16 weights.  Each lane computes a PY x PX block of output pixels for 8
// channels: its K*K weights stay in registers, each input row of its block is read from LDS
// once and applied to every output row and column that uses it (sliding window), with fp32
// accumulation (fp16 operands into v_fma_mix_f32) in (ky, kx) order.
//
// One work-group per tile.  Measured on MI355X, this beats a persistent grid that double-
// buffers the window (two work-groups per CU, the next tile's loads in flight during the
// FMAs): the FMAs and LDS reads need more waves per SIMD than that leaves to hide their
// latencies, and several single-tile work-groups per CU overlap one's loads with another's
// FMAs anyway.
struct DwTile {
  int G, BX, BY;      // 8-channel groups per tile; lane blocks along x and y
  int ntx, nty, nct;  // tiles along x, along y, channel tiles
  int IW, IH;         // input window of a tile, pixels
};

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// acc + a.h * b.h in fp32 with one rounding, a and b fp16 halves (h = 0: low, 1: high) of
// one dword each: v_fma_mix_f32 converts its fp16 operands exactly, so this equals
// fmaf((float)a.h, (float)b.h, acc).  Written out because the compiler otherwise converts
// every register-resident weight to fp32 once (8 more VGPRs per tap) and uses v_fmac_f32.
template <int H>
__device__ __forceinline__ void fma_mix(float & acc, unsigned a, unsigned b)
{
  if (H == 0) asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,1,0]" : "+v"(acc) : "v"(a), "v"(b));
  else asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "+v"(acc) : "v"(a), "v"(b));
}

// LDS pieces (16 bytes) of the depthwise window and weights: at most kDwMaxIt per lane, all
// loaded into registers before the first LDS store (64 KiB)
constexpr int kDwMaxIt = 16;
constexpr int kDwBufPieces = kDwMaxIt * 256;
constexpr int kDwMaxW = 4;  // weight pieces per lane: K*K*G <= 1024

template <int K, int S, int PX, int PY, int ACT>
__global__ void __launch_bounds__(256) dw_tile_kernel(const ConvParams p, const DwTile t)
{
  extern __shared__ __align__(16) unsigned char dw_lds[];
  constexpr int NX = (PX - 1) * S + K;  // input columns of a lane's block
  constexpr int NR = (PY - 1) * S + K;  // input rows of a lane's block
  const int tid = threadIdx.x, G = t.G;
  const int npix = t.IH * t.IW * G;  // window pieces
  int w = blockIdx.x;
  const int tx = w % t.ntx;
  w /= t.ntx;
  const int ty = w % t.nty;
  w /= t.nty;
  const int tc = w % t.nct, b = w / t.nct;
  const int ox0 = tx * t.BX * PX, oy0 = ty * t.BY * PY;
  const int ix0 = ox0 * S - p.P, iy0 = oy0 * S - p.P, c0 = tc * G * 8;

  // this image's input view from channel c0 on, up to its last element
  const __half * xb = p.x.ptr + (long)b * p.x.img + c0;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(xb), (short)0, (int)((((long)p.H * p.W - 1) * p.x.cs + p.Cin - c0) * 2), kBufDword3);
  const h8 * wg = reinterpret_cast<const h8 *>(p.w2) + tc * G;
  h8 * const xs = reinterpret_cast<h8 *>(dw_lds);  // [IH][IW][G] window pieces, then [K*K][G] weights
  // window piece i = tid + 256 u: row i / RP of the window, piece rem = i % RP of that row
  // (column rem / G, group rem % G); pieces outside the image load from past the buffer
  const int RP = t.IW * G, nit = (npix + 255) >> 8;
  const float inv_rp = __builtin_amdgcn_rcpf((float)RP), inv_g = __builtin_amdgcn_rcpf((float)G);
  const int jlo = max(0, -ix0) * G, jhi = (p.W - ix0) * G;  // a row's pieces inside the image
  // byte offsets: window origin (may be negative; only in-image pieces use it), one image row,
  // one pixel; 24-bit multiplies (full rate) suffice, the host keeps an image below 2^31 bytes
  // and its pixel count below 2^24
  const int base0 = (iy0 * p.W + ix0) * p.x.cs * 2, rowb = p.W * p.x.cs * 2, pixb = p.x.cs * 2;
  h8 v[kDwMaxIt];
  auto load_window = [&](auto contig) {
#pragma unroll
    for (int u = 0; u < kDwMaxIt; ++u) {
      if (u < nit) {
        const int i = tid + u * 256;
        const int row = idiv_small(i, RP, inv_rp), rem = i - (int)__umul24(row, RP), iy = iy0 + row;
        int off = base0 + (int)__umul24(row, rowb);
        if (decltype(contig)::value) {
          off += rem * 16;  // whole pixels: the window row is one run of RP pieces
        } else {
          const int col = idiv_small(rem, G, inv_g);
          off += (int)__umul24(col, pixb) + (rem - (int)__umul24(col, G)) * 16;
        }
        const bool in = i < npix && (unsigned)iy < (unsigned)p.H && rem >= jlo && rem < jhi;
        v[u] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, in ? (unsigned)off : kBufOOB, 0, 0));
      }
    }
  };
  if (p.x.cs == 8 * G) load_window(std::true_type{});
  else load_window(std::false_type{});
  // weights: K*K*G pieces (at most kDwMaxW per lane)
  const int nw = K * K * G;
  h8 wv[kDwMaxW];
#pragma unroll
  for (int u = 0; u < kDwMaxW; ++u) {
    const int i = tid + u * 256;
    if (i < nw) {
      const int tap = idiv_small(i, G, inv_g);
      wv[u] = wg[(int)__umul24(tap, p.Cin >> 3) + i - (int)__umul24(tap, G)];
    }
  }
#pragma unroll
  for (int u = 0; u < kDwMaxIt; ++u) {
    const int i = tid + u * 256;
    if (u < nit && (u < nit - 1 || i < npix)) xs[i] = v[u];
  }
#pragma unroll
  for (int u = 0; u < kDwMaxW; ++u)
    if (tid + u * 256 < nw) xs[npix + tid + u * 256] = wv[u];
  __syncthreads();
  if (tid >= G * t.BX * t.BY) return;

  const int q = tid / G, g = tid - q * G;
  const int by = q / t.BX, bx = q - by * t.BX;
  u32x4 wr[K * K];
#pragma unroll
  for (int k = 0; k < K * K; ++k) wr[k] = __builtin_bit_cast(u32x4, xs[npix + k * G + g]);
  float acc[PY][PX][8];
#pragma unroll
  for (int i = 0; i < PY; ++i)
#pragma unroll
    for (int j = 0; j < PX; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i][j][e] = 0.0f;
  const h8 * base = xs + ((by * PY * S) * t.IW + bx * PX * S) * G + g;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    u32x4 xv[NX];
#pragma unroll
    for (int c = 0; c < NX; ++c) xv[c] = __builtin_bit_cast(u32x4, base[(r * t.IW + c) * G]);
#pragma unroll
    for (int i = 0; i < PY; ++i) {
      const int ky = r - i * S;
      if (ky < 0 || ky >= K) continue;
#pragma unroll
      for (int kx = 0; kx < K; ++kx)
#pragma unroll
        for (int j = 0; j < PX; ++j)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            fma_mix<0>(acc[i][j][2 * d], xv[j * S + kx][d], wr[ky * K + kx][d]);
            fma_mix<1>(acc[i][j][2 * d + 1], xv[j * S + kx][d], wr[ky * K + kx][d]);
          }
    }
  }

  const int c = c0 + g * 8;
  float bv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (p.bias) {
    const float4 b0 = *reinterpret_cast<const float4 *>(p.bias + c), b1 = *reinterpret_cast<const float4 *>(p.bias + c + 4);
    bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
    bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
  }
  _Float16 * yb = reinterpret_cast<_Float16 *>(p.y.ptr) + (long)b * p.y.img + c;
  const _Float16 * rb = p.r.ptr ? reinterpret_cast<const _Float16 *>(p.r.ptr) + (long)b * p.r.img + c : nullptr;
#pragma unroll
  for (int i = 0; i < PY; ++i) {
    const int oy = oy0 + by * PY + i;
#pragma unroll
    for (int j = 0; j < PX; ++j) {
      const int ox = ox0 + bx * PX + j;
      if (oy >= p.Ho || ox >= p.Wo) continue;
      const long hw = (long)oy * p.Wo + ox;
      h8 out;
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = (_Float16)act_fast<ACT>(acc[i][j][e] + bv[e]);
      if (rb) {  // act, one rounding, then the residual (the reference order)
        const h8 rv = *reinterpret_cast<const h8 *>(rb + hw * p.r.cs);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (_Float16)((float)out[e] + (float)rv[e]);
      }
      *reinterpret_cast<h8 *>(yb + hw * p.y.cs) = out;
    }
  }
}

// Strip kernel for the 5x5 stride-2 layers at large batch: one lane = 8 channels x a strip
// of PX = 4 output pixels of one row, straight from global memory (L1/L2) into registers,
// each loaded input column reused by the strip's taps, no LDS.  With stride 2 the tiled
// kernel's window is about 4x its output tile and every tap is an LDS read; measured on
// MI355X (72 channels, 28x28 -> 14x14, batch 256) this kernel takes 11.7 us against the
// tiled kernel's 15.5, while at batch 64 the tiled kernel wins (6.7 against 7.5 us).
template <int K, int S, int PX, int ACT>
__global__ void __launch_bounds__(256) dw_strip_kernel(const ConvParams p, FastDiv d_c8, FastDiv d_strip, FastDiv d_ho)
{
  // lane = (8-channel group, strip of PX output pixels of one row), channel groups fastest so
  // that neighbouring lanes read and write neighbouring 16-byte pieces
  constexpr int NX = (PX - 1) * S + K;  // input columns of a strip
  const int C8 = p.Cin >> 3, nstrip = (p.Wo + PX - 1) / PX;
  const unsigned idx = blockIdx.x * 256u + threadIdx.x;
  const unsigned q = fastdiv(idx, d_c8), rowi = fastdiv(q, d_strip), b = fastdiv(rowi, d_ho);
  if (b >= (unsigned)p.batch) return;
  const int c8 = (int)(idx - q * C8), strip = (int)(q - rowi * nstrip), oy = (int)(rowi - b * p.Ho);
  const int c = c8 * 8, ox0 = strip * PX, ix0 = ox0 * S - p.P;
  const _Float16 * xb = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img + c;
  const _Float16 * W = reinterpret_cast<const _Float16 *>(p.w2) + c;
  float acc[PX][8];
#pragma unroll
  for (int j = 0; j < PX; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
#pragma unroll
  for (int ky = 0; ky < K; ++ky) {
    const int iy = oy * S - p.P + ky;
    if ((unsigned)iy >= (unsigned)p.H) continue;
    const _Float16 * xr = xb + (long)iy * p.W * p.x.cs;
    h8 xv[NX];
#pragma unroll
    for (int t = 0; t < NX; ++t) {
      const int ix = ix0 + t;
      xv[t] = (unsigned)ix < (unsigned)p.W ? *reinterpret_cast<const h8 *>(xr + (long)ix * p.x.cs) : h8{};
    }
#pragma unroll
    for (int kx = 0; kx < K; ++kx) {
      const h8 wv = *reinterpret_cast<const h8 *>(W + (ky * K + kx) * p.Cin);
#pragma unroll
      for (int j = 0; j < PX; ++j) {
        const h8 v = xv[j * S + kx];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] += (float)v[e] * (float)wv[e];
      }
    }
  }
  float bv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (p.bias) {
    const float4 b0 = *reinterpret_cast<const float4 *>(p.bias + c), b1 = *reinterpret_cast<const float4 *>(p.bias + c + 4);
    bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
    bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
  }
  _Float16 * yb = reinterpret_cast<_Float16 *>(p.y.ptr) + (long)b * p.y.img + c;
  const _Float16 * rb = p.r.ptr ? reinterpret_cast<const _Float16 *>(p.r.ptr) + (long)b * p.r.img + c : nullptr;
#pragma unroll
  for (int j = 0; j < PX; ++j) {
    const int ox = ox0 + j;
    if (PX > 1 && ox >= p.Wo) break;
    const long hw = (long)oy * p.Wo + ox;
    h8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)act_fast<ACT>(acc[j][e] + bv[e]);
    if (rb) {  // act, one rounding, then the residual (the reference order)
      const h8 rv = *reinterpret_cast<const h8 *>(rb + hw * p.r.cs);
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = (_Float16)((float)out[e] + (float)rv[e]);
    }
    *reinterpret_cast<h8 *>(yb + hw * p.y.cs) = out;
  }
}

// Any-layout depthwise: one lane = one output pixel of one channel plane, grid (pixel
// blocks, channel, image) so that the channel's weights are wave-uniform (scalar loads) and,
// on NCHW tensors, neighbouring lanes read neighbouring pixels.  Same tap order and roundings
// as the channels-last kernels: act(sum + b), one fp16 rounding, then the residual.
__global__ void __launch_bounds__(256) dw_generic_kernel(const ConvParams p, FastDiv d_wo)
{
  const int HWo = p.Ho * p.Wo;
  const int hw = blockIdx.x * 256 + threadIdx.x;
  if (hw >= HWo) return;
  const int c = blockIdx.y, b = blockIdx.z;
  const int oy = (int)fastdiv((unsigned)hw, d_wo), ox = hw - oy * p.Wo;
  const float * W = reinterpret_cast<const float *>(p.w);
  float acc = 0.0f;
  for (int ky = 0; ky < p.K; ++ky) {
    const int iy = oy * p.S - p.P + ky;
    if ((unsigned)iy >= (unsigned)p.H) continue;
    for (int kx = 0; kx < p.K; ++kx) {
      const int ix = ox * p.S - p.P + kx;
      if ((unsigned)ix >= (unsigned)p.W) continue;
      acc += vld(p.x, b, c, (long)iy * p.W + ix) * W[(ky * p.K + kx) * p.Cin + c];
    }
  }
  float v = (float)(_Float16)act_f(acc + (p.bias ? p.bias[c] : 0.0f), p.act);
  if (p.r.ptr) v += vld(p.r, b, c, hw);
  vst(p.y, b, c, hw, v);
}

// Channel-planar depthwise (NCHW input, output in any layout) with K in {3, 5}: one lane =
// PX consecutive output pixels of one row of one channel plane (strips of a plane on
// neighbouring lanes, then the next channel), grid (strips of all planes, image); each input
// row segment of the strip is loaded once for its PX outputs.  Same tap order and roundings
// as the other kernels.
template <int K, int S, int PX>
__global__ void __launch_bounds__(256) dw_nchw_kernel(const ConvParams p, FastDiv d_strips, FastDiv d_plane)
{
  constexpr int NX = (PX - 1) * S + K;
  const int strips = (p.Wo + PX - 1) / PX, plane = p.Ho * strips;
  const int q = blockIdx.x * 256 + threadIdx.x;
  if (q >= p.Cin * plane) return;
  const int c = (int)fastdiv((unsigned)q, d_plane), r = q - c * plane, b = blockIdx.y;
  const int oy = (int)fastdiv((unsigned)r, d_strips), ox0 = (r - oy * strips) * PX;
  const _Float16 * xp = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img + (long)c * p.x.cs;
  const float * W = reinterpret_cast<const float *>(p.w) + c;
  float w[K * K];
#pragma unroll
  for (int k = 0; k < K * K; ++k) w[k] = W[k * p.Cin];
  const int iy0 = oy * S - p.P, ix0 = ox0 * S - p.P;
  float acc[PX];
#pragma unroll
  for (int j = 0; j < PX; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int ky = 0; ky < K; ++ky) {
    const int iy = iy0 + ky;
    if ((unsigned)iy >= (unsigned)p.H) continue;
    float xr[NX];
#pragma unroll
    for (int t = 0; t < NX; ++t) {
      const int ix = ix0 + t;
      xr[t] = (unsigned)ix < (unsigned)p.W ? (float)xp[iy * p.W + ix] : 0.0f;
    }
#pragma unroll
    for (int kx = 0; kx < K; ++kx)
#pragma unroll
      for (int j = 0; j < PX; ++j) acc[j] += xr[j * S + kx] * w[ky * K + kx];
  }
  const float bias = p.bias ? p.bias[c] : 0.0f;
#pragma unroll
  for (int j = 0; j < PX; ++j) {
    const int ox = ox0 + j;
    if (ox >= p.Wo) continue;
    const int hw = oy * p.Wo + ox;
    float v = (float)(_Float16)act_f(acc[j] + bias, p.act);
    if (p.r.ptr) v += vld(p.r, b, c, hw);
    vst(p.y, b, c, hw, v);  // channel planes or channels-last
  }
}

bool dwconv_vectorizable(const ConvParams & p)
{
  auto al = [](const View & v) {
    return v.layout == kNHWC && ((v.cs | (int)v.img | (int)(reinterpret_cast<uintptr_t>(v.ptr) >> 1)) & 7) == 0;
  };
  return p.w2 && (reinterpret_cast<uintptr_t>(p.w2) & 15) == 0 && (p.Cin % 8) == 0 && (p.K == 3 || p.K == 5) &&
         (p.S == 1 || p.S == 2) && al(p.x) && al(p.y) &&
         (!p.r.ptr || al(p.r)) && (long)p.batch * p.Ho * p.Wo * (p.Cin / 8) < (1L << 31) &&
         (((long)p.H * p.W - 1) * p.x.cs + p.Cin) * 2 < (1L << 31) &&  // one image's buffer range
         (long)p.H * p.W < (1L << 24);
}

// Tile choice for dw_tile_kernel.  Candidates: per-lane blocks PX x PY of at most two
// pixels (larger blocks measured slower on MI355X: fewer waves, longer dependent FMA
// chains), channel groups G = Cin/8 (whole pixels: a window row is one contiguous run) or a
// divisor of it of at least 8 (runs of 128 bytes or more), lane blocks BX x BY (at most 256
// lanes, window and weights within kDwBufPieces).  Cost: the largest of the VALU cycles per
// SIMD (4 cycles per wave64 instruction, FMAs plus staging), the LDS cycles per CU (128
// bytes per cycle, window stores plus block and weight reads) and the HBM bytes at 2500 per
// shader cycle (about 5 TB/s), halo re-reads at four times that.  Launches with at least
// 2.5 waves per SIMD hide their load latency; below that the candidate with the most waves
// is taken (small batches); among those with enough, work-groups of two or more waves, then
// the cheapest.
struct DwPick {
  int PX = 0, PY = 0;
  DwTile t{};
  size_t lds = 0;
};

static DwPick dw_pick_search(const ConvParams & p)
{
  const int C8 = p.Cin / 8, K = p.K, S = p.S;
  const double hbm = (double)p.batch * ((double)p.H * p.W + (double)p.Ho * p.Wo) * p.Cin * 2.0;
  constexpr double kEnoughWaves = 2.5 * 1024;
  DwPick best;
  double best_cost = 1e300, best_wk = 0.0;
  bool best_big = false;
  for (const int PX : {1, 2}) {
    for (const int PY : {1, 2}) {
      if (PX * PY > 2) continue;
      const int nbx = (p.Wo + PX - 1) / PX, nby = (p.Ho + PY - 1) / PY;
      const int NR = (PY - 1) * S + K, NX = (PX - 1) * S + K;
      for (int G = 1; G <= C8; ++G) {
        if (C8 % G || (G < C8 && G < 8)) continue;
        for (int sx = 1, last_bx = 0; sx <= nbx && sx <= 16; ++sx) {
          const int BX = (nbx + sx - 1) / sx;
          if (BX == last_bx) continue;
          last_bx = BX;
          for (int sy = 1, last_by = 0; sy <= nby && sy <= 64; ++sy) {
            const int BY = (nby + sy - 1) / sy;
            if (BY == last_by) continue;
            last_by = BY;
            const int lanes = G * BX * BY;
            if (lanes > 256) continue;
            const int IW = (BX * PX - 1) * S + K, IH = (BY * PY - 1) * S + K;
            const int nbuf = (IH * IW + K * K) * G;
            if (nbuf > kDwBufPieces || K * K * G > kDwMaxW * 256) continue;
            const int ntx = (p.Wo + BX * PX - 1) / (BX * PX), nty = (p.Ho + BY * PY - 1) / (BY * PY);
            const double nwg = (double)ntx * nty * (C8 / G) * p.batch;
            if (nwg >= 2147483648.0) continue;
            const double waves = nwg * ((lanes + 63) / 64);
            const double valu = waves * (PX * PY * K * K * 8 + ((nbuf + 255) / 256) * 25 + 150) * 4.0 / 1024.0;
            const double lds = nwg * (nbuf + (double)lanes * (NR * NX + K * K)) * 16.0 / (256.0 * 128.0);
            const double mem = hbm / 2500.0 + nwg * IH * IW * G * 16.0 / 10000.0;
            const double cost = std::max(valu, std::max(lds, mem));
            // rank: waves up to enough; then work-groups of at least two waves (one-wave
            // groups pay the staging latency for a quarter of the lanes); then cost
            const double wk = std::min(waves, kEnoughWaves);
            const bool big = lanes >= 128;
            const bool better = best.PX == 0 || wk > best_wk || (wk == best_wk && big > best_big) ||
                                (wk == best_wk && big == best_big && cost < best_cost);
            if (better) {
              best_cost = cost;
              best_wk = wk;
              best_big = big;
              best.PX = PX;
              best.PY = PY;
              best.t = DwTile{G, BX, BY, ntx, nty, C8 / G, IW, IH};
              best.lds = (size_t)nbuf * 16;
            }
          }
        }
      }
    }
  }
  return best;
}

// The search costs a few microseconds per call; eager runs call it every launch, so the
// picks are kept per shape.
static DwPick dw_pick(const ConvParams & p)
{
  static std::mutex mu;
  static std::map<std::array<int, 7>, DwPick> cache;
  const std::array<int, 7> key{p.Cin, p.H, p.W, p.K, p.S, p.P, p.batch};
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  const DwPick d = dw_pick_search(p);
  cache.emplace(key, d);
  return d;
}

template <int K, int S, int PX, int PY>
static void launch_dw_tile(const ConvParams & p, const DwPick & d, hipStream_t s)
{
  const unsigned nwg = (unsigned)((long)d.t.ntx * d.t.nty * d.t.nct * p.batch);
  switch (p.act) {
#define IVH_DW_CASE(A)                                                                                     \
  case A: hipLaunchKernelGGL((dw_tile_kernel<K, S, PX, PY, A>), dim3(nwg), dim3(256), d.lds, s, p, d.t); break;
  IVH_DW_CASE(kActSiLU)
  IVH_DW_CASE(kActReLU)
  IVH_DW_CASE(kActHSwish)
  IVH_DW_CASE(kActHSigmoid)
  IVH_DW_CASE(kActSigmoid)
  default: hipLaunchKernelGGL((dw_tile_kernel<K, S, PX, PY, kActNone>), dim3(nwg), dim3(256), d.lds, s, p, d.t); break;
#undef IVH_DW_CASE
  }
}

template <int K, int S>
static void launch_dw_ks(const ConvParams & p, const DwPick & d, hipStream_t s)
{
  if (d.PX == 2) launch_dw_tile<K, S, 2, 1>(p, d, s);
  else if (d.PY == 2) launch_dw_tile<K, S, 1, 2>(p, d, s);
  else launch_dw_tile<K, S, 1, 1>(p, d, s);
}

template <int ACT>
static void launch_dw_strip(const ConvParams & p, hipStream_t s)
{
  constexpr int PX = 4;
  const int nstrip = (p.Wo + PX - 1) / PX;
  const long n = (long)p.batch * p.Ho * nstrip * (p.Cin / 8);
  hipLaunchKernelGGL((dw_strip_kernel<5, 2, PX, ACT>), dim3(nblk(n, 256)), dim3(256), 0, s, p,
                     fastdiv_make((unsigned)(p.Cin / 8)), fastdiv_make((unsigned)nstrip), fastdiv_make((unsigned)p.Ho));
}

// The strip kernel is taken for 5x5 stride 2 once it has at least 1.5 waves per SIMD.
static bool dw_use_strip(const ConvParams & p)
{
  return p.K == 5 && p.S == 2 && (long)p.batch * p.Ho * ((p.Wo + 3) / 4) * (p.Cin / 8) >= 1536L * 64;
}

std::string dw_launch_tag(const ConvParams & p)
{
  if (!dwconv_vectorizable(p))
    return p.x.layout == kNCHW && (p.K == 3 || p.K == 5) && (p.S == 1 || p.S == 2) ? "planar px=4" : "generic";
  if (dw_use_strip(p)) return "strip px=4";
  const DwPick d = dw_pick(p);
  char b[128];
  snprintf(b, sizeof b, "tile px=%d py=%d g=%d bx=%d by=%d", d.PX, d.PY, d.t.G, d.t.BX, d.t.BY);
  return b;
}

void launch_dwconv(const ConvParams & p, hipStream_t s)
{
  if (!dwconv_vectorizable(p)) {
    if (p.Cin > 65535 || p.batch > 65535) throw std::runtime_error("depthwise: grid");
    const dim3 grid(nblk((long)p.Ho * p.Wo, 256), (unsigned)p.Cin, (unsigned)p.batch);
    const bool planar = p.x.layout == kNCHW && (long)p.H * p.W < (1L << 31) && (p.K == 3 || p.K == 5) &&
                        (p.S == 1 || p.S == 2);
    if (planar) {
      constexpr int PX = 4;
      const int strips = (p.Wo + PX - 1) / PX;
      const long n = (long)p.Cin * p.Ho * strips;
      if (n >= (1L << 31)) throw std::runtime_error("depthwise: grid");
      const dim3 g(nblk(n, 256), (unsigned)p.batch);
      const FastDiv f = fastdiv_make((unsigned)strips), fp = fastdiv_make((unsigned)(p.Ho * strips));
      if (p.K == 3 && p.S == 1) hipLaunchKernelGGL((dw_nchw_kernel<3, 1, PX>), g, dim3(256), 0, s, p, f, fp);
      else if (p.K == 3) hipLaunchKernelGGL((dw_nchw_kernel<3, 2, PX>), g, dim3(256), 0, s, p, f, fp);
      else if (p.S == 1) hipLaunchKernelGGL((dw_nchw_kernel<5, 1, PX>), g, dim3(256), 0, s, p, f, fp);
      else hipLaunchKernelGGL((dw_nchw_kernel<5, 2, PX>), g, dim3(256), 0, s, p, f, fp);
    } else {
      hipLaunchKernelGGL(dw_generic_kernel, grid, dim3(256), 0, s, p, fastdiv_make((unsigned)p.Wo));
    }
    return;
  }
  if (dw_use_strip(p)) {
    switch (p.act) {
    case kActSiLU: launch_dw_strip<kActSiLU>(p, s); break;
    case kActReLU: launch_dw_strip<kActReLU>(p, s); break;
    case kActHSwish: launch_dw_strip<kActHSwish>(p, s); break;
    case kActHSigmoid: launch_dw_strip<kActHSigmoid>(p, s); break;
    case kActSigmoid: launch_dw_strip<kActSigmoid>(p, s); break;
    default: launch_dw_strip<kActNone>(p, s); break;
    }
    return;
  }
  const DwPick d = dw_pick(p);
  if (d.PX == 0) throw std::runtime_error("depthwise: no tile fits");
  if (p.K == 3) {
    if (p.S == 1) launch_dw_ks<3, 1>(p, d, s);
    else launch_dw_ks<3, 2>(p, d, s);
  } else {
    if (p.S == 1) launch_dw_ks<5, 1>(p, d, s);
    else launch_dw_ks<5, 2>(p, d, s);
  }
}

// ------------------------------------------------------------------ small ops
// Semantics of kernels/ops.cl (fp32 compute, fp16 store), batch on grid axis y.

__device__ __forceinline__ float binop(float a, float b, int op)
{
  switch (op) {
  case 0: return a + b;
  case 1: return a - b;
  case 2: return a * b;
  default: return a / b;
  }
}

// iteration index -> (c, p) in the output's physical order (coalesced stores)
__device__ __forceinline__ void cp_of(const SmallParams & q, long i, int & c, long & p)
{
  const long HW = (long)q.H * q.W;
  if (q.y.layout == kNHWC) { p = i / q.C; c = (int)(i - p * q.C); }
  else { c = (int)(i / HW); p = i - (long)c * HW; }
}

__global__ void ew_same_kernel(const SmallParams q)  // ew_binary / ew_binary_v (ops.cl:34-48,373-391)
{
  const long n = (long)q.C * q.H * q.W;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  cp_of(q, i, c, p);
  const float av = vld(q.a, b, c, p);
  const float bv = (q.b.img == 0 && q.b.cs == 0) ? (float)reinterpret_cast<const _Float16 *>(q.b.ptr)[0]
                                                 : vld(q.b, b, c, p);
  vst(q.y, b, c, p, binop(av, bv, q.op));
}

__global__ void ew_unary_kernel(const SmallParams q)  // ew_unary (ops.cl:50-63), canonical code in op
{
  const long n = (long)q.C * q.H * q.W;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  cp_of(q, i, c, p);
  vst(q.y, b, c, p, act_f(vld(q.a, b, c, p), q.op));
}

__global__ void copy_kernel(const SmallParams q)  // copy_c / concat part / layout change
{
  const long n = (long)q.C * q.H * q.W;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  cp_of(q, i, c, p);
  const long si = vidx(q.a, b, c, p), di = vidx(q.y, b, c, p);
  reinterpret_cast<_Float16 *>(q.y.ptr)[di] = reinterpret_cast<const _Float16 *>(q.a.ptr)[si];
}

// ew_binary_ch (ops.cl:311-341): one operand is per-channel [C]; i0 = 1 if that is `a`.
__global__ void ew_chan_kernel(const SmallParams q)
{
  const long n = (long)q.C * q.H * q.W;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  cp_of(q, i, c, p);
  const _Float16 * ap = reinterpret_cast<const _Float16 *>(q.a.ptr);
  const _Float16 * bp = reinterpret_cast<const _Float16 *>(q.b.ptr);
  float av, bv;
  if (q.i0) { av = (float)ap[(long)b * q.a.img + c]; bv = vld(q.b, b, c, p); }
  else { av = vld(q.a, b, c, p); bv = (float)bp[(long)b * q.b.img + c]; }
  vst(q.y, b, c, p, binop(av, bv, q.op));
}

// ew_binary_bcast (ops.cl:10-32): flat NCHW, dims = [out, a_strides, b_strides].
__global__ void ew_bcast_kernel(const SmallParams q)
{
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= q.n) return;
  long rem = i, ai = 0, bi = 0;
  for (int r = q.rank - 1; r >= 0; --r) {
    const long od = q.dims[r];
    const long coord = rem % od;
    rem /= od;
    ai += coord * q.dims[q.rank + r];
    bi += coord * q.dims[2 * q.rank + r];
  }
  const float av = (float)reinterpret_cast<const _Float16 *>(q.a.ptr)[(long)b * q.a.img + ai];
  const float bv = (float)reinterpret_cast<const _Float16 *>(q.b.ptr)[(long)b * q.b.img + bi];
  reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + i] = (_Float16)binop(av, bv, q.op);
}

__global__ void slice_axis_kernel(const SmallParams q)  // ops.cl:74-91
{
  const long total = (long)q.i0 * q.i4 * q.i2;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= total) return;
  const long li = (long)q.i4 * q.i2;
  const long o = i / li, rem = i - o * li;
  const _Float16 * x = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)b * q.a.img;
  reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + i] = x[(o * q.i1 + q.i3) * q.i2 + rem];
}

// One source of concat4 (ops.cl:93-119) with outer > 1:
// y[o][off + ax][r] = x[o][ax][r], i0 outer, i1 src axis len, i2 inner, i3 dst axis len, i4 off.
__global__ void concat_outer_kernel(const SmallParams q)
{
  const long total = (long)q.i0 * q.i1 * q.i2;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= total) return;
  const long r = i % q.i2, t = i / q.i2;
  const long ax = t % q.i1, o = t / q.i1;
  reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + (o * q.i3 + q.i4 + ax) * q.i2 + r] =
    reinterpret_cast<const _Float16 *>(q.a.ptr)[(long)b * q.a.img + i];
}

__global__ void maxpool_kernel(const SmallParams q)  // ops.cl:148-166, OOB taps ignored
{
  const long n = (long)q.C * q.Ho * q.Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  SmallParams o = q;
  o.H = q.Ho; o.W = q.Wo;
  cp_of(o, i, c, p);
  const int oh = (int)(p / q.Wo), ow = (int)(p % q.Wo);
  float m = -3.4e38f;
  for (int kh = 0; kh < q.K; ++kh) {
    const int yy = oh * q.S - q.P + kh;
    if ((unsigned)yy >= (unsigned)q.H) continue;
    for (int kw = 0; kw < q.K; ++kw) {
      const int xx = ow * q.S - q.P + kw;
      if ((unsigned)xx >= (unsigned)q.W) continue;
      m = fmaxf(m, vld(q.a, b, c, (long)yy * q.W + xx));
    }
  }
  vst(q.y, b, c, p, m);
}

__global__ void resize_nn_kernel(const SmallParams q)  // ops.cl:168-179, i0 = scale
{
  const long n = (long)q.C * q.Ho * q.Wo;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= n) return;
  int c; long p;
  SmallParams o = q;
  o.H = q.Ho; o.W = q.Wo;
  cp_of(o, i, c, p);
  const int oh = (int)(p / q.Wo), ow = (int)(p % q.Wo);
  const long si = vidx(q.a, b, c, (long)(oh / q.i0) * q.W + ow / q.i0);
  reinterpret_cast<_Float16 *>(q.y.ptr)[vidx(q.y, b, c, p)] = reinterpret_cast<const _Float16 *>(q.a.ptr)[si];
}

__global__ void softmax_kernel(const SmallParams q)  // ops.cl:181-197
{
  const long total = (long)q.i0 * q.i2;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= total) return;
  const long o = i / q.i2, r = i - o * q.i2;
  const _Float16 * x = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)b * q.a.img + o * q.i1 * q.i2 + r;
  _Float16 * y = reinterpret_cast<_Float16 *>(q.y.ptr) + (long)b * q.y.img + o * q.i1 * q.i2 + r;
  float m = -3.4e38f;
  for (int a = 0; a < q.i1; ++a) m = fmaxf(m, (float)x[(long)a * q.i2]);
  float s = 0.0f;
  for (int a = 0; a < q.i1; ++a) s += __expf((float)x[(long)a * q.i2] - m);
  const float inv = 1.0f / s;
  for (int a = 0; a < q.i1; ++a) y[(long)a * q.i2] = (_Float16)(__expf((float)x[(long)a * q.i2] - m) * inv);
}

__global__ void permute_kernel(const SmallParams q)  // ops.cl:199-222
{
  const long total = (long)q.i0 * q.i1 * q.i2;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= total) return;
  // i enumerates the OUTPUT (coalesced stores)
  long src;
  if (q.op == 0) {  // out [D2][D1][I]
    const long r = i % q.i2, t = i / q.i2;
    const long d1 = t % q.i0, d2 = t / q.i0;
    src = (d1 * q.i1 + d2) * q.i2 + r;
  } else {          // out [D1][I][D2]
    const long d2 = i % q.i1, t = i / q.i1;
    const long r = t % q.i2, d1 = t / q.i2;
    src = (d1 * q.i1 + d2) * q.i2 + r;
  }
  reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + i] =
    reinterpret_cast<const _Float16 *>(q.a.ptr)[(long)b * q.a.img + src];
}

// gap / gap_r (ops.cl:224-266): one 64-lane wave per (image, channel), fp32 tree reduction.
__global__ void __launch_bounds__(256) gap_kernel(const SmallParams q)
{
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + wave;
  const int b = blockIdx.y;
  if (c >= q.C) return;
  const long HW = (long)q.H * q.W;
  float s = 0.0f;
  for (long p = lane; p < HW; p += 64) s += vld(q.a, b, c, p);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0)
    reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + c] = (_Float16)(s / (float)HW);
}

// bmm (ops.cl:276-294): fp32 accumulation, one lane per output.
__global__ void bias_add_kernel(const SmallParams q)  // ops.cl:268-274
{
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= q.n) return;
  const float x = (float)reinterpret_cast<const _Float16 *>(q.a.ptr)[(long)b * q.a.img + i];
  const float bb = (float)reinterpret_cast<const _Float16 *>(q.b.ptr)[i / q.i0];
  reinterpret_cast<_Float16 *>(q.y.ptr)[(long)b * q.y.img + i] = (_Float16)(x + bb);
}


// ---------------------------------------------------------- 16-byte vector paths
// Used when every operand of an op is channels-last with C % 8 == 0 (one lane = one pixel x
// 8 channels) or dense NCHW with 8 | C*H*W (one lane = 8 consecutive elements).  The
// per-channel operand of ew_binary_ch is a plain [C] vector per image.

__device__ __forceinline__ h8 ld8(const __half * p, long off) { return *reinterpret_cast<const h8 *>(reinterpret_cast<const _Float16 *>(p) + off); }
__device__ __forceinline__ void st8(__half * p, long off, h8 v) { *reinterpret_cast<h8 *>(reinterpret_cast<_Float16 *>(p) + off) = v; }

// mode: 0 binary, 1 binary with scalar b, 2 unary (op = act), 3 copy, 4 chan (a = [C]), 5 chan (b = [C])
__global__ void __launch_bounds__(256) ew_vec8_kernel(const SmallParams q, int mode)
{
  const int HW = q.H * q.W;
  const int C8 = q.C >> 3;
  const int total8 = (int)(((long)q.C * HW) >> 3);
  const int i8 = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (i8 >= total8) return;
  const bool nhwc = q.y.layout == kNHWC;
  int c;
  long pa, pb, py;
  if (nhwc) {
    const int p = i8 / C8;
    c = (i8 - p * C8) * 8;
    pa = (long)p * q.a.cs + c;
    pb = (long)p * q.b.cs + c;
    py = (long)p * q.y.cs + c;
  } else {
    const long e = (long)i8 * 8;
    c = (int)(e / HW);
    pa = pb = py = e;
  }
  pa += (long)b * q.a.img;
  pb += (long)b * q.b.img;
  py += (long)b * q.y.img;
  h8 out;
  if (mode == 3) {
    out = ld8(q.a.ptr, pa);
  } else if (mode == 2) {
    const h8 x = ld8(q.a.ptr, pa);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)act_f((float)x[e], q.op);
  } else {
    const _Float16 * ap = reinterpret_cast<const _Float16 *>(q.a.ptr);
    const _Float16 * bp = reinterpret_cast<const _Float16 *>(q.b.ptr);
    float av[8], bv[8];
    if (mode == 4) {
#pragma unroll
      for (int e = 0; e < 8; ++e) av[e] = (float)ap[(long)b * q.a.img + c + (nhwc ? e : 0)];
    } else {
      const h8 x = ld8(q.a.ptr, pa);
#pragma unroll
      for (int e = 0; e < 8; ++e) av[e] = (float)x[e];
    }
    if (mode == 5) {
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = (float)bp[(long)b * q.b.img + c + (nhwc ? e : 0)];
    } else if (mode == 1) {
      const float s0 = (float)bp[0];
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = s0;
    } else {
      const h8 x = ld8(q.b.ptr, pb);
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = (float)x[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)binop(av[e], bv[e], q.op);
  }
  st8(q.y.ptr, py, out);
}

// nearest resize / max pool, channels-last, one lane = one output pixel x 8 channels.  KP > 0:
// a KP x KP max pool with the window unrolled, so every tap's 16-byte load is issued before
// the first maximum (out-of-image taps are skipped by predication, not by a loop exit).
template <int KP>
__global__ void __launch_bounds__(256) pool_vec8_kernel(const SmallParams q, int is_max)
{
  const int C8 = q.C >> 3;
  const int HWo = q.Ho * q.Wo;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= HWo * C8) return;
  const int p = i / C8, c = (i - p * C8) * 8;
  const int oh = p / q.Wo, ow = p - oh * q.Wo;
  const long abase = (long)b * q.a.img + c;
  h8 out;
  if (!is_max) {
    out = ld8(q.a.ptr, abase + (long)((oh / q.i0) * q.W + ow / q.i0) * q.a.cs);
  } else {
    float m[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) m[e] = -3.4e38f;
    auto tap = [&](int yy, int xx) {
      if ((unsigned)yy < (unsigned)q.H && (unsigned)xx < (unsigned)q.W) {
        const h8 v = ld8(q.a.ptr, abase + (long)(yy * q.W + xx) * q.a.cs);
#pragma unroll
        for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], (float)v[e]);
      }
    };
    if (KP > 0) {
#pragma unroll
      for (int kh = 0; kh < KP; ++kh)
#pragma unroll
        for (int kw = 0; kw < KP; ++kw) tap(oh * q.S - q.P + kh, ow * q.S - q.P + kw);
    } else {
      for (int kh = 0; kh < q.K; ++kh)
        for (int kw = 0; kw < q.K; ++kw) tap(oh * q.S - q.P + kh, ow * q.S - q.P + kw);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)m[e];
  }
  st8(q.y.ptr, (long)b * q.y.img + (long)p * q.y.cs + c, out);
}

// KP x KP stride-1 max pool, channels-last (SPPF's 5x5): one lane = RO consecutive output
// rows of one column x 8 channels.  The horizontal maximum of each of the RO + KP - 1 input
// rows is taken once (KP loads) and reused by the KP output rows whose window holds it, so an
// output costs (RO + KP - 1) * KP / RO loads instead of KP * KP; every load is issued before
// the first maximum (the window is unrolled, out-of-image taps are predicated off).
template <int KP, int RO>
__global__ void __launch_bounds__(256) maxpool_s1_cols_kernel(const SmallParams q)
{
  const int C8 = q.C >> 3, nrb = (q.Ho + RO - 1) / RO;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= q.Wo * C8 * nrb) return;
  const int cc = i / C8, c = (i - cc * C8) * 8;  // (row block, column) fastest after channels
  const int rb = cc / q.Wo, ox = cc - rb * q.Wo;
  const int oy0 = rb * RO;
  const long abase = (long)b * q.a.img + c;
  float hm[RO + KP - 1][8];
#pragma unroll
  for (int r = 0; r < RO + KP - 1; ++r) {
#pragma unroll
    for (int e = 0; e < 8; ++e) hm[r][e] = -3.4e38f;
    const int yy = oy0 - q.P + r;
#pragma unroll
    for (int kw = 0; kw < KP; ++kw) {
      const int xx = ox - q.P + kw;
      if ((unsigned)yy < (unsigned)q.H && (unsigned)xx < (unsigned)q.W) {
        const h8 v = ld8(q.a.ptr, abase + (long)(yy * q.W + xx) * q.a.cs);
#pragma unroll
        for (int e = 0; e < 8; ++e) hm[r][e] = fmaxf(hm[r][e], (float)v[e]);
      }
    }
  }
#pragma unroll
  for (int o = 0; o < RO; ++o) {
    if (oy0 + o >= q.Ho) break;
    h8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float m = hm[o][e];
#pragma unroll
      for (int k = 1; k < KP; ++k) m = fmaxf(m, hm[o + k][e]);
      out[e] = (_Float16)m;
    }
    st8(q.y.ptr, (long)b * q.y.img + (long)((oy0 + o) * q.Wo + ox) * q.y.cs + c, out);
  }
}

// SPPF's three chained max pools (5x5, stride 1, pad 2, each reading the previous one's
// output) from one read of the first input: the chain's outputs are the 5x5, 9x9 and 13x13
// max pools of that input with windows clipped at the borders (a max over maxima is the max
// over the union of their windows, and clipping composes the same way).  One work-group per
// (image, 8 channels): the plane into LDS, row maxima of widths 5 / 9 / 13, then column
// maxima.  Maxima of fp16 values are fp16 values: packed fp16 max (IEEE maxNum, as fmaxf)
// gives every output bit for bit as the chained pools compute it.  The work-groups of one
// image's neighbouring channel groups, which read and write the same 128-byte lines of the
// channels-last tensors, run on one XCD (xcd_tile), so those lines meet in one L2 instead of
// leaving eight partially written copies to be merged behind the L2s.
__global__ void __launch_bounds__(256) maxpool_sppf3_kernel(const SmallParams q)
{
  extern __shared__ h8 pl[];  // 4 planes of H * W pixels: input, row maxima 5 / 9 / 13
  const int HW = q.H * q.W, C8 = q.C / 8;
  const int t = xcd_tile(blockIdx.x, (int)gridDim.x);
  const int b = t / C8, c = (t - b * C8) * 8;
  const h8 ninf = (h8)(_Float16)(-__builtin_inff());
  for (int p = threadIdx.x; p < HW; p += 256) pl[p] = ld8(q.a.ptr, (long)b * q.a.img + (long)p * q.a.cs + c);
  __syncthreads();
  for (int p = threadIdx.x; p < HW; p += 256) {
    const int y = p / q.W, x = p - y * q.W;
    h8 m5 = ninf, m9 = ninf, m13 = ninf;
#pragma unroll
    for (int d = -6; d <= 6; ++d) {
      const int xx = x + d;
      if ((unsigned)xx >= (unsigned)q.W) continue;
      const h8 v = pl[y * q.W + xx];
      m13 = __builtin_elementwise_max(m13, v);
      if (d >= -4 && d <= 4) m9 = __builtin_elementwise_max(m9, v);
      if (d >= -2 && d <= 2) m5 = __builtin_elementwise_max(m5, v);
    }
    pl[HW + p] = m5;
    pl[2 * HW + p] = m9;
    pl[3 * HW + p] = m13;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < HW; p += 256) {
    const int y = p / q.W, x = p - y * q.W;
    h8 m5 = ninf, m9 = ninf, m13 = ninf;
#pragma unroll
    for (int d = -6; d <= 6; ++d) {
      const int yy = y + d;
      if ((unsigned)yy >= (unsigned)q.H) continue;
      const int i = yy * q.W + x;
      m13 = __builtin_elementwise_max(m13, pl[3 * HW + i]);
      if (d >= -4 && d <= 4) m9 = __builtin_elementwise_max(m9, pl[2 * HW + i]);
      if (d >= -2 && d <= 2) m5 = __builtin_elementwise_max(m5, pl[HW + i]);
    }
    st8(q.y.ptr, (long)b * q.y.img + (long)p * q.y.cs + c, m5);
    st8(q.b.ptr, (long)b * q.b.img + (long)p * q.b.cs + c, m9);
    st8(q.c.ptr, (long)b * q.c.img + (long)p * q.c.cs + c, m13);
  }
}

// Row copies of `L` contiguous elements (L % 8 == 0): slice_axis, concat along an inner
// axis, permute mode 0.  kind 0 slice, 1 concat part, 2 permute.
__global__ void __launch_bounds__(256) rows_vec8_kernel(const SmallParams q, int kind, int L, int rows)
{
  const int L8 = L >> 3;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (t >= rows * L8) return;
  const int r = t / L8, j = (t - r * L8) * 8;
  long src, dst;
  if (kind == 0) {        // y row r = (o, l) <- x row o*axdim + start + l
    const int o = r / q.i4, l = r - o * q.i4;
    dst = (long)r * L;
    src = (long)(o * q.i1 + q.i3 + l) * L;
  } else if (kind == 1) { // x block o (axis x inner, L elements) -> y at (o*tot + off)*inner
    src = (long)r * L;
    dst = ((long)r * q.i3 + q.i4) * q.i2;
  } else {                // y row r = (d2, d1) <- x row d1*D2 + d2
    const int d2 = r / q.i0, d1 = r - d2 * q.i0;
    dst = (long)r * L;
    src = (long)(d1 * q.i1 + d2) * L;
  }
  st8(q.y.ptr, (long)b * q.y.img + dst + j, ld8(q.a.ptr, (long)b * q.a.img + src + j));
}

// ew_binary_bcast with 8 consecutive outputs per lane (output innermost extent % 8 == 0).
// Coordinates by float-reciprocal divisions (outputs per image < 2^22); an operand whose
// innermost stride is 1 (and 8-aligned start) is read as one 16-byte vector, a stride-0 one
// as one scalar, anything else element by element.
__global__ void __launch_bounds__(256) ew_bcast8_kernel(const SmallParams q)
{
  const int t = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  const int n8 = (int)(q.n >> 3);
  if (t >= n8) return;
  int rem = t * 8, ai = 0, bi = 0;
  for (int r = q.rank - 1; r >= 0; --r) {
    const int od = q.dims[r];
    const int qt = idiv_small(rem, od, __builtin_amdgcn_rcpf((float)od));
    const int coord = rem - qt * od;
    rem = qt;
    ai += coord * q.dims[q.rank + r];
    bi += coord * q.dims[2 * q.rank + r];
  }
  const int sa = q.dims[2 * q.rank - 1], sb = q.dims[3 * q.rank - 1];
  const _Float16 * ap = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)b * q.a.img;
  const _Float16 * bp = reinterpret_cast<const _Float16 *>(q.b.ptr) + (long)b * q.b.img;
  auto load8 = [](const _Float16 * base, int i0, int st) {
    h8 v;
    if (st == 1 && ((i0 | (int)(reinterpret_cast<uintptr_t>(base) >> 1)) & 7) == 0) {
      v = *reinterpret_cast<const h8 *>(base + i0);
    } else if (st == 0) {
      const _Float16 x = base[i0];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = x;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = base[i0 + e * st];
    }
    return v;
  };
  const h8 av = load8(ap, ai, sa), bv = load8(bp, bi, sb);
  h8 out;
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (_Float16)binop((float)av[e], (float)bv[e], q.op);
  st8(q.y.ptr, (long)b * q.y.img + (long)t * 8, out);
}

// softmax over an axis with stride `inner` > 1: values cached in registers (axdim <= 32).
__global__ void __launch_bounds__(256) softmax_reg_kernel(const SmallParams q)
{
  const int total = q.i0 * q.i2;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= total) return;
  const int o = i / q.i2, r = i - o * q.i2;
  const long base = (long)o * q.i1 * q.i2 + r;
  const _Float16 * x = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)b * q.a.img + base;
  _Float16 * y = reinterpret_cast<_Float16 *>(q.y.ptr) + (long)b * q.y.img + base;
  float v[32];
  float m = -3.4e38f;
#pragma unroll
  for (int a = 0; a < 32; ++a)
    if (a < q.i1) { v[a] = (float)x[(long)a * q.i2]; m = fmaxf(m, v[a]); }
  float s = 0.0f;
#pragma unroll
  for (int a = 0; a < 32; ++a)
    if (a < q.i1) { v[a] = __expf(v[a] - m); s += v[a]; }
  const float inv = 1.0f / s;
#pragma unroll
  for (int a = 0; a < 32; ++a)
    if (a < q.i1) y[(long)a * q.i2] = (_Float16)(v[a] * inv);
}

// softmax over a short strided axis with 8 consecutive inner positions per lane (inner % 8
// == 0): 16-byte loads and stores; the axis values stay in registers as fp16 and exp is
// recomputed for the output (the same fp32 arithmetic as softmax_reg_kernel).
template <int AMAX>
__global__ void __launch_bounds__(256) softmax_vec8_kernel(const SmallParams q)
{
  const int I8 = q.i2 >> 3;
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (i >= q.i0 * I8) return;
  const int o = i / I8, r = (i - o * I8) * 8;
  const long base = (long)b * q.a.img + (long)o * q.i1 * q.i2 + r;
  const long ybase = (long)b * q.y.img + (long)o * q.i1 * q.i2 + r;
  h8 xv[AMAX];
  float m[8], sum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { m[e] = -3.4e38f; sum[e] = 0.0f; }
#pragma unroll
  for (int a = 0; a < AMAX; ++a)
    if (a < q.i1) {
      xv[a] = ld8(q.a.ptr, base + (long)a * q.i2);
#pragma unroll
      for (int e = 0; e < 8; ++e) m[e] = fmaxf(m[e], (float)xv[a][e]);
    }
#pragma unroll
  for (int a = 0; a < AMAX; ++a)
    if (a < q.i1) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sum[e] += __expf((float)xv[a][e] - m[e]);
    }
#pragma unroll
  for (int e = 0; e < 8; ++e) sum[e] = 1.0f / sum[e];
#pragma unroll
  for (int a = 0; a < AMAX; ++a)
    if (a < q.i1) {
      h8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (_Float16)(__expf((float)xv[a][e] - m[e]) * sum[e]);
      st8(q.y.ptr, ybase + (long)a * q.i2, v);
    }
}

// softmax over the contiguous last axis (inner == 1): one wave per row, shuffle reductions.
__global__ void __launch_bounds__(256) softmax_row_kernel(const SmallParams q)
{
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int b = blockIdx.y;
  if (row >= q.i0) return;
  const _Float16 * x = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)b * q.a.img + (long)row * q.i1;
  _Float16 * y = reinterpret_cast<_Float16 *>(q.y.ptr) + (long)b * q.y.img + (long)row * q.i1;
  float m = -3.4e38f;
  for (int a = lane; a < q.i1; a += 64) m = fmaxf(m, (float)x[a]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  float s = 0.0f;
  for (int a = lane; a < q.i1; a += 64) s += __expf((float)x[a] - m);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  const float inv = 1.0f / s;
  for (int a = lane; a < q.i1; a += 64) y[a] = (_Float16)(__expf((float)x[a] - m) * inv);
}

namespace {
bool al8(const View & v) { return ((v.img | (long)(reinterpret_cast<uintptr_t>(v.ptr) >> 1)) & 7) == 0; }
// every listed view channels-last, 8-channel aligned
bool nhwc8(const SmallParams & q, std::initializer_list<const View *> vs)
{
  if (q.C % 8) return false;
  for (const View * v : vs)
    if (v->layout != kNHWC || (v->cs % 8) || !al8(*v)) return false;
  return true;
}
// every listed view dense NCHW (channel stride == H*W), 8 | C*H*W
bool dense8(const SmallParams & q, std::initializer_list<const View *> vs, bool chan)
{
  const long HW = (long)q.H * q.W;
  if (((long)q.C * HW) % 8 || (chan && HW % 8)) return false;
  for (const View * v : vs)
    if (v->layout != kNCHW || (q.C > 1 && v->cs != HW) || !al8(*v)) return false;
  return true;
}
}  // namespace

// Picks the vector kernel for a small op when its operands allow it; returns false to
// fall back to the scalar kernel.
bool launch_small_vec(int kind, const SmallParams & q, hipStream_t s)
{
  const dim3 blk(256);
  const unsigned B = (unsigned)q.batch;
  const long n8 = (long)q.C * q.H * q.W / 8;
  auto ew = [&](int mode, std::initializer_list<const View *> vs, bool chan) {
    if (!(nhwc8(q, vs) || dense8(q, vs, chan))) return false;
    hipLaunchKernelGGL(ew_vec8_kernel, dim3(nblk(n8, 256), B), blk, 0, s, q, mode);
    return true;
  };
  switch (kind) {
  case kEwSame:
    if (q.b.img == 0 && q.b.cs == 0) return ew(1, {&q.a, &q.y}, false);
    return ew(0, {&q.a, &q.b, &q.y}, false);
  case kEwUnary: return ew(2, {&q.a, &q.y}, false);
  case kCopy: return ew(3, {&q.a, &q.y}, false);
  case kEwChan: return q.i0 ? ew(4, {&q.b, &q.y}, true) : ew(5, {&q.a, &q.y}, true);
  case kMaxPool:
  case kResizeNN:
    if (!nhwc8(q, {&q.a, &q.y})) return false;
    if (kind == kMaxPool && q.K == 5 && q.S == 1 && q.Ho == q.H && q.Wo == q.W) {
      constexpr int RO = 4;
      hipLaunchKernelGGL((maxpool_s1_cols_kernel<5, RO>), dim3(nblk((long)((q.Ho + RO - 1) / RO) * q.Wo * (q.C / 8), 256), B),
                         blk, 0, s, q);
    } else if (kind == kMaxPool && q.K == 5)
      hipLaunchKernelGGL(pool_vec8_kernel<5>, dim3(nblk((long)q.Ho * q.Wo * (q.C / 8), 256), B), blk, 0, s, q, 1);
    else if (kind == kMaxPool && q.K == 3)
      hipLaunchKernelGGL(pool_vec8_kernel<3>, dim3(nblk((long)q.Ho * q.Wo * (q.C / 8), 256), B), blk, 0, s, q, 1);
    else
      hipLaunchKernelGGL(pool_vec8_kernel<0>, dim3(nblk((long)q.Ho * q.Wo * (q.C / 8), 256), B), blk, 0, s, q,
                         kind == kMaxPool ? 1 : 0);
    return true;
  case kSliceAxis:
  case kConcatOuter:
  case kPermute: {
    // concat: one row per outer index, axis x inner contiguous elements on both sides
    const int L = kind == kConcatOuter ? q.i1 * q.i2 : q.i2;
    if (L % 8 || !al8(q.a) || !al8(q.y)) return false;
    if (kind == kConcatOuter && (((long)q.i3 * q.i2) % 8 || ((long)q.i4 * q.i2) % 8)) return false;
    if (kind == kPermute && q.op != 0) return false;
    const int rows = kind == kSliceAxis ? q.i0 * q.i4 : (kind == kConcatOuter ? q.i0 : q.i0 * q.i1);
    const int k = kind == kSliceAxis ? 0 : (kind == kConcatOuter ? 1 : 2);
    hipLaunchKernelGGL(rows_vec8_kernel, dim3(nblk((long)rows * (L / 8), 256), B), blk, 0, s, q, k, L, rows);
    return true;
  }
  case kEwBcast:
    if (q.n % 8 || q.dims[q.rank - 1] % 8 || !al8(q.y) || q.n >= (1L << 22)) return false;
    hipLaunchKernelGGL(ew_bcast8_kernel, dim3(nblk(q.n / 8, 256), B), blk, 0, s, q);
    return true;
  case kSoftmax:
    if (q.i2 % 8 == 0 && q.i1 <= 32 && al8(q.a) && al8(q.y)) {
      const unsigned g = nblk((long)q.i0 * (q.i2 / 8), 256);
      if (q.i1 <= 16) hipLaunchKernelGGL(softmax_vec8_kernel<16>, dim3(g, B), blk, 0, s, q);
      else hipLaunchKernelGGL(softmax_vec8_kernel<32>, dim3(g, B), blk, 0, s, q);
      return true;
    }
    if (q.i2 > 1 && q.i1 <= 32) {
      hipLaunchKernelGGL(softmax_reg_kernel, dim3(nblk((long)q.i0 * q.i2, 256), B), blk, 0, s, q);
      return true;
    }
    if (q.i2 == 1) {
      hipLaunchKernelGGL(softmax_row_kernel, dim3((unsigned)((q.i0 + 3) / 4), B), blk, 0, s, q);
      return true;
    }
    return false;
  default: return false;
  }
}

void launch_small(int kind, const SmallParams & q, hipStream_t s)
{
  if (kind == kMaxPoolSppf) {
    hipLaunchKernelGGL(maxpool_sppf3_kernel, dim3((unsigned)(q.C / 8 * q.batch)), dim3(256),
                       (size_t)4 * q.H * q.W * 16, s, q);
    return;
  }
  if (launch_small_vec(kind, q, s)) return;
  const dim3 blk(256);
  const unsigned B = (unsigned)q.batch;
  const long nchw = (long)q.C * q.H * q.W;
  switch (kind) {
  case kEwSame: hipLaunchKernelGGL(ew_same_kernel, dim3(nblk(nchw, 256), B), blk, 0, s, q); break;
  case kEwUnary: hipLaunchKernelGGL(ew_unary_kernel, dim3(nblk(nchw, 256), B), blk, 0, s, q); break;
  case kCopy: hipLaunchKernelGGL(copy_kernel, dim3(nblk(nchw, 256), B), blk, 0, s, q); break;
  case kEwChan: hipLaunchKernelGGL(ew_chan_kernel, dim3(nblk(nchw, 256), B), blk, 0, s, q); break;
  case kEwBcast: hipLaunchKernelGGL(ew_bcast_kernel, dim3(nblk(q.n, 256), B), blk, 0, s, q); break;
  case kSliceAxis:
    hipLaunchKernelGGL(slice_axis_kernel, dim3(nblk((long)q.i0 * q.i4 * q.i2, 256), B), blk, 0, s, q);
    break;
  case kConcatOuter:
    hipLaunchKernelGGL(concat_outer_kernel, dim3(nblk((long)q.i0 * q.i1 * q.i2, 256), B), blk, 0, s, q);
    break;
  case kMaxPool:
    hipLaunchKernelGGL(maxpool_kernel, dim3(nblk((long)q.C * q.Ho * q.Wo, 256), B), blk, 0, s, q);
    break;
  case kResizeNN:
    hipLaunchKernelGGL(resize_nn_kernel, dim3(nblk((long)q.C * q.Ho * q.Wo, 256), B), blk, 0, s, q);
    break;
  case kSoftmax:
    hipLaunchKernelGGL(softmax_kernel, dim3(nblk((long)q.i0 * q.i2, 256), B), blk, 0, s, q);
    break;
  case kPermute:
    hipLaunchKernelGGL(permute_kernel, dim3(nblk((long)q.i0 * q.i1 * q.i2, 256), B), blk, 0, s, q);
    break;
  case kGap: hipLaunchKernelGGL(gap_kernel, dim3((unsigned)((q.C + 3) / 4), B), blk, 0, s, q); break;
  case kBmm: launch_bmm_mfma(q, s); break;
  case kBiasAdd: hipLaunchKernelGGL(bias_add_kernel, dim3(nblk(q.n, 256), B), blk, 0, s, q); break;
  default: break;
  }
}

// ------------------------------------------------------------------ fused head decode
// The plan's Detect / Pose decode tail (DFL softmax + bin projection, dist2bbox x strides,
// sigmoid classes, keypoints (xy * c + (anchors - 0.5)) x strides and sigmoid visibility)
// for one anchor of one image per thread; the node chain it replaces is described at the
// executor's fuseDecode pass.  Every value a node of the chain would store is rounded to
// fp16 here too (rh), with each node's fp32 formula (softmax_kernel, the 1x1 projection,
// binop, act_f), so the output is the chain's up to the order of the projection's fp32 sum.
namespace {
__device__ __forceinline__ float rh(float v) { return (float)(_Float16)v; }
__device__ __forceinline__ float hv(const __half * p, long i) { return (float)reinterpret_cast<const _Float16 *>(p)[i]; }

// R_ / NC_ / NK_ > 0: compile-time channel counts (loops unroll, fx / fk index registers);
// 0: the run-time counts in p.
template <int R_, int NC_, int NK_, class FX, class FC, class FK>
__device__ __forceinline__ void decode_anchor(const DecodeParams & p, int b, int a, FX && fx, FC && fc, FK && fk)
{
  const int R = R_ > 0 ? R_ : p.R, nc = NC_ > 0 ? NC_ : p.nc, nk = NK_ > 0 ? NK_ : p.nk;
  _Float16 * y = reinterpret_cast<_Float16 *>(p.y.ptr) + (long)b * p.y.img + a;
  const long ys = p.y.cs;
  const float ax = hv(p.anc, a), ay = hv(p.anc, (long)p.A + a), st = hv(p.st, a);
  float d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float m = -3.4e38f;
#pragma unroll
    for (int k = 0; k < R; ++k) m = fmaxf(m, fx(j * R + k));
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < R; ++k) s += __expf(fx(j * R + k) - m);
    const float inv = 1.0f / s;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < R; ++k) acc += hv(p.dflw, k) * rh(__expf(fx(j * R + k) - m) * inv);
    d[j] = rh(acc);
  }
  const float x1 = rh(ax - d[0]), y1 = rh(ay - d[1]), x2 = rh(ax + d[2]), y2 = rh(ay + d[3]);
  const float cb = hv(p.cbox, 0);
  const float sx = rh(x1 + x2), sy = rh(y1 + y2);
  const float cx = rh(p.box_div ? sx / cb : sx * cb), cy = rh(p.box_div ? sy / cb : sy * cb);
  y[0] = (_Float16)(cx * st);
  y[ys] = (_Float16)(cy * st);
  y[2 * ys] = (_Float16)(rh(x2 - x1) * st);
  y[3 * ys] = (_Float16)(rh(y2 - y1) * st);
#pragma unroll
  for (int c = 0; c < nc; ++c) y[(4 + c) * ys] = (_Float16)act_f(fc(c), kActSigmoid);
  if (nk > 0) {
    const float ck = hv(p.ckpt, 0), mx = hv(p.ancm, a), my = hv(p.ancm, (long)p.A + a);
    _Float16 * yk = y + (4 + nc) * ys;
    for (int k = 0; k < nk; ++k) {
      yk[(3 * k) * ys] = (_Float16)(rh(rh(fk(3 * k) * ck) + mx) * st);
      yk[(3 * k + 1) * ys] = (_Float16)(rh(rh(fk(3 * k + 1) * ck) + my) * st);
      yk[(3 * k + 2) * ys] = (_Float16)act_f(fk(3 * k + 2), kActSigmoid);
    }
  }
}

__device__ __forceinline__ View pick_view(const View (&v)[4], int s)
{
  View r = v[0];
  if (s >= 1) r = v[1];
  if (s >= 2) r = v[2];
  if (s >= 3) r = v[3];
  return r;
}

__device__ __forceinline__ int decode_scale(const DecodeParams & p, int a)
{
  int s = 0;
  if (p.nscale > 1 && a >= p.off[1]) s = 1;
  if (p.nscale > 2 && a >= p.off[2]) s = 2;
  if (p.nscale > 3 && a >= p.off[3]) s = 3;
  return s;
}

// NCHW heads, compile-time channel counts: each channel is one 2-byte load per lane,
// consecutive lanes on consecutive pixels (coalesced), every channel read once
template <int R, int NC, int NK>
__global__ void __launch_bounds__(256) pose_decode_nchw_kernel(const DecodeParams p)
{
  constexpr int NX = 4 * R, NKC = 3 * NK;
  const int a = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
  if (a >= p.A) return;
  const int s = decode_scale(p, a), i = a - p.off[s];
  const View xv = pick_view(p.x, s), cv = pick_view(p.c, s);
  const _Float16 * xp = reinterpret_cast<const _Float16 *>(xv.ptr) + (long)b * xv.img + i;
  const _Float16 * cp = reinterpret_cast<const _Float16 *>(cv.ptr) + (long)b * cv.img + i;
  _Float16 x[NX], cl[NC];
#pragma unroll
  for (int c = 0; c < NX; ++c) x[c] = xp[(long)c * xv.cs];
#pragma unroll
  for (int c = 0; c < NC; ++c) cl[c] = cp[(long)c * cv.cs];
  _Float16 k[NKC > 0 ? NKC : 1];
  if (NK > 0) {
    const View kv = pick_view(p.k, s);
    const _Float16 * kp = reinterpret_cast<const _Float16 *>(kv.ptr) + (long)b * kv.img + i;
#pragma unroll
    for (int c = 0; c < NKC; ++c) k[c] = kp[(long)c * kv.cs];
  }
  decode_anchor<R, NC, NK>(p, b, a, [&](int c) { return (float)x[c]; }, [&](int c) { return (float)cl[c]; },
                           [&](int c) { return (float)k[c]; });
}

// any layout, run-time channel counts (decode_anchor's unroll requests cannot be met here)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
__global__ void __launch_bounds__(256) pose_decode_kernel(const DecodeParams p)
{
  const int a = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
  if (a >= p.A) return;
  const int s = decode_scale(p, a), i = a - p.off[s];
  const View xv = pick_view(p.x, s), cv = pick_view(p.c, s), kv = pick_view(p.k, s);
  auto at = [&](const View & v, int c) {
    return hv(v.ptr, (long)b * v.img + (v.layout == kNHWC ? (long)i * v.cs + c : (long)c * v.cs + i));
  };
  decode_anchor<0, 0, 0>(p, b, a, [&](int c) { return at(xv, c); }, [&](int c) { return at(cv, c); },
                         [&](int c) { return at(kv, c); });
}
#pragma clang diagnostic pop
}  // namespace

void launch_pose_decode(const DecodeParams & p, hipStream_t s)
{
  const dim3 grid((unsigned)((p.A + 255) / 256), (unsigned)p.batch), blk(256);
  if (p.nchw && p.R == 16 && p.nc == 1 && p.nk == 17)
    hipLaunchKernelGGL((pose_decode_nchw_kernel<16, 1, 17>), grid, blk, 0, s, p);
  else if (p.nchw && p.R == 16 && p.nc == 80 && p.nk == 0)
    hipLaunchKernelGGL((pose_decode_nchw_kernel<16, 80, 0>), grid, blk, 0, s, p);
  else
    hipLaunchKernelGGL(pose_decode_kernel, grid, blk, 0, s, p);
}

// ------------------------------------------------------------- boundary conversions
// f32 -> f16 exactly as include/infvino/Half.hpp:14-24: truncate the mantissa, flush
// results with exponent <= 0 to signed zero, saturate exponent >= 31 (NaN too) to inf.
__global__ void f32_to_f16_trunc_kernel(const float * in, uint16_t * out, long n)
{
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t x = __float_as_uint(in[i]);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int exp = (int)((x >> 23) & 0xffu) - 112;
  uint32_t h;
  if (exp <= 0) h = sign;
  else if (exp >= 31) h = sign | 0x7c00u;
  else h = sign | ((uint32_t)exp << 10) | ((x & 0x7fffffu) >> 13);
  out[i] = (uint16_t)h;
}

__global__ void f16_to_f32_kernel(const __half * in, float * out, long n)
{
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = (float)reinterpret_cast<const _Float16 *>(in)[i];
}

void launch_f32_to_f16_trunc(const float * in, __half * out, long n, hipStream_t s)
{
  hipLaunchKernelGGL(f32_to_f16_trunc_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, in,
                     reinterpret_cast<uint16_t *>(out), n);
}

// Staging area of the allocation-free f32 input conversion (ivh_set_input_f32_noalloc): a
// fixed array in every GPU's memory, so that path needs no hipMalloc.  Host code must not use
// the array's name as an address (it names a host-side shadow); boundary_scratch() returns
// the device address of the current GPU's copy, resolved once per device.
static __device__ __align__(256) float scratch[kBoundaryScratchFloats];

namespace {
std::mutex & scratch_map_mutex()
{
  static std::mutex mu;
  return mu;
}
}  // namespace

std::mutex & boundary_scratch_lock(int device)
{
  static std::map<int, std::unique_ptr<std::mutex>> lock_of;
  std::lock_guard<std::mutex> lock(scratch_map_mutex());
  auto & m = lock_of[device];
  if (!m) m = std::make_unique<std::mutex>();
  return *m;
}

float * boundary_scratch(int device)
{
  static std::map<int, float *> ptr_of;
  std::lock_guard<std::mutex> lock(scratch_map_mutex());
  const auto it = ptr_of.find(device);
  if (it != ptr_of.end()) return it->second;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != device)
    throw std::runtime_error("HIP error: boundary scratch asked for device " + std::to_string(device) +
                             " while another is current");
  void * ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    throw std::runtime_error(std::string("HIP error: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  ptr_of[device] = static_cast<float *>(ptr);
  return static_cast<float *>(ptr);
}

void launch_f16_to_f32(const __half * in, float * out, long n, hipStream_t s)
{
  hipLaunchKernelGGL(f16_to_f32_kernel, dim3(nblk(n, 256)), dim3(256), 0, s, in, out, n);
}

}  // namespace ivh
