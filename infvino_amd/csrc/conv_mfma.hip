// Implicit-GEMM convolution on gfx950 fp16 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulate.
//
// Replaces, for conv1x1 / conv3x3 / conv_general with 8-aligned NHWC input, the reference
// kernels gemm_f16 (kernels/gemm.cl:183-669), gemm_sk_f16 (gemm_sk.cl:75-175),
// conv1x1_blk (conv1x1_blk.cl:142-330), conv3x3_ov (conv_ov.cl:133-297), conv3x3_blk
// (conv_blk.cl:118-296) and conv3x3_f16 (conv.cl:150-414): same math
//   y[co][p] = act(sum_k W[co][k] * im2col(x)[k][p] + b[co]) (+ r[co][p])
// with the residual added after the activation (gemm.cl:644-650, conv_ov.cl:285-288).
//
// GEMM mapping (MI355X-first, not a translation):
//   M = output pixels of ALL images in the batch (batch is the parallel axis),
//   N = output channels, K = (ky, kx, ci) with ci padded to a multiple of 8 so that every
//   8-element K chunk is one 16-byte NHWC load of one input pixel.
//   The MFMA computes D[co][pixel]: operand A = weight fragment, operand B = pixel fragment.
// Work-group: 4 waves (256 lanes), tile BM pixels x BN channels, each wave TM x TN 32x32
// MFMA blocks.  The im2col A tile and the weight B tile are staged global -> registers ->
// LDS (double buffered, one barrier per K step, next tile's global loads in flight while
// the current tile feeds the MFMAs).  The epilogue applies bias + activation in fp32,
// rounds once to fp16, stages the tile in LDS and stores 16-byte vectors (NHWC: along
// channels, NCHW: along pixels), adding the residual in that coalesced pass.
#include "ivh_internal.hpp"
#include "kernels.hpp"

namespace ivh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float act_f(float v, int act)
{
  switch (act) {
  case kActSiLU: return v / (1.0f + __expf(-v));
  case kActReLU: return fmaxf(v, 0.0f);
  case kActHSwish: return v * fminf(fmaxf(v + 3.0f, 0.0f), 6.0f) / 6.0f;
  case kActHSigmoid: return fminf(fmaxf(v + 3.0f, 0.0f), 6.0f) / 6.0f;
  case kActSigmoid: return 1.0f / (1.0f + __expf(-v));
  default: return v;
  }
}

template <int WGM, int WGN, int TM, int TN, int BK>
struct IgemmShape {
  static constexpr int BM = WGM * TM * 32;
  static constexpr int BN = WGN * TN * 32;
  static constexpr int LDK = BK + 8;  // padded LDS row: 16B-read conflict free
  static constexpr int KCH = BK / 8;
  static constexpr int A_IT = BM * KCH / 256;
  static constexpr int B_IT = (BN * KCH + 255) / 256;  // BN = 32: half the lanes load B
  static constexpr int STAGE = 2 * (BM + BN) * LDK;  // halves, both operand buffers
  static constexpr int OUT_NHWC = BM * (BN + 8);     // halves, epilogue tile [pixel][co]
  static constexpr int OUT_NCHW = BN * (BM + 8);     // halves, epilogue tile [co][pixel]
  static constexpr int LDS = STAGE > OUT_NHWC ? (STAGE > OUT_NCHW ? STAGE : OUT_NCHW)
                                              : (OUT_NHWC > OUT_NCHW ? OUT_NHWC : OUT_NCHW);
};

template <int WGM, int WGN, int TM, int TN, int BK>
__global__ void __launch_bounds__(256) conv_igemm_kernel(const ConvParams p)
{
  using S = IgemmShape<WGM, WGN, TM, TN, BK>;
  constexpr int BM = S::BM, BN = S::BN, LDK = S::LDK, KCH = S::KCH;
  static_assert(WGM * WGN == 4, "four waves per work-group");
  static_assert((BM * KCH) % 256 == 0 && (256 % KCH) == 0, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) _Float16 lds[S::LDS];
  _Float16 * As = lds;                    // [2][BM][LDK]
  _Float16 * Bs = lds + 2 * BM * LDK;     // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int HWo = p.Ho * p.Wo;
  const long M = (long)p.batch * HWo;
  const long m0 = (long)blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;

  // ---- A (im2col) load slots: thread owns rows r_i = tid/KCH + i*(256/KCH), chunk kc.
  const int kc = tid % KCH;
  const _Float16 * arow[S::A_IT];
  int aiy[S::A_IT], aix[S::A_IT];
#pragma unroll
  for (int i = 0; i < S::A_IT; ++i) {
    const long pm = m0 + tid / KCH + i * (256 / KCH);
    if (pm < M) {
      const int b = (int)(pm / HWo), hw = (int)(pm - (long)b * HWo);
      const int oy = hw / p.Wo, ox = hw - oy * p.Wo;
      arow[i] = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)b * p.x.img;
      aiy[i] = oy * p.S - p.P;
      aix[i] = ox * p.S - p.P;
    } else {
      arow[i] = nullptr;
      aiy[i] = -100000;
      aix[i] = -100000;
    }
  }
  // K range of this work-group (split-K: blockIdx.z-th slice of the K tiles)
  const int nk_all = p.kpad / BK;
  const int per = (nk_all + p.ksplit - 1) / p.ksplit;
  const int kt0 = blockIdx.z * per;
  const int kt1 = kt0 + per < nk_all ? kt0 + per : nk_all;
  // K position of this thread's chunk: tap (ky,kx) and channel ci, advanced by BK per step.
  const int taps = p.K * p.K;
  int ci = kt0 * BK + kc * 8, tap = 0, ky = 0, kx = 0;
  auto norm_k = [&]() {
    while (ci >= p.cin8) {
      ci -= p.cin8;
      ++tap;
      if (++kx == p.K) { kx = 0; ++ky; }
    }
  };
  norm_k();

  const _Float16 * wbase = reinterpret_cast<const _Float16 *>(p.w);
  const bool ragged = (p.Cin & 7) != 0;

  h8 ra[S::A_IT], rb[S::B_IT];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < S::A_IT; ++i) {
      h8 v = {};
      if (tap < taps) {
        const int iy = aiy[i] + ky, ix = aix[i] + kx;
        if ((unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W) {
          v = *reinterpret_cast<const h8 *>(arow[i] + ((long)iy * p.W + ix) * p.x.cs + ci);
          if (ragged) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (ci + e >= p.Cin) v[e] = (_Float16)0.0f;
          }
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < S::B_IT; ++i) {
      const int r = tid / KCH + i * (256 / KCH);
      if (r < BN) rb[i] = *reinterpret_cast<const h8 *>(wbase + (long)(n0 + r) * p.kpad + kt * BK + kc * 8);
    }
    ci += BK;
    norm_k();
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < S::A_IT; ++i) {
      const int r = tid / KCH + i * (256 / KCH);
      *reinterpret_cast<h8 *>(As + (buf * BM + r) * LDK + kc * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < S::B_IT; ++i) {
      const int r = tid / KCH + i * (256 / KCH);
      if (r < BN) *reinterpret_cast<h8 *>(Bs + (buf * BN + r) * LDK + kc * 8) = rb[i];
    }
  };

  f16v acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  const int nk = kt1 - kt0;
  if (nk > 0) {
    load_tile(kt0);
    store_tile(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile(kt0 + kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      h8 fa[TN], fb[TM];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        fa[tn] = *reinterpret_cast<const h8 *>(
          Bs + (cur * BN + wn * TN * 32 + tn * 32 + (lane & 31)) * LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        fb[tm] = *reinterpret_cast<const h8 *>(
          As + (cur * BM + wm * TM * 32 + tm * 32 + (lane & 31)) * LDK + kk * 16 + (lane >> 5) * 8);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[tn], fb[tm], acc[tn][tm], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- split-K: fp32 partials to the workspace [z][co][pixel]; the reduce kernel finishes
  if (p.ksplit > 1) {
    const int Npad = gridDim.y * BN;
    float * wsz = p.ws + (long)blockIdx.z * Npad * M;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const long pm = m0 + wm * TM * 32 + tm * 32 + (lane & 31);
        if (pm >= M) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int co = n0 + wn * TN * 32 + tn * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          wsz[(long)co * M + pm] = acc[tn][tm][v];
        }
      }
    return;
  }

  // ---- epilogue phase 1: bias + activation in fp32, one rounding, tile into LDS.
  // D layout of 32x32 MFMA: lane holds column j = lane%32 (pixel) and rows
  // i = 8*(v/4) + 4*(lane/32) + v%4 (output channel) for v = 0..15.
  const bool nhwc = p.y.layout == kNHWC;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int pl = wm * TM * 32 + tm * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int cl = wn * TN * 32 + tn * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int co = n0 + cl;
        float val = acc[tn][tm][v];
        if (p.bias && co < p.Cout) val += p.bias[co];
        val = act_f(val, p.act);
        const _Float16 hv = (_Float16)val;
        if (nhwc) lds[pl * (BN + 8) + cl] = hv;
        else lds[cl * (BM + 8) + pl] = hv;
      }
    }
  __syncthreads();

  // ---- epilogue phase 2: coalesced 16-byte stores (+ residual, added after activation).
  const _Float16 * rbase = reinterpret_cast<const _Float16 *>(p.r.ptr);
  _Float16 * ybase = reinterpret_cast<_Float16 *>(p.y.ptr);
  if (nhwc) {
    const bool yvec = ((p.y.cs | (int)(reinterpret_cast<uintptr_t>(ybase) >> 1) | (int)p.y.img) & 7) == 0;
    const bool rvec = !rbase || (p.r.layout == kNHWC &&
                      ((p.r.cs | (int)(reinterpret_cast<uintptr_t>(rbase) >> 1) | (int)p.r.img) & 7) == 0);
    constexpr int CPR = BN / 8;  // 16-byte chunks per pixel row
    for (int c = tid; c < BM * CPR; c += 256) {
      const int pl = c / CPR, c8 = (c % CPR) * 8;
      const long pm = m0 + pl;
      const int co = n0 + c8;
      if (pm >= M || co >= p.Cout) continue;
      const int b = (int)(pm / HWo), hw = (int)(pm - (long)b * HWo);
      h8 v = *reinterpret_cast<const h8 *>(lds + pl * (BN + 8) + c8);
      const int nv = p.Cout - co < 8 ? p.Cout - co : 8;
      if (rbase) {
        if (rvec && nv == 8) {
          const h8 rv = *reinterpret_cast<const h8 *>(rbase + (long)b * p.r.img + (long)hw * p.r.cs + co);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)rv[e]);
        } else {
          for (int e = 0; e < nv; ++e) {
            const long ri = p.r.layout == kNHWC ? (long)hw * p.r.cs + co + e : (long)(co + e) * p.r.cs + hw;
            v[e] = (_Float16)((float)v[e] + (float)rbase[(long)b * p.r.img + ri]);
          }
        }
      }
      _Float16 * yp = ybase + (long)b * p.y.img + (long)hw * p.y.cs + co;
      if (yvec && nv == 8) *reinterpret_cast<h8 *>(yp) = v;
      else
        for (int e = 0; e < nv; ++e) yp[e] = v[e];
    }
  } else {
    const bool yvec = ((HWo | p.y.cs | (int)(reinterpret_cast<uintptr_t>(ybase) >> 1) | (int)p.y.img) & 7) == 0;
    const bool rvec = !rbase || (p.r.layout == kNCHW &&
                      ((HWo | p.r.cs | (int)(reinterpret_cast<uintptr_t>(rbase) >> 1) | (int)p.r.img) & 7) == 0);
    constexpr int PPR = BM / 8;  // 16-byte chunks per channel row
    for (int c = tid; c < BN * PPR; c += 256) {
      const int cl = c / PPR, p8 = (c % PPR) * 8;
      const int co = n0 + cl;
      const long pm = m0 + p8;
      if (co >= p.Cout || pm >= M) continue;
      h8 v = *reinterpret_cast<const h8 *>(lds + cl * (BM + 8) + p8);
      const int b = (int)(pm / HWo), hw = (int)(pm - (long)b * HWo);
      if (yvec && rvec && pm + 8 <= M) {
        // HWo % 8 == 0 and pm % 8 == 0: the 8 pixels lie in one image, contiguous
        if (rbase) {
          const h8 rv = *reinterpret_cast<const h8 *>(rbase + (long)b * p.r.img + (long)co * p.r.cs + hw);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)rv[e]);
        }
        *reinterpret_cast<h8 *>(ybase + (long)b * p.y.img + (long)co * p.y.cs + hw) = v;
      } else {
        for (int e = 0; e < 8; ++e) {
          const long q = pm + e;
          if (q >= M) break;
          const int bq = (int)(q / HWo), hq = (int)(q - (long)bq * HWo);
          float o = (float)v[e];
          if (rbase) {
            const long ri = p.r.layout == kNHWC ? (long)hq * p.r.cs + co : (long)co * p.r.cs + hq;
            o += (float)rbase[(long)bq * p.r.img + ri];
          }
          ybase[(long)bq * p.y.img + (long)co * p.y.cs + hq] = (_Float16)o;
        }
      }
    }
  }
}

// Split-K finish: y = act(sum_z ws[z] + b) (+ r), partials summed in fixed z order so the
// result does not depend on scheduling.  One lane per (channel, pixel), pixels fastest.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const ConvParams p, int npad)
{
  const int HWo = p.Ho * p.Wo;
  const long M = (long)p.batch * HWo;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * p.Cout) return;
  const int co = (int)(i / M);
  const long pm = i - (long)co * M;
  float v = 0.0f;
  for (int z = 0; z < p.ksplit; ++z) v += p.ws[((long)z * npad + co) * M + pm];
  if (p.bias) v += p.bias[co];
  v = act_f(v, p.act);
  const int b = (int)(pm / HWo), hw = (int)(pm - (long)b * HWo);
  const _Float16 hv = (_Float16)v;  // one rounding before the residual, as the fused epilogue
  float o = (float)hv;
  if (p.r.ptr) {
    const long ri = p.r.layout == kNHWC ? (long)hw * p.r.cs + co : (long)co * p.r.cs + hw;
    o += (float)reinterpret_cast<const _Float16 *>(p.r.ptr)[(long)b * p.r.img + ri];
  }
  const long yi = p.y.layout == kNHWC ? (long)hw * p.y.cs + co : (long)co * p.y.cs + hw;
  reinterpret_cast<_Float16 *>(p.y.ptr)[(long)b * p.y.img + yi] = (_Float16)o;
}

// ---------------------------------------------------------------- host side

// Tile table: a small CDNA4 choice per op (BN from Cout; BM = 128 pixels).
// Each entry is (WGM, WGN, TM, TN), BK = 32.
int igemm_bn(int cout) { return cout <= 32 ? 32 : (cout <= 64 ? 64 : 128); }

template <int WGM, int WGN, int TM, int TN>
static void launch_t(const ConvParams & p, hipStream_t s)
{
  using Sh = IgemmShape<WGM, WGN, TM, TN, 32>;
  const long M = (long)p.batch * p.Ho * p.Wo;
  dim3 grid((unsigned)((M + Sh::BM - 1) / Sh::BM), (unsigned)((p.Cout + Sh::BN - 1) / Sh::BN),
            (unsigned)p.ksplit);
  hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN, 32>), grid, dim3(256), 0, s, p);
  if (p.ksplit > 1) {
    const long n = M * p.Cout;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p,
                       (int)grid.y * Sh::BN);
  }
}

// Split-K factor: convs whose output tiles cannot fill the chip (batch 1, 20x20 / 40x40
// feature maps) and whose K loop is long get their K range split across work-groups.
int igemm_ksplit(long M, int cout, int kpad)
{
  const int bn = igemm_bn(cout);
  const long tiles = ((M + 127) / 128) * ((cout + bn - 1) / bn);
  const int nk = kpad / kIgemmBK;
  if (tiles >= 192 || nk < 8) return 1;
  int s = (int)((384 + tiles - 1) / tiles);
  s = s < nk / 4 ? s : nk / 4;
  s = s < 16 ? s : 16;
  return s < 2 ? 1 : s;
}

void launch_conv_igemm(const ConvParams & p, hipStream_t s)
{
  switch (igemm_bn(p.Cout)) {
  case 32: launch_t<4, 1, 1, 1>(p, s); break;
  case 64: launch_t<2, 2, 2, 1>(p, s); break;
  default: launch_t<2, 2, 2, 2>(p, s); break;
  }
}

}  // namespace ivh
