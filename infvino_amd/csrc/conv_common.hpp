// Device-side pieces shared by the MFMA convolution kernels: fragment types, the two gfx950
// fp16 MFMA shapes behind one interface, the activation formulas and the fused epilogue.
#pragma once

#include <type_traits>

#include "ivh_internal.hpp"

namespace ivh {

// fn(integral_constant<int, i>) for i = B .. E - 1: a loop the compiler cannot leave rolled
template <int B, int E, class Fn> __device__ __forceinline__ void static_for(Fn && fn)
{
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    static_for<B + 1, E>(fn);
  }
}

// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding)
constexpr int kVmWait0 = (0x7 << 4) | (0xf << 8);
// s_waitcnt vmcnt(n), 0 <= n < 64, the other counters left alone
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// Raw buffer resources (gfx9 family): dword3 of a plain byte-addressed buffer, and an
// offset at or past 2^31 bytes, which is outside every range used here (the host keeps
// buffer views below 2^31 bytes) so such a load returns zeros.
constexpr int kBufDword3 = 0x00020000;
constexpr unsigned kBufOOB = 0x80000000u;

// n / d for 0 <= n < 2^22 and 1 <= d < 2^22 with inv = 1/d (float): the float quotient is
// within 1 of the exact one, and one correction step makes it exact.  Used for tile and
// image index arithmetic, where a full integer division would cost ~25 VALU instructions.
__device__ __forceinline__ int idiv_small(int n, int d, float inv)
{
  int q = (int)((float)n * inv);
  const int r = n - (int)__umul24((unsigned)q, (unsigned)d);  // q, d < 2^24: a full-rate multiply
  q += (r >= d) - (r < 0);
  return q;
}

// n / d with f = fastdiv_make(d): see FastDiv.
__device__ __forceinline__ unsigned fastdiv(unsigned n, FastDiv f)
{
  return (unsigned)(((unsigned long long)__umulhi(n, f.m) + n) >> f.l);
}

// Work-group w of a launch is dispatched to XCD w % 8, and each XCD has its own L2.  This
// maps the hardware order to a tile order in which every XCD owns one contiguous range of
// tiles (a bijection on [0, n)), so neighbouring tiles -- which share input rows -- run on
// the same XCD and hit its L2 instead of HBM.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_tile(int w, int n)
{
  const int per = n / kXcds, rem = n - per * kXcds;
  const int x = w % kXcds, i = w / kXcds;
  return x * per + (x < rem ? x : rem) + i;
}

// Activation codes and formulas of the reference epilogues (kernels/gemm.cl:137-154,
// conv_ov.cl:121-131, conv_general.cl:71-83), evaluated in fp32.
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

// The same formulas for the MFMA epilogues, with the hardware reciprocal (v_rcp_f32, about
// 1 ulp) in place of the IEEE division and 1/6 as a multiplier: a few fp32 ulps from act_f,
// far below the fp16 rounding that follows.
template <int ACT>
__device__ __forceinline__ float act_fast(float v)
{
  if (ACT == kActSiLU) return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
  if (ACT == kActReLU) return fmaxf(v, 0.0f);
  if (ACT == kActHSwish) return v * fminf(fmaxf(v + 3.0f, 0.0f), 6.0f) * (1.0f / 6.0f);
  if (ACT == kActHSigmoid) return fminf(fmaxf(v + 3.0f, 0.0f), 6.0f) * (1.0f / 6.0f);
  if (ACT == kActSigmoid) return __builtin_amdgcn_rcpf(1.0f + __expf(-v));
  return v;
}

// MFMA block of MB x MB outputs.  Operand A = weights (row i = output channel), operand B =
// pixels (column j = pixel); each lane supplies 8 consecutive K values of one row / column.
//   MB = 32: v_mfma_f32_32x32x16_f16, K slice 16, lane k offset 8*(lane/32);
//            D: lane holds column lane%32, rows 8*(v/4) + 4*(lane/32) + v%4, v < 16
//   MB = 16: v_mfma_f32_16x16x32_f16, K slice 32, lane k offset 8*(lane/16);
//            D: lane holds column lane%16, rows 4*(lane/16) + v, v < 4
template <int MB> struct Mf;
template <> struct Mf<32> {
  typedef float acc_t __attribute__((ext_vector_type(16)));
  static constexpr int KD = 16, NV = 16;
  static __device__ __forceinline__ int kq(int lane) { return (lane >> 5) * 8; }
  static __device__ __forceinline__ int col(int lane) { return lane & 31; }
  static __device__ __forceinline__ int row(int lane, int v) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }
  static __device__ __forceinline__ acc_t mma(h8 a, h8 b, acc_t c)
  {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mf<16> {
  typedef float acc_t __attribute__((ext_vector_type(4)));
  static constexpr int KD = 32, NV = 4;
  static __device__ __forceinline__ int kq(int lane) { return (lane >> 4) * 8; }
  static __device__ __forceinline__ int col(int lane) { return lane & 15; }
  static __device__ __forceinline__ int row(int lane, int v) { return 4 * (lane >> 4) + v; }
  static __device__ __forceinline__ acc_t mma(h8 a, h8 b, acc_t c)
  {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Work-group tile: 4 waves as WGM (pixels) x WGN (channels), each wave TM x TN MFMA blocks.
template <int MB, int WGM, int WGN, int TM, int TN>
struct TileShape {
  static_assert(WGM * WGN == 4, "four waves per work-group");
  static constexpr int BM = WGM * TM * MB;  // pixel slots
  static constexpr int BN = WGN * TN * MB;  // output channels
  // LDS halves the epilogue stages the tile in (channels-last rows or channel-major rows)
  static constexpr int EPI = (BM * (BN + 8) > BN * (BM + 8)) ? BM * (BN + 8) : BN * (BM + 8);
};

// Bias of a lane's accumulator rows: runs of 4 rows are 4 consecutive channels, one 16-byte
// load each (the MFMA families' bias is zero padded to a multiple of 128 channels).
template <int MB, int WGM, int WGN, int TM, int TN>
__device__ __forceinline__ void load_bias(const ConvParams & p, int n0, float (&bv)[TN][Mf<MB>::NV])
{
  using F = Mf<MB>;
  const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) / WGM;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int v4 = 0; v4 < F::NV; v4 += 4) {
      float4 b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (p.bias) b4 = *reinterpret_cast<const float4 *>(p.bias + n0 + wn * TN * MB + tn * MB + F::row(lane, v4));
      bv[tn][v4] = b4.x;
      bv[tn][v4 + 1] = b4.y;
      bv[tn][v4 + 2] = b4.z;
      bv[tn][v4 + 3] = b4.w;
    }
}

// Epilogue phase 1: bias + activation (compile-time code) in fp32, one rounding to fp16,
// tile into LDS as [pixel][channel] (NHWC output) or [channel][pixel] (NCHW output).
template <int ACT, int MB, int WGM, int WGN, int TM, int TN>
__device__ __forceinline__ void stage_tile(typename Mf<MB>::acc_t (&acc)[TN][TM], const float (&bv)[TN][Mf<MB>::NV],
                                           _Float16 * lds, bool nhwc)
{
  using F = Mf<MB>;
  using T = TileShape<MB, WGM, WGN, TM, TN>;
  constexpr int BM = T::BM, BN = T::BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int pl = wm * TM * MB + tm * MB + F::col(lane);
      // runs of 4 accumulator values are 4 consecutive channels (both MFMA layouts)
#pragma unroll
      for (int v4 = 0; v4 < F::NV; v4 += 4) {
        const int cl = wn * TN * MB + tn * MB + F::row(lane, v4);
        h4 hv;
#pragma unroll
        for (int k = 0; k < 4; ++k) hv[k] = (_Float16)act_fast<ACT>(acc[tn][tm][v4 + k] + bv[tn][v4 + k]);
        if (nhwc) {
          *reinterpret_cast<h4 *>(lds + pl * (BN + 8) + cl) = hv;
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) lds[(cl + k) * (BM + 8) + pl] = hv[k];
        }
      }
    }
  }
}

// Fused epilogue: bias + activation in fp32, one rounding to fp16, then (+ residual) --
// the reference order act(acc + b) + r (gemm.cl:644-650, conv_ov.cl:285-288).  The tile is
// staged in LDS and written with 16-byte stores (NHWC along channels, NCHW along pixels).
// pix(pl, b, hw): tile pixel slot pl -> image b, output pixel hw; false when outside.
// With p.ksplit > 1 the fp32 partials go to the workspace [kz][co][pixel] instead.
// tile_epilogue_bv takes the bias values already loaded (load_bias), for kernels whose
// loads of the next tile are in flight during the epilogue.
template <int MB, int WGM, int WGN, int TM, int TN, class PixFn>
__device__ __forceinline__ void tile_epilogue_bv(typename Mf<MB>::acc_t (&acc)[TN][TM],
                                                 const float (&bv)[TN][Mf<MB>::NV], const ConvParams & p,
                                                 _Float16 * lds, int n0, int kz, PixFn pix)
{
  using F = Mf<MB>;
  using T = TileShape<MB, WGM, WGN, TM, TN>;
  constexpr int BM = T::BM, BN = T::BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int HWo = p.Ho * p.Wo;
  const long M = (long)p.batch * HWo;

  if (p.ksplit > 1) {
    const int Npad = gridDim.y * BN;
    float * wsz = p.ws + (long)kz * Npad * M;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        int b, hw;
        if (!pix(wm * TM * MB + tm * MB + F::col(lane), b, hw)) continue;
        const long pm = (long)b * HWo + hw;
#pragma unroll
        for (int v = 0; v < F::NV; ++v) {
          const int co = n0 + wn * TN * MB + tn * MB + F::row(lane, v);
          wsz[(long)co * M + pm] = acc[tn][tm][v];
        }
      }
    return;
  }

  const bool nhwc = p.y.layout == kNHWC;
  switch (p.act) {
  case kActSiLU: stage_tile<kActSiLU, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  case kActReLU: stage_tile<kActReLU, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  case kActHSwish: stage_tile<kActHSwish, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  case kActHSigmoid: stage_tile<kActHSigmoid, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  case kActSigmoid: stage_tile<kActSigmoid, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  default: stage_tile<kActNone, MB, WGM, WGN, TM, TN>(acc, bv, lds, nhwc); break;
  }
  __syncthreads();

  const _Float16 * rbase = reinterpret_cast<const _Float16 *>(p.r.ptr);
  _Float16 * ybase = reinterpret_cast<_Float16 *>(p.y.ptr);
  if (nhwc) {
    const bool yvec = ((p.y.cs | (int)(reinterpret_cast<uintptr_t>(ybase) >> 1) | (int)p.y.img) & 7) == 0;
    const bool rvec = !rbase || (p.r.layout == kNHWC &&
                      ((p.r.cs | (int)(reinterpret_cast<uintptr_t>(rbase) >> 1) | (int)p.r.img) & 7) == 0);
    constexpr int CPR = BN / 8 > 0 ? BN / 8 : 1;
    for (int c = tid; c < BM * CPR; c += 256) {
      const int pl = c / CPR, c8 = (c % CPR) * 8;
      const int co = n0 + c8;
      int b, hw;
      if (co >= p.Cout || !pix(pl, b, hw)) continue;
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
    const bool yvec = ((p.y.cs | (int)(reinterpret_cast<uintptr_t>(ybase) >> 1) | (int)p.y.img) & 7) == 0;
    const bool rvec = !rbase || (p.r.layout == kNCHW &&
                      ((p.r.cs | (int)(reinterpret_cast<uintptr_t>(rbase) >> 1) | (int)p.r.img) & 7) == 0);
    constexpr int PPR = BM / 8;
    for (int c = tid; c < BN * PPR; c += 256) {
      const int cl = c / PPR, p8 = (c % PPR) * 8;
      const int co = n0 + cl;
      if (co >= p.Cout) continue;
      h8 v = *reinterpret_cast<const h8 *>(lds + cl * (BM + 8) + p8);
      int b0, h0, b7, h7;
      const bool v0 = pix(p8, b0, h0), v7 = pix(p8 + 7, b7, h7);
      if (v0 && v7 && b0 == b7 && h7 - h0 == 7 && (h0 & 7) == 0 && yvec && rvec) {
        if (rbase) {
          const h8 rv = *reinterpret_cast<const h8 *>(rbase + (long)b0 * p.r.img + (long)co * p.r.cs + h0);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)rv[e]);
        }
        *reinterpret_cast<h8 *>(ybase + (long)b0 * p.y.img + (long)co * p.y.cs + h0) = v;
      } else {
        for (int e = 0; e < 8; ++e) {
          int bq, hq;
          if (!pix(p8 + e, bq, hq)) continue;
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

// Fused epilogue with the bias loaded here (the common case).
template <int MB, int WGM, int WGN, int TM, int TN, class PixFn>
__device__ __forceinline__ void tile_epilogue(typename Mf<MB>::acc_t (&acc)[TN][TM], const ConvParams & p,
                                              _Float16 * lds, int n0, int kz, PixFn pix)
{
  float bv[TN][Mf<MB>::NV];
  load_bias<MB, WGM, WGN, TM, TN>(p, n0, bv);
  tile_epilogue_bv<MB, WGM, WGN, TM, TN>(acc, bv, p, lds, n0, kz, pix);
}

}  // namespace ivh
