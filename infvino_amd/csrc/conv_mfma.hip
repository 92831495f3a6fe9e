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
//   N = output channels, K = (ky, kx, ci).  The MFMA computes D[co][pixel]: operand A is a
//   weight fragment, operand B a pixel fragment, both 8 consecutive K values per lane, i.e.
//   one 16-byte load of a channels-last pixel.
// Work-group: 4 waves (256 lanes), tile BM = 128 pixels x BN channels, each wave TM x TN
// 32x32 MFMA blocks.  Two A-operand feeds:
//   conv_igemm_kernel   - linear pixel tiles, the im2col tile gathered from global memory
//                         (any K, stride, pad; every input pixel is re-read per tap from L2)
//   conv3x3_halo_kernel - 3x3 stride 1: a TH x TW output tile; per 32-channel chunk the
//                         (TH+2) x (TW+2) input patch is staged once in LDS and all nine
//                         taps read their fragments from it (no per-tap global re-reads)
// Weight tiles and patches are double buffered (one barrier per K step, next step's global
// loads in flight during the current MFMAs).  The epilogue applies bias + activation in
// fp32, rounds once to fp16, stages the tile in LDS and stores 16-byte vectors (NHWC along
// channels, NCHW along pixels), adding the residual in that coalesced pass.  With split-K
// the fp32 partials go to a workspace instead and splitk_reduce_kernel finishes.
#include "ivh_internal.hpp"
#include "kernels.hpp"

namespace ivh {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
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

template <int WGM, int WGN, int TM, int TN>
struct Tile {
  static constexpr int BM = WGM * TM * 32;
  static constexpr int BN = WGN * TN * 32;
  static constexpr int BK = 32;
  static constexpr int LDK = BK + 8;  // padded LDS row: 16-byte reads conflict free
  static constexpr int KCH = BK / 8;
  static constexpr int OUT = (BM * (BN + 8) > BN * (BM + 8)) ? BM * (BN + 8) : BN * (BM + 8);
};

// ------------------------------------------------------------------ epilogue
// pix(pl, b, hw): local tile pixel pl -> image b, pixel hw; false when outside the output.
template <int WGM, int WGN, int TM, int TN, class PixFn>
__device__ __forceinline__ void igemm_epilogue(f16v (&acc)[TN][TM], const ConvParams & p, _Float16 * lds,
                                               int n0, PixFn pix)
{
  using T = Tile<WGM, WGN, TM, TN>;
  constexpr int BM = T::BM, BN = T::BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int HWo = p.Ho * p.Wo;
  const long M = (long)p.batch * HWo;

  if (p.ksplit > 1) {  // fp32 partials [z][co][pixel]; splitk_reduce_kernel finishes
    const int Npad = gridDim.y * BN;
    float * wsz = p.ws + (long)blockIdx.z * Npad * M;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        int b, hw;
        if (!pix(wm * TM * 32 + tm * 32 + (lane & 31), b, hw)) continue;
        const long pm = (long)b * HWo + hw;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int co = n0 + wn * TN * 32 + tn * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          wsz[(long)co * M + pm] = acc[tn][tm][v];
        }
      }
    return;
  }

  // phase 1: bias + activation in fp32, one rounding, tile into LDS.  D layout of the
  // 32x32 MFMA: lane holds column j = lane%32 (pixel) and rows i = 8*(v/4) + 4*(lane/32)
  // + v%4 (output channel), v = 0..15.
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

  // phase 2: coalesced 16-byte stores (+ residual, added after the activation)
  const _Float16 * rbase = reinterpret_cast<const _Float16 *>(p.r.ptr);
  _Float16 * ybase = reinterpret_cast<_Float16 *>(p.y.ptr);
  if (nhwc) {
    const bool yvec = ((p.y.cs | (int)(reinterpret_cast<uintptr_t>(ybase) >> 1) | (int)p.y.img) & 7) == 0;
    const bool rvec = !rbase || (p.r.layout == kNHWC &&
                      ((p.r.cs | (int)(reinterpret_cast<uintptr_t>(rbase) >> 1) | (int)p.r.img) & 7) == 0);
    constexpr int CPR = BN / 8;
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

// MFMA block product over one 16-deep K slice: A (weights) rows from wrow (row stride
// `wstride` halves per output channel), B (pixels) at per-tile LDS offsets boff[tm].
template <int TM, int TN>
__device__ __forceinline__ void mfma_step(f16v (&acc)[TN][TM], const _Float16 * wrow, const _Float16 * prow,
                                          const int (&boff)[TM], int wstride)
{
  h8 fa[TN], fb[TM];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) fa[tn] = *reinterpret_cast<const h8 *>(wrow + tn * 32 * wstride);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) fb[tm] = *reinterpret_cast<const h8 *>(prow + boff[tm]);
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
      acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[tn], fb[tm], acc[tn][tm], 0, 0, 0);
}

// ------------------------------------------------------------ im2col kernel
template <int WGM, int WGN, int TM, int TN>
__global__ void __launch_bounds__(256) conv_igemm_kernel(const ConvParams p)
{
  using T = Tile<WGM, WGN, TM, TN>;
  constexpr int BM = T::BM, BN = T::BN, BK = T::BK, LDK = T::LDK, KCH = T::KCH;
  constexpr int A_IT = BM * KCH / 256, B_IT = (BN * KCH + 255) / 256;
  constexpr int STAGE = 2 * (BM + BN) * LDK;
  static_assert(WGM * WGN == 4, "four waves per work-group");
  static_assert((BM * KCH) % 256 == 0 && (256 % KCH) == 0, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) _Float16 lds[STAGE > T::OUT ? STAGE : T::OUT];
  _Float16 * As = lds;                 // [2][BM][LDK]
  _Float16 * Bs = lds + 2 * BM * LDK;  // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int HWo = p.Ho * p.Wo;
  const long M = (long)p.batch * HWo;
  const long m0 = (long)blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;

  // A (im2col) load slots: thread owns rows tid/KCH + i*(256/KCH), chunk kc
  const int kc = tid % KCH;
  const _Float16 * arow[A_IT];
  int aiy[A_IT], aix[A_IT];
#pragma unroll
  for (int i = 0; i < A_IT; ++i) {
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

  h8 ra[A_IT], rb[B_IT];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
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
    for (int i = 0; i < B_IT; ++i) {
      const int r = tid / KCH + i * (256 / KCH);
      if (r < BN) rb[i] = *reinterpret_cast<const h8 *>(wbase + (long)(n0 + r) * p.kpad + kt * BK + kc * 8);
    }
    ci += BK;
    norm_k();
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_IT; ++i)
      *reinterpret_cast<h8 *>(As + (buf * BM + tid / KCH + i * (256 / KCH)) * LDK + kc * 8) = ra[i];
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
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

  int boff[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) boff[tm] = (wm * TM * 32 + tm * 32 + (lane & 31)) * LDK + (lane >> 5) * 8;

  const int nk = kt1 - kt0;
  if (nk > 0) {
    load_tile(kt0);
    store_tile(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile(kt0 + kt + 1);
    const _Float16 * wrow = Bs + (cur * BN + wn * TN * 32 + (lane & 31)) * LDK + (lane >> 5) * 8;
    const _Float16 * prow = As + cur * BM * LDK;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) mfma_step<TM, TN>(acc, wrow + kk * 16, prow + kk * 16, boff, LDK);
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  igemm_epilogue<WGM, WGN, TM, TN>(acc, p, lds, n0, [&](int pl, int & b, int & hw) {
    const long pm = m0 + pl;
    if (pm >= M) return false;
    b = (int)(pm / HWo);
    hw = (int)(pm - (long)b * HWo);
    return true;
  });
}

// -------------------------------------------------------------- halo kernel
// 3x3, stride 1.  Output tile TH x TW (= 128 pixels) of one image.  K steps run over
// (32-channel chunk c, tap t); weights are packed [co][c][t][32] so step s = c*9 + t reads
// the contiguous K range [32 s, 32 s + 32).  The (TH+2) x (TW+2) x 32 input patch of chunk
// c is loaded once (global -> registers during chunk c-1's taps -> LDS) and read by all
// nine taps.
template <int WGM, int WGN, int TM, int TN, int TH, int TW>
__global__ void __launch_bounds__(256) conv3x3_halo_kernel(const ConvParams p)
{
  using T = Tile<WGM, WGN, TM, TN>;
  constexpr int BM = T::BM, BN = T::BN, BK = T::BK, LDK = T::LDK, KCH = T::KCH;
  static_assert(BM == TH * TW, "tile shape");
  constexpr int CKP = 40;                 // patch channel pitch (32 + 8 halves)
  constexpr int PH = TH + 2, PW = TW + 2, PP = PH * PW;
  constexpr int P_IT = (PP * 4 + 255) / 256;
  constexpr int B_IT = (BN * KCH + 255) / 256;
  constexpr int STAGE = 2 * PP * CKP + 2 * BN * LDK;
  __shared__ __attribute__((aligned(16))) _Float16 lds[STAGE > T::OUT ? STAGE : T::OUT];
  _Float16 * Ps = lds;                    // [2][PP][CKP]
  _Float16 * Bs = lds + 2 * PP * CKP;     // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int tiles_x = (p.Wo + TW - 1) / TW, tiles_y = (p.Ho + TH - 1) / TH;
  int t = blockIdx.x;
  const int txi = t % tiles_x;
  t /= tiles_x;
  const int tyi = t % tiles_y;
  const int img = t / tiles_y;
  const int oy0 = tyi * TH, ox0 = txi * TW;
  const int iy0 = oy0 - p.P, ix0 = ox0 - p.P;
  const int n0 = blockIdx.y * BN;
  const _Float16 * xb = reinterpret_cast<const _Float16 *>(p.x.ptr) + (long)img * p.x.img;
  const _Float16 * wbase = reinterpret_cast<const _Float16 *>(p.w);
  const int nchunks = (p.Cin + 31) / 32;
  const int nsteps = nchunks * 9;

  h8 rp[P_IT], rb[B_IT];
  auto load_patch = [&](int c) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      const int e = tid + i * 256;
      h8 v = {};
      if (e < PP * 4) {
        const int px = e >> 2, q = e & 3;
        const int py = px / PW, pxx = px - py * PW;
        const int iy = iy0 + py, ix = ix0 + pxx;
        const int ci = c * 32 + q * 8;
        if ((unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W && ci < p.Cin) {
          v = *reinterpret_cast<const h8 *>(xb + ((long)iy * p.W + ix) * p.x.cs + ci);
          if (ci + 8 > p.Cin) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
              if (ci + k >= p.Cin) v[k] = (_Float16)0.0f;
          }
        }
      }
      rp[i] = v;
    }
  };
  auto store_patch = [&](int buf) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      const int e = tid + i * 256;
      if (e < PP * 4) *reinterpret_cast<h8 *>(Ps + (buf * PP + (e >> 2)) * CKP + (e & 3) * 8) = rp[i];
    }
  };
  auto load_w = [&](int s) {
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int r = (tid + i * 256) / KCH, kc = (tid + i * 256) % KCH;
      if (r < BN) rb[i] = *reinterpret_cast<const h8 *>(wbase + (long)(n0 + r) * p.kpad + s * BK + kc * 8);
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int i = 0; i < B_IT; ++i) {
      const int r = (tid + i * 256) / KCH, kc = (tid + i * 256) % KCH;
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

  // per-tm patch offset of this lane's pixel (tap (0,0)) and K half
  int boff[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int pl = wm * TM * 32 + tm * 32 + (lane & 31);
    const int ty = pl / TW, tx = pl - ty * TW;
    boff[tm] = (ty * PW + tx) * CKP + (lane >> 5) * 8;
  }

  load_patch(0);
  load_w(0);
  store_patch(0);
  store_w(0);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int c = s / 9, tap = s - c * 9;
    if (s + 1 < nsteps) load_w(s + 1);
    if (tap == 0 && c + 1 < nchunks) load_patch(c + 1);
    const int ky = tap / 3, kx = tap - ky * 3;
    const _Float16 * wrow = Bs + ((s & 1) * BN + wn * TN * 32 + (lane & 31)) * LDK + (lane >> 5) * 8;
    const _Float16 * prow = Ps + ((c & 1) * PP + ky * PW + kx) * CKP;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) mfma_step<TM, TN>(acc, wrow + kk * 16, prow + kk * 16, boff, LDK);
    if (s + 1 < nsteps) store_w((s + 1) & 1);
    if (tap == 8 && c + 1 < nchunks) store_patch((c + 1) & 1);
    __syncthreads();
  }

  igemm_epilogue<WGM, WGN, TM, TN>(acc, p, lds, n0, [&](int pl, int & b, int & hw) {
    const int ty = pl / TW, tx = pl - ty * TW;
    const int oy = oy0 + ty, ox = ox0 + tx;
    if (oy >= p.Ho || ox >= p.Wo) return false;
    b = img;
    hw = oy * p.Wo + ox;
    return true;
  });
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
  float o = (float)(_Float16)v;  // one rounding before the residual, as the fused epilogue
  if (p.r.ptr) {
    const long ri = p.r.layout == kNHWC ? (long)hw * p.r.cs + co : (long)co * p.r.cs + hw;
    o += (float)reinterpret_cast<const _Float16 *>(p.r.ptr)[(long)b * p.r.img + ri];
  }
  const long yi = p.y.layout == kNHWC ? (long)hw * p.y.cs + co : (long)co * p.y.cs + hw;
  reinterpret_cast<_Float16 *>(p.y.ptr)[(long)b * p.y.img + yi] = (_Float16)o;
}

// ---------------------------------------------------------------- host side

// Tile table: a small CDNA4 choice per op (BN from Cout; BM = 128 pixels).
int igemm_bn(int cout) { return cout <= 32 ? 32 : (cout <= 64 ? 64 : 128); }

template <int WGM, int WGN, int TM, int TN>
static void launch_t(const ConvParams & p, hipStream_t s)
{
  using T = Tile<WGM, WGN, TM, TN>;
  const long M = (long)p.batch * p.Ho * p.Wo;
  dim3 grid((unsigned)((M + T::BM - 1) / T::BM), (unsigned)((p.Cout + T::BN - 1) / T::BN), (unsigned)p.ksplit);
  hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN>), grid, dim3(256), 0, s, p);
  if (p.ksplit > 1) {
    const long n = M * p.Cout;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p,
                       (int)grid.y * T::BN);
  }
}

template <int WGM, int WGN, int TM, int TN, int TH, int TW>
static void launch_h(const ConvParams & p, hipStream_t s)
{
  using T = Tile<WGM, WGN, TM, TN>;
  const unsigned tiles = (unsigned)(((p.Wo + TW - 1) / TW) * ((p.Ho + TH - 1) / TH) * p.batch);
  dim3 grid(tiles, (unsigned)((p.Cout + T::BN - 1) / T::BN), 1);
  hipLaunchKernelGGL((conv3x3_halo_kernel<WGM, WGN, TM, TN, TH, TW>), grid, dim3(256), 0, s, p);
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

int halo_tw(int Ho, int Wo)
{
  // output tile (8 x 16) or (16 x 8): the one wasting fewer pixel slots
  const long w16 = (long)((Wo + 15) / 16) * 16 * ((Ho + 7) / 8) * 8;
  const long w8 = (long)((Wo + 7) / 8) * 8 * ((Ho + 15) / 16) * 16;
  return w8 < w16 ? 8 : 16;
}

void launch_conv_igemm(const ConvParams & p, hipStream_t s)
{
  if (p.halo) {
    const bool t8 = p.halo == 8;
    switch (igemm_bn(p.Cout)) {
    case 32: t8 ? launch_h<4, 1, 1, 1, 16, 8>(p, s) : launch_h<4, 1, 1, 1, 8, 16>(p, s); break;
    case 64: t8 ? launch_h<2, 2, 2, 1, 16, 8>(p, s) : launch_h<2, 2, 2, 1, 8, 16>(p, s); break;
    default: t8 ? launch_h<2, 2, 2, 2, 16, 8>(p, s) : launch_h<2, 2, 2, 2, 8, 16>(p, s); break;
    }
    return;
  }
  switch (igemm_bn(p.Cout)) {
  case 32: launch_t<4, 1, 1, 1>(p, s); break;
  case 64: launch_t<2, 2, 2, 1>(p, s); break;
  default: launch_t<2, 2, 2, 2>(p, s); break;
  }
}

}  // namespace ivh
