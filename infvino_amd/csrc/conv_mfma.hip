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
// 32x32 MFMA blocks.  Linear pixel tiles over all images; the im2col tile is gathered from
// global memory (any K, stride, pad; every input pixel is re-read per tap from L2), BK = 32
// double buffered through LDS.  The 3x3 stride-1 convs with a well-filled grid use the
// LDS-patch kernel of conv_halo.hip instead.  With split-K the fp32 partials go to a
// workspace and splitk_reduce_kernel finishes.
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

typedef Mf<32>::acc_t f16v;

template <int WGM, int WGN, int TM, int TN>
struct Tile {
  static constexpr int BM = WGM * TM * 32;
  static constexpr int BN = WGN * TN * 32;
  static constexpr int BK = 32;
  static constexpr int LDK = BK + 8;  // padded LDS row: 16-byte reads conflict free
  static constexpr int KCH = BK / 8;
  static constexpr int OUT = TileShape<32, WGM, WGN, TM, TN>::EPI;
};

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

  tile_epilogue<32, WGM, WGN, TM, TN>(acc, p, lds, n0, [&](int pl, int & b, int & hw) {
    const long pm = m0 + pl;
    if (pm >= M) return false;
    b = (int)(pm / HWo);
    hw = (int)(pm - (long)b * HWo);
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
  if (p.halo) {
    launch_conv_halo(p, s);
    return;
  }
  switch (igemm_bn(p.Cout)) {
  case 32: launch_t<4, 1, 1, 1>(p, s); break;
  case 64: launch_t<2, 2, 2, 1>(p, s); break;
  default: launch_t<2, 2, 2, 2>(p, s); break;
  }
}

}  // namespace ivh
