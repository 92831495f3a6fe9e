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
// global memory (any K, stride, pad; every input pixel is re-read per tap from L2), K steps
// of 32 or 64 double buffered through LDS.  The 3x3 stride-1 convs with a well-filled grid use the
// LDS-patch kernel of conv_halo.hip instead.  With split-K the fp32 partials go to a
// workspace and splitk_reduce_kernel finishes.
#include "conv_common.hpp"
#include "kernels.hpp"

#include <cstdio>
#include <string>

namespace ivh {

// ------------------------------------------------------------ im2col kernel
// Tile: BM = WGM*TM*32 output pixels (linear over all images) x BN = WGN*TN*32 channels,
// K steps of BK (32 or 64, chosen with the packing).  A (pixel) loads: a thread owns fixed
// tile rows and one 8-channel piece of every K step; the tap / channel of its piece moves
// incrementally, out-of-image taps and K padding load from past the buffer's range (zeros),
// and the ragged channels of a last piece (Cin % 8) are zeroed when written to LDS.  B
// (weight) loads are buffer loads at a loop-invariant offset plus the step's scalar offset.
// Both are double buffered in LDS and prefetched PF steps ahead through a ring of PF
// register stages, so a work-group with a short K loop has its whole K range in flight at
// once instead of waiting one memory latency per step.  RAG: Cin is not a multiple of 8
// (the compile-time switch keeps the masking out of the common case).  XT: a 1x1 conv on
// NCHW channel planes (p.xt): a thread's A piece is 8 consecutive pixels of one channel (one
// 16-byte load along the plane), written transposed into the pixel rows of the LDS tile, so
// the MFMA loop and the epilogue are those of the channels-last case.  UP: a 1x1 conv over a
// channel concat whose first p.cu channels are a 2x nearest upsample of p.xu (p.cu a multiple
// of BK): the K steps below p.cu read pixel (oy / 2, ox / 2) of xu instead of x, so the
// upsampled tensor is never written (the same values reach the same LDS rows as when the
// concat is materialised, hence the same results bit for bit).
template <int WGM, int WGN, int TM, int TN, int BK, int PF, bool RAG, int OCC = 1, bool XT = false, bool UP = false>
__global__ void __launch_bounds__(256, OCC) conv_igemm_kernel(const ConvParams p)
{
  using F = Mf<32>;
  using T = TileShape<32, WGM, WGN, TM, TN>;
  typedef F::acc_t acc_t;
  constexpr int BM = T::BM, BN = T::BN;
  constexpr int LDK = BK + 8;                 // padded LDS row: 16-byte reads conflict free
  constexpr int KC = BK / 8;                  // 16-byte pieces per row and step
  constexpr int RPI = 256 / KC;               // rows covered by one pass of the 256 threads
  constexpr int A_IT = BM / RPI, B_IT = (BN + RPI - 1) / RPI;
  constexpr int STAGE = BM * LDK + BN * LDK;
  constexpr int L_ALL = 2 * STAGE > T::EPI ? 2 * STAGE : T::EPI;
  static_assert(BM % RPI == 0, "tile rows");
  constexpr int PG = BM / 8;                  // XT: 8-pixel pieces per tile row of a channel
  constexpr int X_IT = BK * PG / 256;         // XT: A pieces per thread and step
  static_assert(!XT || X_IT * 256 == BK * PG, "planar tile pieces");
  constexpr int A_N = XT ? X_IT : A_IT;       // A register pieces per stage
  __shared__ __attribute__((aligned(16))) _Float16 lds[L_ALL];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int HWo = p.Ho * p.Wo;
  const unsigned M = (unsigned)p.batch * HWo;  // below 2^31 (the launcher's batch chunks)
  // XCD-aware order over (channel tile, pixel tile, K slice), channel tiles fastest: the
  // channel tiles of one pixel tile, which gather the same input, run together on one XCD and
  // share its L2, and neighbouring pixel tiles (sharing input rows) follow on the same XCD
  const int lin = xcd_tile(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z),
                           gridDim.x * gridDim.y * gridDim.z);
  const int by = lin % gridDim.y, bx = (lin / gridDim.y) % gridDim.x, bz = lin / (gridDim.x * gridDim.y);
  const unsigned m0 = (unsigned)bx * BM;
  const int n0 = by * BN;
  const int kc = tid % KC, r0 = tid / KC;

  // end of the input view: the last pixel's channel pieces (channels-last), or the end of the
  // last channel plane (XT)
  const long x_last = (long)(p.batch - 1) * p.x.img +
                      (XT ? (long)(p.Cin - 1) * p.x.cs + (long)p.H * p.W : ((long)p.H * p.W - 1) * p.x.cs + p.cin8);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w + (long)n0 * p.kpad), (short)0, BN * p.kpad * 2, kBufDword3);

  // A rows of this thread: image base offset and the input corner of the output pixel; UP:
  // the element offset of the row's source pixel in xu (-1 past the batch)
  int abase[A_IT], aiy[A_IT], aix[A_IT], uoff[UP ? A_IT : 1];
#pragma unroll
  for (int i = 0; i < A_IT; ++i) {
    const unsigned pm = m0 + r0 + i * RPI;
    if (pm < M) {
      const int b = (int)fastdiv(pm, p.dv_hwo), hw = (int)pm - b * HWo;
      const int oy = (int)fastdiv((unsigned)hw, p.dv_wo), ox = hw - oy * p.Wo;
      abase[i] = b * (int)p.x.img;
      aiy[i] = oy * p.S - p.P;
      aix[i] = ox * p.S - p.P;
      if constexpr (UP) uoff[i] = b * (int)p.xu.img + ((oy >> 1) * (p.W >> 1) + (ox >> 1)) * p.xu.cs;
    } else {
      abase[i] = 0;
      aiy[i] = -0x4000000;  // never inside the image
      aix[i] = 0;
      if constexpr (UP) uoff[i] = -1;
    }
  }
  // UP: the upsample source's range, its last pixel's first p.cu channels
  const long u_last = UP ? (long)(p.batch - 1) * p.xu.img + ((long)(p.H >> 1) * (p.W >> 1) - 1) * p.xu.cs + p.cu : 0;
  const __amdgpu_buffer_rsrc_t ur = __builtin_amdgcn_make_buffer_rsrc(
      UP ? const_cast<__half *>(p.xu.ptr) : const_cast<__half *>(p.x.ptr), (short)0, (int)(u_last * 2), kBufDword3);
  // XT: piece i of this thread is channel xc[i] of the step, pixels m0 + 8 xg[i] .. + 7
  // (one image: its plane holds a multiple of 8 pixels); byte offset of the piece in step
  // 0, or past the buffer range for pixels past the batch
  int xc[XT ? X_IT : 1], xg[XT ? X_IT : 1];
  unsigned xoff[XT ? X_IT : 1];
  if constexpr (XT) {
#pragma unroll
    for (int i = 0; i < X_IT; ++i) {
      const int e = tid + i * 256;
      xc[i] = e / PG;
      xg[i] = e - xc[i] * PG;
      const unsigned pm = m0 + 8 * xg[i];
      xoff[i] = kBufOOB;
      if (pm < M) {
        const int b = (int)fastdiv(pm, p.dv_hwo), hw = (int)pm - b * HWo;
        xoff[i] = (unsigned)((b * (int)p.x.img + xc[i] * p.x.cs + hw) * 2);
      }
    }
  }
  unsigned bsrc[B_IT];
#pragma unroll
  for (int i = 0; i < B_IT; ++i) {
    const int r = r0 + i * RPI < BN ? r0 + i * RPI : 0;
    bsrc[i] = (unsigned)((r * p.kpad + kc * 8) * 2);
  }

  // K range of this work-group (split-K: blockIdx.z-th slice of the K steps)
  const int nk_all = p.kpad / BK;
  const int per = (nk_all + p.ksplit - 1) / p.ksplit;
  const int kt0 = bz * per;
  const int kt1 = kt0 + per < nk_all ? kt0 + per : nk_all;
  const int nk = kt1 > kt0 ? kt1 - kt0 : 0;
  const int taps = p.K * p.K;
  // position (tap, ci) of this thread's piece in the current load step; a step advances it
  // by dq taps and dr channels.  ky = tap / K as (tap * kmul) >> 16, exact for tap < 2^16 / K
  // (the launcher keeps K * K + 16 below that).
  const int dq = BK / p.cin8, dr = BK - dq * p.cin8;
  const unsigned kmul = (65536u + p.K - 1) / p.K;
  int tap = (kt0 * BK + kc * 8) / p.cin8;
  int ci = kt0 * BK + kc * 8 - tap * p.cin8;
  auto advance = [&]() {
    ci += dr;
    tap += dq;
    if (ci >= p.cin8) {
      ci -= p.cin8;
      ++tap;
    }
  };

  // register ring: stage d holds the pieces of step d (mod PF) between load and LDS store
  h8 ra[PF][A_N], rb[PF][B_IT];
  int aci[PF];  // channel of the loaded A piece (for the ragged mask at store time)
  auto load = [&](int kt, int d) {
    if constexpr (XT) {
      // channels past Cin read zeros (their packed weights are zero too)
#pragma unroll
      for (int i = 0; i < X_IT; ++i) {
        const bool ok = kt * BK + xc[i] < p.Cin && xoff[i] != kBufOOB;
        const unsigned off = ok ? xoff[i] + (unsigned)(kt * BK * p.x.cs * 2) : kBufOOB;
        ra[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < B_IT; ++i)
        rb[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wr, bsrc[i], kt * BK * 2, 0));
      return;
    }
    aci[d] = ci;
    if constexpr (UP) {
      // a K step below p.cu lies wholly in the upsampled channels (p.cu % BK == 0)
      if (kt * BK < p.cu) {
#pragma unroll
        for (int i = 0; i < A_IT; ++i) {
          const unsigned off = uoff[i] >= 0 ? (unsigned)((uoff[i] + ci) * 2) : kBufOOB;
          ra[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < B_IT; ++i)
          rb[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wr, bsrc[i], kt * BK * 2, 0));
        advance();
        return;
      }
    }
    const int ky = (int)(((unsigned)tap * kmul) >> 16), kx = tap - ky * p.K;
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      const int iy = aiy[i] + ky, ix = aix[i] + kx;
      const bool ok = tap < taps && (unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W;
      const unsigned off = ok ? (unsigned)((abase[i] + (iy * p.W + ix) * p.x.cs + ci) * 2) : kBufOOB;
      ra[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i)
      rb[d][i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wr, bsrc[i], kt * BK * 2, 0));
    advance();
  };
  auto store = [&](_Float16 * st, int d) {
    if constexpr (XT) {
#pragma unroll
      for (int i = 0; i < X_IT; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) st[(8 * xg[i] + j) * LDK + xc[i]] = ra[d][i][j];
#pragma unroll
      for (int i = 0; i < B_IT; ++i)
        if (r0 + i * RPI < BN) *reinterpret_cast<h8 *>(st + (BM + r0 + i * RPI) * LDK + kc * 8) = rb[d][i];
      return;
    }
    u16x8 keep;
    if (RAG) {
#pragma unroll
      for (int e = 0; e < 8; ++e) keep[e] = aci[d] + e < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
    }
#pragma unroll
    for (int i = 0; i < A_IT; ++i) {
      h8 v = ra[d][i];
      if (RAG) v = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, v) & keep);
      *reinterpret_cast<h8 *>(st + (r0 + i * RPI) * LDK + kc * 8) = v;
    }
#pragma unroll
    for (int i = 0; i < B_IT; ++i)
      if (r0 + i * RPI < BN) *reinterpret_cast<h8 *>(st + (BM + r0 + i * RPI) * LDK + kc * 8) = rb[d][i];
  };

  acc_t acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) acc[a][b][v] = 0.0f;

  const int brow = (wm * TM * 32 + (lane & 31)) * LDK + F::kq(lane);
  const int arow = (BM + wn * TN * 32 + (lane & 31)) * LDK + F::kq(lane);
  // step s (register stage d = s mod PF): step s + PF's loads go into stage d, whose
  // pieces reached LDS at the end of step s - 1; the MFMAs read LDS buffer s & 1; step
  // s + 1's pieces then go to the other buffer.
  auto step = [&](int s, int d, const _Float16 * cur, _Float16 * nxt) {
    if (s + PF < nk) load(kt0 + s + PF, d);
#pragma unroll
    for (int j = 0; j < BK / 16; ++j) {
      h8 fa[TN], fb[TM];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) fa[tn] = *reinterpret_cast<const h8 *>(cur + arow + tn * 32 * LDK + j * 16);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) fb[tm] = *reinterpret_cast<const h8 *>(cur + brow + tm * 32 * LDK + j * 16);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = F::mma(fa[tn], fb[tm], acc[tn][tm]);
    }
    if (s + 1 < nk) store(nxt, (d + 1) % PF);
    __syncthreads();
  };
  _Float16 * const S0 = lds;
  _Float16 * const S1 = lds + STAGE;
#pragma unroll
  for (int d = 0; d < PF; ++d)
    if (d < nk) load(kt0 + d, d);
  if (nk > 0) store(S0, 0);
  __syncthreads();
  // unrolled so that both the register stage and the LDS buffer of a step are static
  constexpr int U = PF % 2 == 0 ? PF : 2 * PF;
  for (int s = 0; s < nk; s += U) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (s + u < nk) step(s + u, u % PF, (u & 1) ? S1 : S0, (u & 1) ? S0 : S1);
  }

  tile_epilogue<32, WGM, WGN, TM, TN>(acc, p, lds, n0, bz, [&](int pl, int & b, int & hw) {
    const unsigned pm = m0 + pl;
    if (pm >= M) return false;
    b = (int)fastdiv(pm, p.dv_hwo);
    hw = (int)pm - b * HWo;
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

// What the UP build assumes: a 1x1 stride-1 conv on even maps, channels-last x and xu with
// 16-byte channel pieces, the upsampled channels a whole number of K steps, no ragged tail
bool upcat_ok(const ConvParams & p)
{
  return p.cu > 0 && p.K == 1 && p.S == 1 && p.P == 0 && p.G == 1 && p.H % 2 == 0 && p.W % 2 == 0 &&
         p.Ho == p.H && p.Wo == p.W && p.cu < p.Cin && p.cu % p.bk == 0 && p.Cin % 8 == 0 && p.cin8 == p.Cin &&
         !p.xt && !p.pw && !p.halo && !p.res && !p.pipe && !p.wide && !p.s2 && p.x.layout == kNHWC &&
         p.xu.layout == kNHWC && p.xu.cs % 8 == 0 && p.xu.img % 8 == 0 && p.xu.cs >= p.cu &&
         (reinterpret_cast<uintptr_t>(p.xu.ptr) & 15) == 0;
}

template <int WGM, int WGN, int TM, int TN, int BK, int PF, int OCC = 1>
static void launch_t(const ConvParams & p, hipStream_t s)
{
  using T = TileShape<32, WGM, WGN, TM, TN>;
  const long M = (long)p.batch * p.Ho * p.Wo;
  if (M >= (1L << 31) || p.K * p.K + 16 >= 65536 / p.K) throw std::runtime_error("implicit-GEMM conv geometry");
  if (p.cu && !upcat_ok(p)) throw std::runtime_error("implicit-GEMM upsample-concat geometry");
  ConvParams q = p;
  q.dv_hwo = fastdiv_make((unsigned)(p.Ho * p.Wo));
  q.dv_wo = fastdiv_make((unsigned)p.Wo);
  dim3 grid((unsigned)((M + T::BM - 1) / T::BM), (unsigned)((p.Cout + T::BN - 1) / T::BN), (unsigned)p.ksplit);
  if (p.xt) hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN, BK, PF, false, 1, true>), grid, dim3(256), 0, s, q);
  else if (p.cu) hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN, BK, PF, false, OCC, false, true>), grid, dim3(256), 0, s, q);
  else if (p.Cin & 7) hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN, BK, PF, true>), grid, dim3(256), 0, s, q);
  else hipLaunchKernelGGL((conv_igemm_kernel<WGM, WGN, TM, TN, BK, PF, false, OCC>), grid, dim3(256), 0, s, q);
  if (p.ksplit > 1) {
    const long n = M * p.Cout;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p,
                       (int)grid.y * T::BN);
  }
}

// Output tiles of a layer (BM = 128 pixels x BN channels) over the batch
static long igemm_tiles(const ConvParams & p)
{
  const int bn = igemm_bn(p.Cout);
  return ((long)p.batch * p.Ho * p.Wo + 127) / 128 * ((p.Cout + bn - 1) / bn);
}

// The 128-VGPR build (four resident work-groups per CU) of the 128-wide tile: 1x1 convs with
// K step 32 whose 769..1024 tiles overflow three work-groups per CU
static bool igemm_occ4(const ConvParams & p)
{
  return p.K == 1 && p.bk == 32 && igemm_bn(p.Cout) == 128 && !(p.Cin & 7) && !p.xt && p.ksplit == 1 &&
         igemm_tiles(p) > 3 * 256 && igemm_tiles(p) <= 4 * 256;
}

// Register prefetch depth (K steps in flight) per tile width (measured on MI355X over
// depths 1..6: deeper rings cost occupancy on the wide tiles and gain little elsewhere).
constexpr int PF32 = 2, PF64 = 2, PF128 = 2;
template <int BK>
static void launch_bk(const ConvParams & p, hipStream_t s)
{
  switch (igemm_bn(p.Cout)) {
  case 32: launch_t<4, 1, 1, 1, BK, PF32>(p, s); break;
  case 64: launch_t<2, 2, 2, 1, BK, PF64>(p, s); break;
  default:
    // 1x1 convs whose tiles overflow three resident work-groups per CU (at 144 VGPRs) but
    // fit four: the 128-VGPR build of the same tile (40x40 maps at batch 64, 800 tiles:
    // 22-34 -> 20-30 us).  3x3 convs lose more to the register cap than they gain (measured).
    if constexpr (BK == 32) {
      if (igemm_occ4(p)) {
        launch_t<2, 2, 2, 2, BK, PF128, 4>(p, s);
        break;
      }
    }
    launch_t<2, 2, 2, 2, BK, PF128>(p, s);
    break;
  }
}

// K step of a layer (measured on MI355X): 64 for wide layers with a long K, where the MFMA
// work per barrier matters; 32 otherwise, where the smaller LDS stages keep more
// work-groups resident for the memory-bound layers.  The packed K is a multiple of it.
int igemm_bk(int cout, int kk)
{
  if (cout <= 64 || kk < 512) return 32;
  const int k64 = (kk + 63) / 64 * 64;
  return (k64 - kk) * 8 <= kk ? 64 : 32;
}

int igemm_kpad(int cout, int kk)
{
  const int bk = igemm_bk(cout, kk);
  return (kk + bk - 1) / bk * bk;
}

// Split-K factor: convs whose output tiles cannot fill the chip (batch 1, 20x20 / 40x40
// feature maps) and whose K loop is long get their K range split across work-groups, by 3
// or more: a split by 2 did not pay for its reduce launch (MI355X, YOLOv8n-pose batch 1:
// 32->64 s2 at 160x160 12.0 vs 8.7 us, 256->128 1x1 at 40x40 11.1 vs 9.8 us).
int igemm_ksplit(long M, int cout, int kpad)
{
  const int bn = igemm_bn(cout);
  const long tiles = ((M + 127) / 128) * ((cout + bn - 1) / bn);
  const int nk = kpad / kIgemmBK;
  if (tiles >= 192 || nk < 8) return 1;
  int s = (int)((384 + tiles - 1) / tiles);
  s = s < nk / 4 ? s : nk / 4;
  s = s < 16 ? s : 16;
  return s < 3 ? 1 : s;
}

// Batch chunk that keeps a conv's input view below 2^31 bytes (the kernels' buffer ranges
// and 32-bit element offsets); every image of a chunk is independent of the others.
int conv_batch_chunk(const ConvParams & p)
{
  const long per = std::max<long>(std::max(p.x.img, p.cu ? p.xu.img : 0L) * 2, 1);
  return (int)std::max<long>(1, std::min<long>(p.batch, ((1L << 31) - 1) / per - 1));
}

ConvParams conv_batch_slice(const ConvParams & p, int b0, int nb)
{
  ConvParams q = p;
  q.batch = nb;
  q.x.ptr += (long)b0 * p.x.img;
  q.y.ptr += (long)b0 * p.y.img;
  if (q.r.ptr) q.r.ptr += (long)b0 * p.r.img;
  if (q.cu) q.xu.ptr += (long)b0 * p.xu.img;
  return q;
}

std::string igemm_launch_tag(const ConvParams & p)
{
  char b[160];
  if (p.pw == 2)
    snprintf(b, sizeof b, "blocks=%ld lds=%zu planar-out%s", pw_blocks(p), pwt_lds_bytes(p), p.xt ? " planar-in" : "");
  else if (p.pw)
    snprintf(b, sizeof b, "blocks=%ld lds=%zu", pw_blocks(p), pw_lds_bytes(p));
  else if (p.wide)
    snprintf(b, sizeof b, "tm=%d ranges=%d wgs=%ld", p.th, p.tw, wide_grid(p));
  else if (p.pipe)
    snprintf(b, sizeof b, "cfg=%d th=%d tw=%d items=%ld", p.pipe - 1, p.th, p.tw, pipe_items(p));
  else if (p.res)
    snprintf(b, sizeof b, "cfg=%d th=%d tw=%d ck=%d store=%d", p.res - 1, p.th, p.tw, p.ck, res_store_width(p));
  else if (p.halo)
    snprintf(b, sizeof b, "cfg=%d th=%d tw=%d ck=%d", p.halo - 1, p.th, p.tw, p.ck);
  else if (p.s2 > 2)
    snprintf(b, sizeof b, "cfg=%d th=%d tw=%d tiles=%ld", p.s2 - 1, p.th, p.tw, s2pk_tiles(p));
  else if (p.s2)
    snprintf(b, sizeof b, "cfg=%d th=%d tw=%d", p.s2 - 1, p.th, p.tw);
  else
    snprintf(b, sizeof b, "bn=%d bk=%d ksplit=%d%s%s%s%s", igemm_bn(p.Cout), p.bk, p.ksplit,
             igemm_occ4(p) ? " vgpr128" : "", p.xt ? " planar" : "", (p.Cin & 7) ? " cin-ragged" : "",
             p.cu ? " upsample-concat" : "");
  return b;
}

void launch_conv_igemm(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_igemm(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  if (p.pw) {
    launch_conv_pw(p, s);
    return;
  }
  if (p.wide) {
    launch_conv_wide(p, s);
    return;
  }
  if (p.pipe) {
    launch_conv_pipe(p, s);
    return;
  }
  if (p.res) {
    launch_conv_res(p, s);
    return;
  }
  if (p.halo) {
    launch_conv_halo(p, s);
    return;
  }
  if (p.s2) {
    launch_conv_s2(p, s);
    return;
  }
  if (p.bk == 64) launch_bk<64>(p, s);
  else launch_bk<32>(p, s);
}

}  // namespace ivh
