// 3x3 stride-1 pad-1 convolution on gfx950 fp16 MFMA with an LDS input patch.
//
// Replaces the reference's 3x3 stride-1 kernels conv3x3_ov (kernels/conv_ov.cl:133-297),
// conv3x3_blk (conv_blk.cl:118-296) and conv3x3_f16 (conv.cl:150-414) on channels-last
// input: y[co][p] = act(sum_{tap,ci} W[co][ci][tap] x[ci][p + tap] + b[co]) (+ r[co][p]).
//
// Geometry.  The batch is one tall image: image b occupies rows [b*(H+1), b*(H+1)+H) and a
// zero separator row follows each image, so a 3x3 window never mixes two images and the
// pad-1 border is the separator (or the top/bottom edge).  Output tiles are TH x TW pixels
// of that tall image (runtime shape, chosen per layer on the host to waste few slots); the
// slots that land on separator rows or past the right edge are computed and discarded.
//
// K loop.  Input channels are taken in chunks of CK (16 / 32 / 64).  For each chunk the
// (TH+2) x (TW+2) x CK input patch is loaded once from HBM into LDS and every tap reads its
// MFMA pixel fragments from it at a shifted offset.  One K step is BK = max(CK, 32) deep;
// with CK = 16 a step spans two taps and a 10th tap of zero weights reads an all-zero patch
// row.  Weights are packed [co][chunk][tap][CK] so a step's weights are one contiguous K
// range; they are double buffered in LDS and prefetched one step ahead in registers.  The
// next chunk's patch is loaded into registers after a chunk's first step and written to LDS
// after its last tap.  All global loads are buffer loads with loop-invariant per-thread
// offsets (the step / chunk offset is scalar); out-of-image patch pixels use an offset past
// the buffer's range, which the hardware answers with zeros.
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

template <int MB, int WGM, int WGN, int TM, int TN, int CK, int PMAX>
__global__ void __launch_bounds__(256) conv3x3s1_kernel(const ConvParams p)
{
  using F = Mf<MB>;
  using T = TileShape<MB, WGM, WGN, TM, TN>;
  typedef typename F::acc_t acc_t;
  constexpr int BN = T::BN;
  constexpr int BK = CK >= 32 ? CK : 32;            // K depth of one step
  constexpr int TAPS = (9 * CK) % BK == 0 ? 9 : 10;  // taps per chunk in the packing
  constexpr int SPC = TAPS * CK / BK;               // steps per chunk
  constexpr int CKP = CK + 8;                       // patch pixel pitch (halves)
  constexpr int LDK = BK + 8;                       // weight row pitch (halves)
  constexpr int NSUB = BK / F::KD;                  // MFMA K slices per step
  constexpr int CQ = CK / 8;                        // 16-byte pieces per patch pixel
  constexpr int P_IT = (PMAX * CQ + 255) / 256;
  constexpr int WCH = BK / 8;
  constexpr int W_IT = (BN * WCH + 255) / 256;
  constexpr bool W_FULL = W_IT * 256 == BN * WCH;
  // patch rows padded so each starts where a linear layout of the same pixels would, modulo
  // 256 bytes: MFMA pixel fragments that wrap a tile row stay LDS bank-conflict free.  Not
  // with 16-channel chunks: those layers are latency bound and the pad's LDS reserve would
  // cost them two of eight resident work-groups per CU (measured slower)
  constexpr int PADH = CK == 16 ? 0 : ((256 - (4 * CKP) % 256) % 256) / 2;
  constexpr int ZOFF = PMAX * CKP + kHaloMaxRows * PADH;  // all-zero patch pixel
  constexpr int L_PATCH = ZOFF + CKP;
  constexpr int L_MAIN = L_PATCH + 2 * BN * LDK;
  constexpr int L_ALL = L_MAIN > T::EPI ? L_MAIN : T::EPI;
  __shared__ __attribute__((aligned(16))) _Float16 lds[L_ALL];
  _Float16 * Ps = lds;
  _Float16 * Ws = lds + L_PATCH;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int TH = p.th, TW = p.tw, PW = TW + 2, PP = (TH + 2) * PW, RPH = PW * CKP + PADH;
  const int Hs = p.H + 1;                                  // rows per image incl. separator
  const int Htot = p.batch * Hs - 1;                       // tall-image rows
  const int tiles_x = (p.Wo + TW - 1) / TW;
  // XCD-aware order over (spatial tile, channel tile), spatial tiles fastest
  const int lin = xcd_tile(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
  const int bx = lin % gridDim.x, by = lin / gridDim.x;
  const int tyi = bx / tiles_x, txi = bx - tyi * tiles_x;
  const int oy0 = tyi * TH, ox0 = txi * TW;
  const int n0 = by * BN;
  const int nchunks = (p.Cin + CK - 1) / CK;
  const int nsteps = nchunks * SPC;
  const float inv_pw = __builtin_amdgcn_rcpf((float)PW), inv_tw = __builtin_amdgcn_rcpf((float)TW);
  const float inv_hs = __builtin_amdgcn_rcpf((float)Hs);

  // Buffer resources: the input view up to its last element (the host keeps it below 2^31
  // bytes), and this work-group's BN rows of packed weights.  A load at an offset past the
  // range returns zeros: that is how out-of-image patch pixels are filled.
  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w + (long)n0 * p.kpad), (short)0, BN * p.kpad * 2, kBufDword3);

  // patch slots: element e = tid + 256 i -> patch pixel e / CQ, piece e % CQ (= tid % CQ,
  // since 256 is a multiple of CQ).  Byte offset of the piece in chunk 0, or out of range.
  const int q8 = (tid % CQ) * 8;
  unsigned psrc[P_IT];
  int pdst[P_IT];  // LDS offset of the piece, -1 past the patch
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int pp = (tid + i * 256) / CQ;
    psrc[i] = kBufOOB;
    pdst[i] = -1;
    if (pp < PP) {
      const int py = idiv_small(pp, PW, inv_pw), px = pp - py * PW;
      pdst[i] = py * RPH + px * CKP + q8;
      const int gy = oy0 - 1 + py, ix = ox0 - 1 + px;
      if (gy >= 0 && gy < Htot && (unsigned)ix < (unsigned)p.W) {
        const int b = idiv_small(gy, Hs, inv_hs), r = gy - b * Hs;
        if (r < p.H) psrc[i] = (unsigned)((b * (int)p.x.img + (r * p.W + ix) * p.x.cs + q8) * 2);
      }
    }
  }
  unsigned wsrc[W_IT];
  int wdst[W_IT];
#pragma unroll
  for (int i = 0; i < W_IT; ++i) {
    const int e = tid + i * 256;
    const int r = (W_FULL || e / WCH < BN) ? e / WCH : 0;
    wsrc[i] = (unsigned)((r * p.kpad + (e % WCH) * 8) * 2);
    wdst[i] = r * LDK + (e % WCH) * 8;
  }
  const bool ragged = (p.Cin % CK) != 0;

  h8 rp[P_IT], rw[W_IT];
  auto load_patch = [&](int c) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i)
      rp[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, psrc[i] + c * CK * 2, 0, 0));
  };
  // pieces of a ragged last chunk: channels >= Cin are zeroed bitwise (whatever bits the
  // pixel's padding channels or the next pixel hold never reach the MFMAs)
  auto store_patch = [&](int c) {
    u16x8 keep;
#pragma unroll
    for (int k = 0; k < 8; ++k) keep[k] = c * CK + q8 + k < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      if (pdst[i] >= 0) {
        h8 v = rp[i];
        if (ragged) v = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, v) & keep);
        *reinterpret_cast<h8 *>(Ps + pdst[i]) = v;
      }
    }
  };
  auto load_w = [&](int s) {
#pragma unroll
    for (int i = 0; i < W_IT; ++i)
      rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wr, wsrc[i], s * BK * 2, 0));
  };
  auto store_w = [&](_Float16 * wbuf) {
#pragma unroll
    for (int i = 0; i < W_IT; ++i)
      if (W_FULL || (tid + i * 256) / WCH < BN) *reinterpret_cast<h8 *>(wbuf + wdst[i]) = rw[i];
  };

  // B-fragment address of a pixel block = lane base (slot's patch pixel + the lane's K
  // offset within a 16/32-deep slice) + a tap offset that is uniform across the wave
  // (scalar) + the slice's channel offset (immediate).  With CK = 16 the two taps of a
  // step differ per slice (MB = 32) or per lane half (MB = 16).
  int bl[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    int pl = wm * TM * MB + tm * MB + F::col(lane);
    if (pl >= TH * TW) pl = 0;
    const int ty = idiv_small(pl, TW, inv_tw), tx = pl - ty * TW;
    bl[tm] = ty * RPH + tx * CKP + (F::kq(lane) % CK);
  }
  const int lane_tap = (CK == 16 && MB == 16) ? (F::kq(lane) >= 16 ? 1 : 0) : 0;
  const int zbase = ZOFF + (F::kq(lane) % CK);
  auto tapoff = [&](int tap) { return (tap / 3) * RPH + (tap % 3) * CKP; };
  const int arow = (wn * TN * MB + (lane % MB)) * LDK + F::kq(lane);

  acc_t acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) acc[a][b][v] = 0.0f;

  if (TAPS == 10 && tid < CQ) *reinterpret_cast<h8 *>(Ps + ZOFF + tid * 8) = h8{};
  load_patch(0);
  load_w(0);
  store_patch(0);
  store_w(Ws);
  __syncthreads();

  // step s: MFMAs on weight buffer s&1 while step s+1's weights load into registers; they
  // go to the other buffer after the MFMAs.  The next chunk's patch loads are issued after
  // the chunk's first step (so waiting for weights never waits on them) and go to LDS after
  // its last tap.
  int c = 0, u = 0;
  auto step = [&](int s, _Float16 * wcur, _Float16 * wnext) {
    if (s + 1 < nsteps) load_w(s + 1);
    int boff[NSUB][TM];
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
      const int tap = CK >= 32 ? u : (MB == 32 ? 2 * u + j : 2 * u + lane_tap);
      const bool z = TAPS == 10 && tap >= 9;
      const int to = tapoff(z ? 0 : tap) + (CK >= 32 ? j * F::KD : 0);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) boff[j][tm] = z ? zbase : bl[tm] + to;
    }
    const _Float16 * wb = wcur + arow;
#pragma unroll
    for (int j = 0; j < NSUB; ++j) {
      h8 fa[TN], fb[TM];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) fa[tn] = *reinterpret_cast<const h8 *>(wb + tn * MB * LDK + j * F::KD);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) fb[tm] = *reinterpret_cast<const h8 *>(Ps + boff[j][tm]);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = F::mma(fa[tn], fb[tm], acc[tn][tm]);
    }
    if (s + 1 < nsteps) store_w(wnext);
    if (u == 0 && c + 1 < nchunks) load_patch(c + 1);
    __syncthreads();
    if (++u == SPC) {
      u = 0;
      ++c;
      if (c < nchunks) {
        store_patch(c);
        __syncthreads();
      }
    }
  };
  _Float16 * const W0 = Ws;
  _Float16 * const W1 = Ws + BN * LDK;
  for (int s = 0; s < nsteps; s += 2) {
    step(s, W0, W1);
    if (s + 1 < nsteps) step(s + 1, W1, W0);
  }

  tile_epilogue<MB, WGM, WGN, TM, TN>(acc, p, lds, n0, 0, [&](int pl, int & b, int & hw) {
    if (pl >= TH * TW) return false;
    const int ty = idiv_small(pl, TW, inv_tw), tx = pl - ty * TW;
    const int gy = oy0 + ty, ox = ox0 + tx;
    if (gy >= Htot || ox >= p.Wo) return false;
    b = idiv_small(gy, Hs, inv_hs);
    const int r = gy - b * Hs;
    if (r >= p.H) return false;
    hw = r * p.Wo + ox;
    return true;
  });
}

// ---------------------------------------------------------------- host side

namespace {
struct HaloCfgDesc {
  int bm, bn, pmax;
};
// configs: 0..3 BM 256 (BN 16/32/64/128), 4..7 BM 128 (BN 16/32/64/128), 8 BM 64 BN 64
constexpr HaloCfgDesc kHaloCfg[kHaloCfgs] = {
    {256, 16, 360}, {256, 32, 360}, {256, 64, 360}, {256, 128, 360},
    {128, 16, 216}, {128, 32, 216}, {128, 64, 216}, {128, 128, 216},
    {64, 64, 144},
};
}  // namespace

// Chunk per config (measured on MI355X): the BM 128 x BN 128 config runs 64-channel steps
// (two work-groups per CU fit either way); every other config uses 32-channel chunks, which
// keep the BM 256 configs at two work-groups per CU.
int halo_cfg_ck(int cfg, int cin) { return cin <= 16 ? 16 : (cin <= 32 || cfg != 7 ? 32 : 64); }
int halo_taps(int ck) { return ck == 16 ? 10 : 9; }

// Best tile of one config for a layer: fewest pixel slots plus patch fill; false if none.
static bool halo_tile(int cfg, int cout, int H, int W, int batch, long * wgs, int * th, int * tw)
{
  const HaloCfgDesc & d = kHaloCfg[cfg];
  const long Htot = (long)batch * (H + 1) - 1;
  double best = 1e30;
  for (int w = 1; w <= W && w <= d.bm; ++w) {
    int h = d.bm / w;
    h = (int)std::min<long>(h, Htot);
    h = std::min(h, d.pmax / (w + 2) - 2);
    h = std::min(h, kHaloMaxRows - 2);  // padded patch rows fit the LDS reserve
    if (h < 1) continue;
    const long ty = (Htot + h - 1) / h, tx = (W + w - 1) / w;
    const int hh = (int)((Htot + ty - 1) / ty), ww = (int)((W + tx - 1) / tx);  // balanced
    const double cost = (double)(ty * tx) * (d.bm + 0.3 * (hh + 2) * (ww + 2));
    if (cost < best) {
      best = cost;
      *th = hh;
      *tw = ww;
      *wgs = ty * tx * ((cout + d.bn - 1) / d.bn);
    }
  }
  return best < 1e30;
}

// Config choice (from MI355X measurements of the conv sweep shapes at batch 64): wide
// layers take BM 256 pixel tiles when that grid still gives 1.5 work-groups per CU, else
// BM 128; Cout <= 64 takes BM 128 (BN 64); Cout <= 32 takes BM 256.  Small grids fall back
// to the other BM.
bool halo_plan(int cin, int cout, int H, int W, int batch, int * cfg, int * th, int * tw)
{
  (void)cin;
  // tall-image rows and widths stay below 2^22 (the kernel's float-reciprocal divisions)
  if (H < 2 || W < 2 || (long)batch * (H + 1) >= (1L << 22) || W >= (1 << 22)) return false;
  const int bnc = cout <= 16 ? 0 : (cout <= 32 ? 1 : (cout <= 64 ? 2 : 3));
  const int big = bnc, small = 4 + bnc;
  long wb = 0, ws = 0;
  int hb = 0, hs = 0, tb = 0, ts = 0;
  const bool okb = halo_tile(big, cout, H, W, batch, &wb, &hb, &tb);
  const bool oks = halo_tile(small, cout, H, W, batch, &ws, &hs, &ts);
  int c;
  if (bnc == 3) c = (okb && wb >= 384) ? big : small;
  else if (bnc == 2) c = small;
  else c = (okb && wb >= 256) ? big : small;
  if (c == big && !okb) c = small;
  if (c == small && !oks) c = big;
  if ((c == big && !okb) || (c == small && !oks)) return false;
  *cfg = c;
  *th = c == big ? hb : hs;
  *tw = c == big ? tb : ts;
  // a grid of fewer work-groups than CUs (wide layers on small maps): BM 64 x BN 64 tiles
  long wq = 0;
  int hq = 0, tq = 0;
  if (cout > 32 && (c == big ? wb : ws) < 256 && halo_tile(8, cout, H, W, batch, &wq, &hq, &tq)) {
    *cfg = 8;
    *th = hq;
    *tw = tq;
  }
  return true;
}

long halo_grid_x(const ConvParams & p)
{
  const long Htot = (long)p.batch * (p.H + 1) - 1;
  return ((Htot + p.th - 1) / p.th) * ((p.Wo + p.tw - 1) / p.tw);
}

int halo_bn(int cfg) { return kHaloCfg[cfg].bn; }
int halo_pmax(int cfg) { return kHaloCfg[cfg].pmax; }

template <int MB, int WGM, int WGN, int TM, int TN, int PMAX>
static void launch_hc(const ConvParams & p, hipStream_t s)
{
  using T = TileShape<MB, WGM, WGN, TM, TN>;
  dim3 grid((unsigned)halo_grid_x(p), (unsigned)((p.Cout + T::BN - 1) / T::BN), 1);
  const int ck = p.ck;
  if (ck == 16) hipLaunchKernelGGL((conv3x3s1_kernel<MB, WGM, WGN, TM, TN, 16, PMAX>), grid, dim3(256), 0, s, p);
  else if (ck == 32) hipLaunchKernelGGL((conv3x3s1_kernel<MB, WGM, WGN, TM, TN, 32, PMAX>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((conv3x3s1_kernel<MB, WGM, WGN, TM, TN, 64, PMAX>), grid, dim3(256), 0, s, p);
}

void launch_conv_halo(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_halo(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  switch (p.halo - 1) {
  case 0: launch_hc<16, 4, 1, 4, 1, 360>(p, s); break;
  case 1: launch_hc<32, 4, 1, 2, 1, 360>(p, s); break;
  case 2: launch_hc<32, 2, 2, 4, 1, 360>(p, s); break;
  case 3: launch_hc<32, 2, 2, 4, 2, 360>(p, s); break;
  case 4: launch_hc<16, 4, 1, 2, 1, 216>(p, s); break;
  case 5: launch_hc<32, 4, 1, 1, 1, 216>(p, s); break;
  case 6: launch_hc<32, 2, 2, 2, 1, 216>(p, s); break;
  case 7: launch_hc<32, 2, 2, 2, 2, 216>(p, s); break;
  default: launch_hc<32, 2, 2, 1, 1, 144>(p, s); break;
  }
}

}  // namespace ivh
