// 3x3 stride-1 pad-1 convolution with Cin <= 64 on gfx950 fp16 MFMA, weights resident in LDS.
//
// Replaces, for the narrow layers that dominate the YOLO heads and C2f/C3k2 bottlenecks, the
// reference's conv3x3_ov (kernels/conv_ov.cl:133-297), conv3x3_blk (conv_blk.cl:118-296) and
// conv3x3_f16 (conv.cl:150-414):
//   y[co][p] = act(sum_{tap,ci} W[co][ci][tap] x[ci][p + tap] + b[co]) (+ r[co][p]).
//
// With Cin <= 64 the whole K range (9 taps x Cin) of a BN-channel block is at most 74 KB of
// fp16, so a work-group loads it into LDS once and keeps it there.  The grid is persistent
// (about one work-group per CU); each work-group walks a contiguous range of output tiles of
// the batch-as-one-tall-image (image b at rows [b*(H+1), b*(H+1)+H), a zero separator row
// after each image, as in conv_halo.hip).  Per tile:
//   * the (TH+2) x (TW+2) x CK input patch is in LDS; 9*CK/16 MFMA K slices run back to
//     back with no barrier (every operand is already resident);
//   * the next two tiles' patches are in flight in registers (buffer loads issued two tiles
//     ahead, out-of-image pixels read zeros from past the buffer's range);
//   * the previous tile's epilogue (bias, activation, fp16 rounding, stores) is interleaved
//     with this tile's MFMAs, so its VALU work -- two transcendentals per SiLU output -- can
//     overlap the matrix pipe instead of following it;
//   * two barriers per tile, around the write of the next patch to LDS.
// Outputs go straight from the accumulators to HBM: with 8-channel stores (SM 2) the two
// 4-channel runs a lane holds of a pixel and the two its partner lane (lane +- 32) holds are
// exchanged with v_permlane32_swap, so every lane writes 8 consecutive channels (16 bytes):
// half the store instructions of 4-channel (8-byte) stores, each touching the same number of
// 128-byte lines with twice the bytes.
// Wave layout: the 4 waves split the tile's pixels (TM 32-pixel blocks each) and share all
// BN = TN*32 channels, so an A (weight) fragment feeds TM MFMAs and a B (pixel) fragment TN.
#include <algorithm>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

// SM: output stores of 8 channels (2), 4 channels (1) or single elements (0)
template <int WGM, int WGN, int TM, int TN, int CK, int PMAX, int ACT, bool RES, int SM>
__global__ void __launch_bounds__(64 * WGM * WGN, 1) conv3x3s1_res_kernel(const ConvParams p)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  constexpr int NT = 64 * WGM * WGN;         // threads
  constexpr int BN = WGN * TN * 32;
  constexpr int NS = CK / 16;              // MFMA K slices per tap
  constexpr int NSL = 9 * NS;              // K slices per tile
  constexpr int KROW = 9 * CK;             // weights per output channel kept in LDS
  constexpr int LDK = KROW + 8;            // weight row pitch (halves): conflict-free reads
  constexpr int CKP = CK + 8;              // patch pixel pitch (halves)
  // Patch rows are padded so that every row starts where an unpadded linear layout of the
  // same pixels would start modulo 256 bytes: the 32 lanes of a B fragment (32 consecutive
  // tile pixels, wrapping tile rows) then hit LDS banks exactly as consecutive pixels do,
  // which is conflict-free (measured: a 32-pixel fragment over 8-wide tile rows read at half
  // the LDS rate without the pad).
  constexpr int PADH = ((256 - (4 * CKP) % 256) % 256) / 2;  // halves: -2 pixels mod 256 B
  constexpr int L_PATCH = PMAX * CKP + kResMaxRows * PADH;
  constexpr int CQ = CK / 8;               // 16-byte pieces per patch pixel
  constexpr int P_IT = (PMAX * CQ + NT - 1) / NT;
  constexpr int WQ = KROW / 8;             // 16-byte pieces per weight row
  constexpr int W_IT = (BN * WQ + NT - 1) / NT;
  constexpr int NG = TN * TM * 4;          // epilogue groups (4 accumulator values) per lane
  constexpr int NE = SM == 2 ? NG / 2 : NG;  // epilogue steps (a step is two groups with SM 2)
  __shared__ __attribute__((aligned(16))) _Float16 lds[BN * LDK + L_PATCH];
  __shared__ __attribute__((aligned(16))) float bias_s[BN];
  _Float16 * const Ws = lds;
  _Float16 * const Ps = lds + BN * LDK;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int TH = p.th, TW = p.tw, PW = TW + 2, PP = (TH + 2) * PW, RPH = PW * CKP + PADH;
  const int Hs = p.H + 1;                       // rows per image incl. separator
  const int tiles_x = (p.W + TW - 1) / TW;
  const int ntiles = ((p.batch * Hs - 1 + TH - 1) / TH) * tiles_x;
  // this work-group's contiguous tile range; XCD-aware so neighbouring ranges (which share
  // input rows at their ends) run on one XCD
  const int G = gridDim.x;
  const int r = xcd_tile(blockIdx.x, G);
  const int t_lo = (int)((long)r * ntiles / G), t_hi = (int)((long)(r + 1) * ntiles / G);
  const int ntl = t_hi - t_lo;
  if (ntl <= 0) return;
  const int n0 = blockIdx.y * BN;
  const float inv_tw = __builtin_amdgcn_rcpf((float)TW), inv_pw = __builtin_amdgcn_rcpf((float)PW);

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w + (long)n0 * p.kpad), (short)0, BN * p.kpad * 2, kBufDword3);

  // patch pieces of this thread: element e = tid + NT i -> patch pixel e / CQ (row, column
  // packed as row << 16 | column; row 0x7fff past the patch), piece e % CQ = tid % CQ
  const int q8 = (tid % CQ) * 8;
  int pyx[P_IT];
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int pp = (tid + i * NT) / CQ;
    const int py = idiv_small(pp, PW, inv_pw);
    pyx[i] = pp < PP ? (py << 16) | (pp - py * PW) : 0x7fff0000;
  }
  // tile t -> first output row (image b0, row r0 of it) and column of the tall image
  auto tile_origin = [&](int t, int & b0, int & r0, int & ox0) __attribute__((always_inline)) {
    const int ty = t / tiles_x;
    const int oy0 = ty * TH;
    b0 = oy0 / Hs;
    r0 = oy0 - b0 * Hs;
    ox0 = (t - ty * tiles_x) * TW;
  };
  // input pixel (b0 + 1, r - Hs) is at (b0, r) + delta: crossing one image boundary
  const int xcs = p.x.cs, xwcs = p.W * p.x.cs;
  const int xdelta = (int)p.x.img - Hs * xwcs;
  // patch of tile t into registers: branch-free offsets, out-of-image pixels read zeros
  auto load_patch = [&](int t, h8 (&rp)[P_IT]) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
    // first patch row is output row - 1: step back one row (into the previous image's
    // separator, or -1 above the first image)
    int rb = r0 - 1, bb = b0;
    if (rb < 0 && bb > 0) {
      rb += Hs;
      --bb;
    }
    const bool next_ok = bb + 1 < p.batch;
    const int base = bb * (int)p.x.img + (rb * p.W + ox0 - 1) * xcs + q8;
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      const int py = pyx[i] >> 16, px = pyx[i] & 0xffff;
      const int rr = rb + py;
      const bool wrap = rr >= Hs;
      const int rw = wrap ? rr - Hs : rr;
      const int ix = ox0 - 1 + px;
      const bool ok = (unsigned)rw < (unsigned)p.H && (unsigned)ix < (unsigned)p.W && (!wrap || next_ok);
      const int off = base + __umul24(py, xwcs) + __umul24(px, xcs) + (wrap ? xdelta : 0);
      const unsigned src = ok ? (unsigned)off * 2u : kBufOOB;
      rp[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, src, 0, 0));
    }
  };
  // ragged Cin: channels >= Cin of a piece are zeroed bitwise (padding channels or the next
  // pixel's data never reach the MFMAs)
  const bool ragged = (p.Cin % CK) != 0;
  u16x8 keep;
#pragma unroll
  for (int k = 0; k < 8; ++k) keep[k] = q8 + k < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
  auto store_patch = [&](const h8 (&rp)[P_IT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      if (pyx[i] != 0x7fff0000) {  // pixels past the patch are never read
        h8 v = rp[i];
        if (ragged) v = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, v) & keep);
        *reinterpret_cast<h8 *>(Ps + (pyx[i] >> 16) * RPH + (pyx[i] & 0xffff) * CKP + q8) = v;
      }
    }
  };

  h8 rpA[P_IT], rpB[P_IT];  // patches of tiles i + 1 and i + 2 in flight
  // start of this work-group's weight-load order: work-groups w, w + 8, ... share an XCD (and
  // its L2); rotating their orders spreads their first requests over the whole weight block
  // instead of every CU asking for the same lines at once
  const int wrot = (int)(((long)((blockIdx.x / kXcds) % 32) * (BN * WQ / 32)) % (BN * WQ));

  // ---- prologue: bias and weights into LDS, first patch
  if (tid < BN) bias_s[tid] = p.bias ? p.bias[n0 + tid] : 0.0f;
  {
    h8 rw[W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e0 = tid + i * NT;
      const int e = e0 < BN * WQ ? (e0 + wrot) % (BN * WQ) : e0, row = e / WQ, q = e - row * WQ;
      const unsigned src = e < BN * WQ ? (unsigned)((row * p.kpad + q * 8) * 2) : kBufOOB;
      rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wr, src, 0, 0));
    }
    load_patch(t_lo, rpA);
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e0 = tid + i * NT;
      const int e = e0 < BN * WQ ? (e0 + wrot) % (BN * WQ) : e0, row = e / WQ, q = e - row * WQ;
      if (e < BN * WQ) *reinterpret_cast<h8 *>(Ws + row * LDK + q * 8) = rw[i];
    }
    store_patch(rpA);
  }
  // the next two tiles' patches in flight (each is issued two tiles before it is needed)
  load_patch(t_lo + (1 < ntl ? 1 : 0), rpA);
  load_patch(t_lo + (2 < ntl ? 2 : 0), rpB);
  __syncthreads();

  // ---- per-lane fragment addresses and output slots (tile-independent)
  int bl[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int pl = wm * TM * 32 + tm * 32 + F::col(lane);
    const int pc = pl < TH * TW ? pl : 0;  // slot past the tile: computed on pixel 0, never stored
    const int ty = idiv_small(pc, TW, inv_tw), tx = pc - ty * TW;
    bl[tm] = ty * RPH + tx * CKP + F::kq(lane);
  }
  const int arow = (wn * TN * 32 + (lane & 31)) * LDK + F::kq(lane);
  int tapoff[9];
#pragma unroll
  for (int tap = 0; tap < 9; ++tap) tapoff[tap] = (tap / 3) * RPH + (tap % 3) * CKP;

  // output byte offsets of this lane's pixel blocks in tile t (past the buffer range: no
  // output), for y and the residual view.  Stores and residual loads are buffer accesses
  // whose out-of-range lanes are dropped / read zeros, so the epilogue has no branches.
  int syx[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int pl = wm * TM * 32 + tm * 32 + F::col(lane);
    const int ty = idiv_small(pl, TW, inv_tw);
    syx[tm] = pl < TH * TW ? (ty << 16) | (pl - ty * TW) : 0x7fff0000;
  }
  auto out_offsets = [&](int t, unsigned (&yo)[TM], unsigned (&ro)[TM]) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      int rr = r0 + (syx[tm] >> 16), b = b0;
      if (rr >= Hs) {  // TH + 2 <= Hs: at most one image boundary inside a tile
        rr -= Hs;
        ++b;
      }
      const int ox = ox0 + (syx[tm] & 0xffff);
      const bool ok = rr < p.H && b < p.batch && ox < p.W;
      const unsigned hw = (unsigned)(rr * p.W + ox);
      yo[tm] = ok ? ((unsigned)b * (unsigned)p.y.img + hw * (unsigned)p.y.cs + (unsigned)n0) * 2u : kBufOOB;
      if (RES) ro[tm] = ok ? ((unsigned)b * (unsigned)p.r.img + hw * (unsigned)p.r.cs + (unsigned)n0) * 2u : kBufOOB;
    }
  };
  const int cl0 = wn * TN * 32 + F::row(lane, 0);  // lane's first channel in the block
  // SM 1 / 2 with Cout % 4 / % 8 != 0: the last piece also writes the view's padding channels
  // (p.ypad of them, checked on the host)
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.H * p.W - 1) * p.y.cs +
                      (SM == 2 ? (p.Cout + 7) & ~7 : SM == 1 ? (p.Cout + 3) & ~3 : p.Cout);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);
  const long r_last = RES ? (long)(p.batch - 1) * p.r.img + ((long)p.H * p.W - 1) * p.r.cs + p.Cout : 0;
  const __amdgpu_buffer_rsrc_t rr_ = __builtin_amdgcn_make_buffer_rsrc(RES ? p.r.ptr : p.y.ptr, (short)0,
                                                                       (int)(r_last * 2), kBufDword3);
  // lane channel cl (within the block) -> byte offset or out of range
  auto chan_off = [&](unsigned base, int cl) __attribute__((always_inline)) {
    return n0 + cl < p.Cout ? base + (unsigned)cl * 2u : kBufOOB;
  };
  // residual values of this lane's outputs in tile t (channels-last, 4 channels a load)
  auto load_res = [&](const unsigned (&ro)[TM], h4 (&rv)[NG]) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;
      rv[g] = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rr_, chan_off(ro[tm], tn * 32 + cl0 + 2 * v4), 0, 0));
    }
  };
  // epilogue group g of tile accumulators ac (4 values: 4 consecutive channels of one pixel):
  // bias + activation in fp32, one rounding, then + residual (rounded again)
  auto epi_vals = [&](const acc_t (&ac)[TN][TM], const h4 (&rv)[NG], int g) __attribute__((always_inline)) {
    const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;
    const int cl = tn * 32 + cl0 + 2 * v4;  // F::row(lane, v4)
    const float4 b4 = *reinterpret_cast<const float4 *>(bias_s + cl);
    // The fp32 results pass through an empty asm so that every copy of this code (there is
    // one per accumulator set, and the last tile's) rounds them the same way: fp32, then
    // one fp16 rounding, never a fused multiply-convert.  An image's outputs then do not
    // depend on which tile, and so which batch size, computed them.
    float o[4] = {act_fast<ACT>(ac[tn][tm][v4 + 0] + b4.x), act_fast<ACT>(ac[tn][tm][v4 + 1] + b4.y),
                  act_fast<ACT>(ac[tn][tm][v4 + 2] + b4.z), act_fast<ACT>(ac[tn][tm][v4 + 3] + b4.w)};
    h4 hv;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      __asm__("" : "+v"(o[k]));
      hv[k] = (_Float16)o[k];
    }
    if (RES) {
#pragma unroll
      for (int k = 0; k < 4; ++k) hv[k] = (_Float16)((float)hv[k] + (float)rv[g][k]);
    }
    return hv;
  };
  // epilogue step e: group e (SM 0 / 1), or groups 2e and 2e + 1 (SM 2: accumulator values
  // v4 and v4 + 4 of one block, channels c..c+3 and c+8..c+11 on lanes < 32, c+4..c+7 and
  // c+12..c+15 on lanes >= 32), computed and stored
  auto epi_step = [&](const acc_t (&ac)[TN][TM], const unsigned (&yo)[TM], const h4 (&rv)[NG], int e)
      __attribute__((always_inline)) {
    if (SM == 2) {
      const int g = 2 * e;
      const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;  // v4 = 0 or 8
      const u2 a = __builtin_bit_cast(u2, epi_vals(ac, rv, g));
      const u2 b = __builtin_bit_cast(u2, epi_vals(ac, rv, g + 1));
      // lanes < 32 keep their channels c..c+3 and take c+4..c+7 from lane + 32; lanes >= 32
      // take c+8..c+11 from lane - 32 and keep c+12..c+15
      const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
      const u4 q = {s0[0], s1[0], s0[1], s1[1]};
      const int cl = tn * 32 + cl0 + 2 * v4 + 4 * (lane >> 5);  // first of the lane's 8 channels
      __builtin_amdgcn_raw_buffer_store_b128(q, yr, chan_off(yo[tm], cl), 0, 0);
    } else {
      const int tn = e / (TM * 4), tm = (e / 4) % TM, v4 = (e % 4) * 4;
      const int cl = tn * 32 + cl0 + 2 * v4;
      const h4 hv = epi_vals(ac, rv, e);
      if (SM == 1) {
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, hv), yr, chan_off(yo[tm], cl), 0, 0);
      } else {
        // (bit-cast the whole vector: hipcc reads element 0 for a bit cast of hv[k])
        const u16x4 hu = __builtin_bit_cast(u16x4, hv);
#pragma unroll
        for (int k = 0; k < 4; ++k) __builtin_amdgcn_raw_buffer_store_b16(hu[k], yr, chan_off(yo[tm], cl + k), 0, 0);
      }
    }
  };

  // one tile: residual loads of this tile, MFMAs over the resident patch with the previous
  // tile's epilogue interleaved (accp / yop / rvp; on the first tile they hold zeros and
  // out-of-range offsets and store nothing), then the two-barrier patch hand-over
  auto tile = [&](acc_t (&acc)[TN][TM], const acc_t (&accp)[TN][TM], unsigned (&yo)[TM], const unsigned (&yop)[TM],
                  h4 (&rv)[NG], const h4 (&rvp)[NG], h8 (&rp)[P_IT], int i) __attribute__((always_inline)) {
    unsigned ro[TM];
    out_offsets(t_lo + i, yo, ro);
    if (RES) load_res(ro, rv);
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int v = 0; v < F::NV; ++v) acc[a][b][v] = 0.0f;
    // K slices with the fragments of slice s + 1 read from LDS while slice s's MFMAs run
    // (two register sets); the epilogue groups spread evenly over the slices, with a
    // residual from a third of the way in (its loads, issued at the tile's start, land)
    h8 fa[2][TN], fb[2][TM];
    auto frags = [&](int s, h8 (&a)[TN], h8 (&b)[TM]) __attribute__((always_inline)) {
      const int tap = s / NS, j = s % NS;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        a[tn] = *reinterpret_cast<const h8 *>(Ws + arow + tn * 32 * LDK + tap * CK + j * 16);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) b[tm] = *reinterpret_cast<const h8 *>(Ps + bl[tm] + tapoff[tap] + j * 16);
    };
    constexpr int S0 = RES ? NSL / 3 : 0, SPAN = NSL - S0;
    frags(0, fa[0], fb[0]);
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const int s = tap * NS + j;
        if (s + 1 < NSL) frags(s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = F::mma(fa[s & 1][tn], fb[s & 1][tm], acc[tn][tm]);
#pragma unroll
        for (int e = 0; e < NE; ++e)
          if (S0 + e * SPAN / NE == s) epi_step(accp, yop, rvp, e);
      }
    }
    __syncthreads();  // patch reads done
    if (i + 1 < ntl) {
      store_patch(rp);  // tile i + 1
      load_patch(t_lo + (i + 3 < ntl ? i + 3 : i + 1), rp);
      __syncthreads();  // next patch in LDS
    }
  };

  acc_t accA[TN][TM], accB[TN][TM];
  unsigned yoA[TM], yoB[TM];
  h4 rvA[NG], rvB[NG];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) accB[a][b][v] = 0.0f;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) yoB[tm] = kBufOOB;
#pragma unroll
  for (int g = 0; g < NG; ++g) rvB[g] = h4{};
  for (int i = 0; i < ntl; i += 2) {
    tile(accA, accB, yoA, yoB, rvA, rvB, rpA, i);
    if (i + 1 < ntl) tile(accB, accA, yoB, yoA, rvB, rvA, rpB, i + 1);
  }
  // last tile's epilogue
  if (ntl & 1) {
#pragma unroll
    for (int e = 0; e < NE; ++e) epi_step(accA, yoA, rvA, e);
  } else {
#pragma unroll
    for (int e = 0; e < NE; ++e) epi_step(accB, yoB, rvB, e);
  }
}

// ---------------------------------------------------------------- ping-pong variant
//
// 32 < Cin <= 64 with Cin % 8 == 0 and Cout > 32: the same convolution, tiles (BN = 64
// output channels per work-group) and epilogue, with the waves of every SIMD taking turns
// instead of each interleaving its own epilogue with its own MFMAs (measured on gfx950: a
// wave's VALU work and its own MFMAs barely overlap, while one wave's VALU work runs under
// another wave's MFMAs at almost full speed for both).  Twelve waves form three groups of
// four (waves 0-3, 4-7, 8-11: one wave of each per SIMD) and a work-group's tiles rotate
// over the groups.  In phase k the group owning tile k runs all of its MFMAs -- each wave
// 64 pixels x 64 channels, 2 x 2 blocks of 32 x 32, so every fragment read from LDS feeds
// two MFMAs, with one fragment read issued behind each MFMA -- while the group that ran
// tile k - 1 stores the first half of its outputs (activation, one fp16 rounding, residual;
// the accumulators start from the bias) and the group of tiles k - 2 and k + 1 stores the
// second half of tile k - 2 and copies the input patch of tile k + 1 into the buffer tile
// k - 1 used, by buffer loads with the LDS flag (no VGPR round trip); one barrier ends the
// phase.  So a tile's epilogue VALU work -- two transcendentals per SiLU output -- runs on
// two waves per SIMD under the third wave's MFMAs, and output stores are never waited for.
// LDS: the resident weights (64 rows of 9 x 64 fp16, pitch 584: conflict-free A reads), two
// patch buffers and the bias.  A patch buffer holds up to 324 pixels as dense 128-byte rows
// of eight 16-byte pieces (8 channels each); piece q of patch pixel (py, px) sits at
// position q ^ (bits 1..3 of py * TW + px), so the 16 lanes of a B-fragment read quarter --
// 16 consecutive tile pixels, whose py * TW + px are 16 consecutive integers -- hit 16
// distinct 16-byte bank groups with no padding (two buffers and the weights fill 158 KB).
namespace {
typedef __attribute__((address_space(3))) void lds_void_t;
constexpr int kPpLdk = 9 * 64 + 8;   // weight row pitch (halves)
constexpr int kPpPix = 324;          // patch pixels per buffer
constexpr int kPpSlots = 2624;       // patch buffer slots: 41 DMA instructions of 64 >= 8 * 324
constexpr int kPpDmaPerWave = 11;    // patch DMA instructions per wave (4 waves x 11 >= 41)
constexpr int kPpWDma = 73;          // weight DMA instructions: 64 rows x 73 slots (72 + pad)
constexpr int kPpGroups = 3;         // wave groups (one wave of each per SIMD)

__device__ __forceinline__ void pp_dma16(__amdgpu_buffer_rsrc_t r, void * lds, unsigned voff)
{
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 16, (int)voff, 0, 0, 0);
}

typedef unsigned pp_u4 __attribute__((ext_vector_type(4)));
// The same copy issued as inline assembly, so the compiler does not track it: its waitcnt
// pass would otherwise make the next LDS read of any patch buffer wait for every vector
// memory operation still in flight (the epilogue's output stores included).  The caller
// waits for these copies itself (s_waitcnt vmcnt) before the barrier that publishes them.
// rs: the buffer descriptor; lds: the LDS byte address of the 64 destination slots.
__device__ __forceinline__ void pp_dma16_untracked(pp_u4 rs, unsigned lds, unsigned voff)
{
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                   :
                   : "v"(voff), "s"(rs), "s"(lds)
                   : "memory", "m0");
}
}  // namespace

template <int NGRP, int ACT, bool RES, int SM>
__global__ void __launch_bounds__(256 * NGRP, 1) conv3x3s1_pp_kernel(const ConvParams p)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  constexpr int BN = 64, TM = 2, TN = 2, NSL = 36, LDK = kPpLdk;
  static_assert(NGRP == 3 && TM == 2, "three wave groups, an epilogue part per pixel block");
  constexpr int NG = TN * TM * 4;            // epilogue groups (4 accumulator values) per lane
  constexpr int NE = SM == 2 ? NG / 2 : NG;  // epilogue steps
  __shared__ __attribute__((aligned(16))) _Float16 Ws[64 * LDK];
  __shared__ __attribute__((aligned(16))) _Float16 P0[kPpSlots * 8];
  __shared__ __attribute__((aligned(16))) _Float16 P1[kPpSlots * 8];
  __shared__ __attribute__((aligned(16))) float bias_s[BN];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = wave & 3;  // position in the group (the SIMD it shares with its partner)
  const int TH = p.th, TW = p.tw, PW = TW + 2, PP = (TH + 2) * PW;
  const int Hs = p.H + 1;
  const int tiles_x = (p.W + TW - 1) / TW;
  const int ntiles = ((p.batch * Hs - 1 + TH - 1) / TH) * tiles_x;
  const int G = gridDim.x;
  const int r = xcd_tile(blockIdx.x, G);
  const int t_lo = (int)((long)r * ntiles / G), t_hi = (int)((long)(r + 1) * ntiles / G);
  const int ntl = t_hi - t_lo;
  if (ntl <= 0) return;
  const int n0 = blockIdx.y * BN;
  const float inv_tw = __builtin_amdgcn_rcpf((float)TW), inv_pw = __builtin_amdgcn_rcpf((float)PW);

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  // a grouped launch: this channel block's input channels start y * xg channels into x
  const __half * const xp = p.x.ptr + (long)blockIdx.y * p.xg;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(xp), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w + (long)n0 * p.kpad), (short)0, BN * p.kpad * 2, kBufDword3);
  const unsigned long long xaddr = reinterpret_cast<unsigned long long>(xp);
  const pp_u4 xrs = {(unsigned)xaddr, (unsigned)(xaddr >> 32) & 0xffffu, (unsigned)(x_last * 2), (unsigned)kBufDword3};

  // ---- prologue: weights into LDS by DMA (slot s = row s / 73, piece s % 73; piece 72 is
  // the row's pad), bias
  constexpr int NW = 4 * NGRP;  // waves
#pragma unroll
  for (int u = 0; u < (kPpWDma + NW - 1) / NW; ++u) {
    const int i0 = u * NW + wave;
    if (i0 < kPpWDma) {
      // work-groups sharing an XCD (and its L2) start at different instructions, so their
      // first requests spread over the whole weight block
      const int ins = (i0 + (int)(blockIdx.x / kXcds) * 7) % kPpWDma;
      const unsigned s = (unsigned)(ins * 64 + lane), row = s / 73u, c = s - row * 73u;
      pp_dma16(wr, Ws + ins * 512, c < 72u ? (row * (unsigned)p.kpad + c * 8u) * 2u : kBufOOB);
    }
  }
  if (tid < BN) bias_s[tid] = p.bias ? p.bias[n0 + tid] : 0.0f;

  // patch slots of this lane's DMA instructions (instruction u * 4 + wg of its group covers
  // slots 64 (u * 4 + wg) ..): patch row << 16 | column << 3 | channel piece, bit 12 = no
  // input (slots past the patch)
  const int ninst = (PP * 8 + 63) / 64;
  unsigned pdesc[kPpDmaPerWave];
#pragma unroll
  for (int u = 0; u < kPpDmaPerWave; ++u) {
    const int s = (u * 4 + wg) * 64 + lane, pp = s >> 3;
    const int py = idiv_small(pp, PW, inv_pw), px = pp - py * PW;
    const int q = (s & 7) ^ (((py * TW + px) >> 1) & 7);
    pdesc[u] = pp < PP ? ((unsigned)py << 16) | ((unsigned)px << 3) | (unsigned)q : 1u << 12;
  }
  // tile t -> first output row (image b0, row r0 of it) and column of the tall image
  auto tile_origin = [&](int t, int & b0, int & r0, int & ox0) __attribute__((always_inline)) {
    const int ty = t / tiles_x;
    const int oy0 = ty * TH;
    b0 = oy0 / Hs;
    r0 = oy0 - b0 * Hs;
    ox0 = (t - ty * tiles_x) * TW;
  };
  const int xcs = p.x.cs, xwcs = p.W * p.x.cs;
  const int xdelta = (int)p.x.img - Hs * xwcs;  // (b0 + 1, r - Hs) is at (b0, r) + xdelta
  // Source byte offsets of this wave's patch slots for tile t (fn(u, offset) for each of its
  // instructions u): pixels outside the image, separator rows and pieces at or past Cin read
  // zeros from past the buffer range.
  auto patch_src = [&](int t, auto && fn) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
    int rb = r0 - 1, bb = b0;  // patch row 0 is output row - 1
    if (rb < 0 && bb > 0) {
      rb += Hs;
      --bb;
    }
    const bool next_ok = bb + 1 < p.batch;
    const int base = bb * (int)p.x.img + (rb * p.W + ox0 - 1) * xcs;
#pragma unroll
    for (int u = 0; u < kPpDmaPerWave; ++u) {
      if (u * 4 + wg < ninst) {
        unsigned d = pdesc[u];
        __asm__ volatile("" : "+v"(d));  // decoded here, not hoisted out of the phase loop
        const int py = (int)(d >> 16), px = (int)((d >> 3) & 511u), q = (int)(d & 7u);
        const int rr = rb + py;
        const bool wrap = rr >= Hs;
        const int rw = wrap ? rr - Hs : rr;
        const int ix = ox0 - 1 + px;
        const bool ok = !(d & (1u << 12)) && (unsigned)rw < (unsigned)p.H && (unsigned)ix < (unsigned)p.W &&
                        (!wrap || next_ok) && q * 8 < p.Cin;
        const int off = base + __umul24(py, xwcs) + __umul24(px, xcs) + q * 8 + (wrap ? xdelta : 0);
        fn(u, ok ? (unsigned)off * 2u : kBufOOB);
      }
    }
  };
  // patch of tile t into buffer P by DMA: tracked (the first tile) or not (in the phase loop)
  auto dma_patch = [&](int t, _Float16 * P) __attribute__((always_inline)) {
    patch_src(t, [&](int u, unsigned src) __attribute__((always_inline)) { pp_dma16(xr, P + (u * 4 + wg) * 512, src); });
  };
  auto dma_patch_untracked = [&](int t, _Float16 * P) __attribute__((always_inline)) {
    const unsigned lds = (unsigned)reinterpret_cast<unsigned long>((__attribute__((address_space(3))) _Float16 *)P);
    patch_src(t, [&](int u, unsigned src) __attribute__((always_inline)) {
      pp_dma16_untracked(xrs, lds + (unsigned)((u * 4 + wg) * 1024), src);
    });
  };

  // ---- per-lane fragment geometry (tile-independent): the wave's pixels are
  // wg * 64 + tm * 32 + lane % 32 of the tile; a slot past the tile computes pixel 0
  const int h16 = (lane >> 5) << 4;  // the lane's half of a 16-channel slice: piece 2 j + h
  unsigned pb[TM], pv[TM];           // patch byte offset and tile-linear index at tap (0, 0)
  int syx[TM];                       // output (row << 16 | column) in the tile
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int pl = wg * 64 + tm * 32 + F::col(lane);
    const int pc = pl < TH * TW ? pl : 0;
    const int ty = idiv_small(pc, TW, inv_tw), tx = pc - ty * TW;
    pb[tm] = (unsigned)(ty * PW + tx) * 128u;
    pv[tm] = (unsigned)(ty * TW + tx);
    const int oy = idiv_small(pl, TW, inv_tw);
    syx[tm] = pl < TH * TW ? (oy << 16) | (pl - oy * TW) : 0x7fff0000;
  }
  const int arow = ((lane & 31) * LDK + F::kq(lane)) * 2;  // A fragment byte offset at slice 0

  // ---- output side (as in the resident-weight kernel)
  const int cl0 = F::row(lane, 0);
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.H * p.W - 1) * p.y.cs +
                      (SM == 2 ? (p.Cout + 7) & ~7 : SM == 1 ? (p.Cout + 3) & ~3 : p.Cout);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);
  const long r_last = RES ? (long)(p.batch - 1) * p.r.img + ((long)p.H * p.W - 1) * p.r.cs + p.Cout : 0;
  const __amdgpu_buffer_rsrc_t rr_ = __builtin_amdgcn_make_buffer_rsrc(RES ? p.r.ptr : p.y.ptr, (short)0,
                                                                       (int)(r_last * 2), kBufDword3);
  auto out_offsets = [&](int t, unsigned (&yo)[TM], unsigned (&ro)[TM]) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      int rr = r0 + (syx[tm] >> 16), b = b0;
      if (rr >= Hs) {  // TH + 2 <= Hs: at most one image boundary inside a tile
        rr -= Hs;
        ++b;
      }
      const int ox = ox0 + (syx[tm] & 0xffff);
      const bool ok = rr < p.H && b < p.batch && ox < p.W;
      const unsigned hw = (unsigned)(rr * p.W + ox);
      yo[tm] = ok ? ((unsigned)b * (unsigned)p.y.img + hw * (unsigned)p.y.cs + (unsigned)n0) * 2u : kBufOOB;
      if (RES) ro[tm] = ok ? ((unsigned)b * (unsigned)p.r.img + hw * (unsigned)p.r.cs + (unsigned)n0) * 2u : kBufOOB;
    }
  };
  auto chan_off = [&](unsigned base, int cl) __attribute__((always_inline)) {
    return n0 + cl < p.Cout ? base + (unsigned)cl * 2u : kBufOOB;
  };
  // residual values of the groups of pixel block h (all channels)
  auto load_res = [&](const unsigned (&ro)[TM], h4 (&rv)[NG], int h) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;
      if (tm == h)
        rv[g] = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rr_, chan_off(ro[tm], tn * 32 + cl0 + 2 * v4), 0, 0));
    }
  };
  // bias + activation in fp32, one rounding, then + residual (rounded again); the empty asm
  // keeps every copy of this code on the same fp32 -> fp16 path
  auto epi_vals = [&](const acc_t (&ac)[TN][TM], const h4 (&rv)[NG], int g) __attribute__((always_inline)) {
    const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;
    float o[4] = {act_fast<ACT>(ac[tn][tm][v4 + 0]), act_fast<ACT>(ac[tn][tm][v4 + 1]),
                  act_fast<ACT>(ac[tn][tm][v4 + 2]), act_fast<ACT>(ac[tn][tm][v4 + 3])};
    h4 hv;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      __asm__("" : "+v"(o[k]));
      hv[k] = (_Float16)o[k];
    }
    if (RES) {
#pragma unroll
      for (int k = 0; k < 4; ++k) hv[k] = (_Float16)((float)hv[k] + (float)rv[g][k]);
    }
    return hv;
  };
  auto epi_step = [&](const acc_t (&ac)[TN][TM], const unsigned (&yo)[TM], const h4 (&rv)[NG], int e)
      __attribute__((always_inline)) {
    if (SM == 2) {
      const int g = 2 * e;
      const int tn = g / (TM * 4), tm = (g / 4) % TM, v4 = (g % 4) * 4;
      const u2 a = __builtin_bit_cast(u2, epi_vals(ac, rv, g));
      const u2 b = __builtin_bit_cast(u2, epi_vals(ac, rv, g + 1));
      const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
      const u4 q = {s0[0], s1[0], s0[1], s1[1]};
      const int cl = tn * 32 + cl0 + 2 * v4 + 4 * (lane >> 5);
      __builtin_amdgcn_raw_buffer_store_b128(q, yr, chan_off(yo[tm], cl), 0, 0);
    } else {
      const int tn = e / (TM * 4), tm = (e / 4) % TM, v4 = (e % 4) * 4;
      const int cl = tn * 32 + cl0 + 2 * v4;
      const h4 hv = epi_vals(ac, rv, e);
      if (SM == 1) {
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, hv), yr, chan_off(yo[tm], cl), 0, 0);
      } else {
        const u16x4 hu = __builtin_bit_cast(u16x4, hv);
#pragma unroll
        for (int k = 0; k < 4; ++k) __builtin_amdgcn_raw_buffer_store_b16(hu[k], yr, chan_off(yo[tm], cl + k), 0, 0);
      }
    }
  };

  // ---- MFMA phase: the 36 K slices of one tile from buffer P, fragments read two slices
  // ahead into a three-set register ring
  auto mfma_tile = [&](const _Float16 * P, unsigned poff, acc_t (&acc)[TN][TM]) __attribute__((always_inline)) {
    const char * const Pb = reinterpret_cast<const char *>(P);
    const char * const Wb = reinterpret_cast<const char *>(Ws) + arow;
    // the per-tap offsets below are the same in every phase; computed afresh (a few VALU
    // operations per tap) rather than hoisted out of the phase loop into 36+ live registers
    unsigned pbt[TM], pvt[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      pbt[tm] = pb[tm] + poff;
      pvt[tm] = pv[tm];
      __asm__ volatile("" : "+v"(pbt[tm]), "+v"(pvt[tm]));
    }
    unsigned tb[TM], tk[TM];  // B byte offset and swizzled piece offset of the prefetch tap
    auto set_tap = [&](int tap) __attribute__((always_inline)) {
      const int dy = tap / 3, dx = tap % 3;
      const unsigned boff = (unsigned)((dy * PW + dx) * 128), voff = (unsigned)(dy * TW + dx);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        tb[tm] = pbt[tm] + boff;
        tk[tm] = ((((pvt[tm] + voff) >> 1) & 7u) << 4) ^ (unsigned)h16;
      }
    };
    h8 fa[3][TN], fb[3][TM];
    auto frags = [&](auto S) __attribute__((always_inline)) {
      constexpr int s = decltype(S)::value, tap = s / 4, j = s % 4, k = s % 3;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        fa[k][tn] = *reinterpret_cast<const h8 *>(Wb + (tn * 32 * LDK + tap * 64 + j * 16) * 2);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        fb[k][tm] = *reinterpret_cast<const h8 *>(Pb + tb[tm] + (tk[tm] ^ (unsigned)(j << 5)));
    };
    set_tap(0);
    frags(std::integral_constant<int, 0>{});
    frags(std::integral_constant<int, 1>{});
    // the accumulators start from the bias: lane rows 8 i + 4 (lane / 32) + 0..3 of block tn
    // are four consecutive channels
    acc_t bias_v[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 b4 = *reinterpret_cast<const float4 *>(bias_s + tn * 32 + F::row(lane, 4 * i));
        bias_v[tn][4 * i] = b4.x;
        bias_v[tn][4 * i + 1] = b4.y;
        bias_v[tn][4 * i + 2] = b4.z;
        bias_v[tn][4 * i + 3] = b4.w;
      }
    static_for<0, NSL>([&](auto S) __attribute__((always_inline)) {
      constexpr int s = decltype(S)::value, k = s % 3;
      if constexpr (s + 2 < NSL) {
        if constexpr ((s + 2) % 4 == 0) set_tap((s + 2) / 4);
        frags(std::integral_constant<int, s + 2>{});
      }
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          acc[tn][tm] = F::mma(fa[k][tn], fb[k][tm], s == 0 ? bias_v[tn] : acc[tn][tm]);
      // one fragment read and a VALU operation behind each MFMA: a lone wave issues them
      // while the matrix pipe is busy instead of between MFMA groups
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // the first tile's patch into buffer 0
  const int grp = wave >> 2;
  if (grp == 0) dma_patch(t_lo, P0);
  __builtin_amdgcn_s_waitcnt(kVmWait0);
  __syncthreads();

  // Phase k = 0 .. ntl + 1; group g has role (k - g) mod 3 in it:
  //   0: the MFMAs of tile k (patch in buffer k % 2);
  //   1: the first half of the epilogue of tile k - 1;
  //   2: the patch of tile k + 1 -- the group's next tile -- into buffer (k + 1) % 2, which
  //      tile k - 1 read in the phase before, and the second half of the epilogue of tile
  //      k - 2.
  // A tile's epilogue is spread over two phases and two waves per SIMD; output stores are
  // never waited for.  Each group walks its roles in order (code per role, so registers live
  // only where they are used).
  const int nph = ntl + 2;
  acc_t acc[TN][TM];
  int k = 0;
  // epilogue part H: the steps of pixel block H (all 64 channels, so every 128-byte output
  // pixel is written within one phase and leaves L2 whole)
  auto epi_part = [&](int te, auto H) __attribute__((always_inline)) {
    constexpr int h = decltype(H)::value;
    unsigned yo[TM], ro[TM];
    h4 rv[NG];
    out_offsets(t_lo + te, yo, ro);
    if (RES) load_res(ro, rv, h);
    static_for<0, NE>([&](auto E) __attribute__((always_inline)) {
      constexpr int e = decltype(E)::value, g = SM == 2 ? 2 * e : e;
      if constexpr ((g / 4) % TM == h) epi_step(acc, yo, rv, e);
    });
  };
  // LDS hand-over only: no fence, so outstanding output stores do not hold the barrier
  auto end_phase = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_barrier();
    ++k;
  };
  auto role1 = [&]() __attribute__((always_inline)) {
    if (k >= 1 && k - 1 < ntl) epi_part(k - 1, std::integral_constant<int, 0>{});
    end_phase();
  };
  auto role2 = [&]() __attribute__((always_inline)) {
    const bool copy = k + 1 < ntl;
    if (copy) {
      if ((k + 1) & 1) dma_patch_untracked(t_lo + k + 1, P1);
      else dma_patch_untracked(t_lo + k + 1, P0);
    }
    if (k >= 2 && k - 2 < ntl) {
      epi_part(k - 2, std::integral_constant<int, 1>{});
      // the copies were issued before this part's stores, and vector memory operations
      // complete in order: wait for all but the stores
      constexpr int nst = (SM == 0 ? 4 : 1) * (NE / 2);
      __builtin_amdgcn_s_waitcnt(vm_wait(nst < 63 ? nst : 63));
    } else {
      __builtin_amdgcn_s_waitcnt(kVmWait0);
    }
    end_phase();
  };
  if (grp == 2) role1();
  if (grp >= 1) role2();
  while (k < nph) {
    if (k < ntl) {
      __builtin_amdgcn_s_setprio(1);
      // one copy of the MFMA code for both buffers: buffer 1 as a byte offset from buffer 0
      mfma_tile(P0, (k & 1) ? (unsigned)(reinterpret_cast<char *>(P1) - reinterpret_cast<char *>(P0)) : 0u, acc);
      __builtin_amdgcn_s_setprio(0);
    }
    end_phase();
    if (k >= nph) break;
    role1();
    if (k >= nph) break;
    role2();
  }
}

// ---------------------------------------------------------------- host side

namespace {
struct ResCfgDesc {
  int bm, bn, pmax;
};
// Eight waves (two per SIMD, so one wave's epilogue VALU work overlaps the other's MFMAs):
//   0: 4 x 2 waves of 2 x 1 blocks (BM 256, BN 64; Cout > 32)
//   1: 8 x 1 waves of 2 x 1 blocks (BM 512, BN 32; Cout <= 32, Cin <= 32)
//   2: 8 x 1 waves of 1 x 1 blocks (BM 256, BN 32; Cout <= 32, Cin > 32)
//   3: the ping-pong kernel, two groups of 4 waves of 2 x 2 blocks (BM 256, BN 64; Cout > 32,
//      32 < Cin <= 64, Cin % 8 == 0)
// Patch sizes keep resident weights + patch(es) within the 160 KB of LDS at Cin 64.
constexpr int kResP0 = 352, kResP1 = 720, kResP2 = 352;
constexpr ResCfgDesc kResCfg[4] = {{256, 64, kResP0}, {512, 32, kResP1}, {256, 32, kResP2}, {256, 64, kPpPix}};
constexpr int kResCUs = 256;  // one work-group per CU
}  // namespace

int res_ck(int cin) { return cin <= 32 ? 32 : 64; }
int res_bn(int cfg) { return kResCfg[cfg].bn; }
int res_bm(int cfg) { return kResCfg[cfg].bm; }
int res_pmax(int cfg) { return kResCfg[cfg].pmax; }

long res_tiles(const ConvParams & p)
{
  const long Htot = (long)p.batch * (p.H + 1) - 1;
  return ((Htot + p.th - 1) / p.th) * ((p.W + p.tw - 1) / p.tw);
}

// Persistent grid: about one work-group per CU over all channel blocks, a multiple of the
// 8 XCDs when it is that large.
int res_grid_x(const ConvParams & p, int cfg)
{
  const int nblk = (p.Cout + kResCfg[cfg].bn - 1) / kResCfg[cfg].bn;
  long g = std::max(1, kResCUs / nblk);
  if (g >= 8) g = g / 8 * 8;
  return (int)std::min<long>(g, res_tiles(p));
}

// 8-channel stores when every 8-channel piece is inside the view or runs into its own padding
// channels, else 4-channel stores under the same condition, else single elements
int res_store_mode(const ConvParams & p)
{
  if (p.Cout % 8 == 0 || p.ypad >= 8 - p.Cout % 8) return 2;
  if (p.Cout % 4 == 0 || p.ypad >= 4 - p.Cout % 4) return 1;
  return 0;
}
int res_store_width(const ConvParams & p) { return res_store_mode(p) == 2 ? 8 : res_store_mode(p) == 1 ? 4 : 1; }

bool res_views_ok(const ConvParams & p)
{
  auto ok = [&](const View & v) {
    if (v.layout != kNHWC || (v.cs % 4) || (v.img % 4) || (reinterpret_cast<uintptr_t>(v.ptr) % 8)) return false;
    const long last = (long)(p.batch - 1) * v.img + ((long)p.H * p.W - 1) * v.cs + p.Cout + 3;
    return last * 2 < (1L << 31) && (long)p.batch * v.img < (1L << 31);
  };
  if (!ok(p.y)) return false;
  if (p.r.ptr && (!ok(p.r) || p.Cout % 4)) return false;
  return p.H == p.Ho && p.W == p.Wo && (long)p.W * p.x.cs < (1L << 23);
}

bool res_plan(int cin, int cout, int H, int W, int batch, int act, bool pingpong, int * cfg, int * th, int * tw)
{
  if (cin > 64 || cin <= 16 || H < 3 || W < 2 || (long)batch * (H + 1) >= (1L << 22) || W >= (1 << 22)) return false;
  if (act != kActNone && act != kActSiLU && act != kActReLU && act != kActHSwish) return false;
  const int ck = res_ck(cin);
  const int c = cout > 32 ? (pingpong && ck == 64 && cin % 8 == 0 ? 3 : 0) : (ck == 64 ? 2 : 1);
  const ResCfgDesc & d = kResCfg[c];
  const int nblk = (cout + d.bn - 1) / d.bn;
  long g = std::max(1, kResCUs / nblk);
  if (g >= 8) g = g / 8 * 8;
  const long Htot = (long)batch * (H + 1) - 1;
  // fewest rounds of tiles per work-group first (the critical path), then the least work
  // over the chip: MFMA slots plus patch fill of every tile
  long best_rounds = 1L << 40;
  double best = 1e30;
  for (int w = 1; w <= W && w <= d.bm; ++w) {
    int h = std::min(d.bm / w, H - 1);           // TH + 2 <= H + 1
    h = (int)std::min<long>(h, Htot);
    h = std::min(h, d.pmax / (w + 2) - 2);
    h = std::min(h, kResMaxRows - 2);            // padded patch rows fit the LDS reserve
    if (h < 1) continue;
    const long ty = (Htot + h - 1) / h, tx = (W + w - 1) / w;
    const int hh = (int)((Htot + ty - 1) / ty), ww = (int)((W + tx - 1) / tx);  // balanced
    const long n = ty * tx;
    const long rounds = (n + std::min<long>(g, n) - 1) / std::min<long>(g, n);
    const double work = (double)n * (d.bm + 0.1 * (hh + 2) * (ww + 2));
    if (rounds < best_rounds || (rounds == best_rounds && work < best)) {
      best_rounds = rounds;
      best = work;
      *th = hh;
      *tw = ww;
    }
  }
  if (best >= 1e30) return false;
  *cfg = c;
  return true;
}

template <int WGM, int WGN, int TM, int TN, int CK, int PMAX, bool RES, int SM>
static void launch_res_act(const ConvParams & p, int cfg, hipStream_t s)
{
  constexpr int BN = WGN * TN * 32;
  dim3 grid((unsigned)res_grid_x(p, cfg), (unsigned)((p.Cout + BN - 1) / BN), 1), block(64 * WGM * WGN);
  switch (p.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3s1_res_kernel<WGM, WGN, TM, TN, CK, PMAX, kActSiLU, RES, SM>), grid, block, 0, s, p); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3s1_res_kernel<WGM, WGN, TM, TN, CK, PMAX, kActReLU, RES, SM>), grid, block, 0, s, p); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3s1_res_kernel<WGM, WGN, TM, TN, CK, PMAX, kActHSwish, RES, SM>), grid, block, 0, s, p); break;
  default: hipLaunchKernelGGL((conv3x3s1_res_kernel<WGM, WGN, TM, TN, CK, PMAX, kActNone, RES, SM>), grid, block, 0, s, p); break;
  }
}

// residual adds need Cout % 4 == 0 (res_views_ok); the store width follows res_store_mode
template <int WGM, int WGN, int TM, int TN, int CK, int PMAX>
static void launch_res_cfg(const ConvParams & p, int cfg, hipStream_t s)
{
  const int sm = res_store_mode(p);
  if (p.r.ptr) {
    if (sm == 2) launch_res_act<WGM, WGN, TM, TN, CK, PMAX, true, 2>(p, cfg, s);
    else launch_res_act<WGM, WGN, TM, TN, CK, PMAX, true, 1>(p, cfg, s);
  } else if (sm == 2) {
    launch_res_act<WGM, WGN, TM, TN, CK, PMAX, false, 2>(p, cfg, s);
  } else if (sm == 1) {
    launch_res_act<WGM, WGN, TM, TN, CK, PMAX, false, 1>(p, cfg, s);
  } else {
    launch_res_act<WGM, WGN, TM, TN, CK, PMAX, false, 0>(p, cfg, s);
  }
}

template <bool RES, int SM>
static void launch_pp_act(const ConvParams & p, hipStream_t s)
{
  constexpr int NGRP = kPpGroups;
  dim3 grid((unsigned)res_grid_x(p, 3), (unsigned)((p.Cout + 63) / 64), 1), block(256 * NGRP);
  switch (p.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3s1_pp_kernel<NGRP, kActSiLU, RES, SM>), grid, block, 0, s, p); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3s1_pp_kernel<NGRP, kActReLU, RES, SM>), grid, block, 0, s, p); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3s1_pp_kernel<NGRP, kActHSwish, RES, SM>), grid, block, 0, s, p); break;
  default: hipLaunchKernelGGL((conv3x3s1_pp_kernel<NGRP, kActNone, RES, SM>), grid, block, 0, s, p); break;
  }
}

static void launch_pp(const ConvParams & p, hipStream_t s)
{
  const int sm = res_store_mode(p);
  if (p.r.ptr) {
    if (sm == 2) launch_pp_act<true, 2>(p, s);
    else launch_pp_act<true, 1>(p, s);
  } else if (sm == 2) {
    launch_pp_act<false, 2>(p, s);
  } else if (sm == 1) {
    launch_pp_act<false, 1>(p, s);
  } else {
    launch_pp_act<false, 0>(p, s);
  }
}

void launch_conv_res(const ConvParams & p, hipStream_t s)
{
  if (p.xg && p.res != 4) throw std::runtime_error("grouped resident-weight conv outside the ping-pong kernel");
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_res(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  const int cfg = p.res - 1;
  if (cfg == 0) {
    if (p.ck == 32) launch_res_cfg<4, 2, 2, 1, 32, kResP0>(p, cfg, s);
    else launch_res_cfg<4, 2, 2, 1, 64, kResP0>(p, cfg, s);
  } else if (cfg == 1) {
    launch_res_cfg<8, 1, 2, 1, 32, kResP1>(p, cfg, s);
  } else if (cfg == 3) {
    launch_pp(p, s);
  } else {
    launch_res_cfg<8, 1, 1, 1, 64, kResP2>(p, cfg, s);
  }
}

}  // namespace ivh
