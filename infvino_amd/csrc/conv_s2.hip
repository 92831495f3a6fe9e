// 3x3 stride-2 pad-1 convolution of few channels (Cin <= 16, Cout <= 64) on gfx950 fp16 MFMA.
//
// Replaces, for the strided downsampling convs of small width (the YOLO 16->32), the
// reference's conv3x3_ov / conv3x3_f16 with stride 2 (kernels/conv_ov.cl:133-297,
// conv.cl:150-414; dispatch src/PlanModel.cpp:3688-3933):
//   y[co][p] = act(sum_{tap,ci} W[co][ci][tap] x[ci][2p + tap - 1] + b[co]) (+ r[co][p]).
//
// These layers are HBM bound (48 FLOP per byte), and gathering the nine taps of every
// pixel with 16-byte loads (the implicit GEMM's im2col) costs more in L1 / address traffic
// than the HBM stream itself.  Here a work-group owns a TH x TW output tile of one image,
// loads its (2TH+1) x (2TW+1) x CK input patch into LDS once -- whole pixel rows, every input
// pixel of the tile read once -- and each wave reads its nine taps' MFMA pixel fragments from
// the patch.  The work-group's whole weight block (BN x 9 CK, a few KB that every
// work-group reads from L2) is loaded once beside the patch and shared by the four waves, so
// the K loop has no stage and no barrier: the only barriers are "patch and weights in LDS"
// and "patch consumed" (the epilogue then stages the output tile in the patch's LDS).
// Weights use the implicit-GEMM packing fp16 [Cout_pad128][kpad], k = tap * CK + ci.
#include <algorithm>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef unsigned u2q __attribute__((ext_vector_type(2)));
typedef unsigned u4q __attribute__((ext_vector_type(4)));
}  // namespace

template <int CK, int WGM, int WGN, int TN, int PMAX>
__global__ void __launch_bounds__(256) conv3x3s2_kernel(const ConvParams p)
{
  using F = Mf<32>;
  using T = TileShape<32, WGM, WGN, 1, TN>;
  typedef F::acc_t acc_t;
  constexpr int BN = T::BN;
  constexpr int CKP = CK + 8;       // patch pixel pitch (halves): stride-2 fragment reads conflict free
  constexpr int CQ = CK / 8;        // 16-byte pieces per pixel
  constexpr int NJ = CK / 16;       // MFMA K slices per tap
  constexpr int KW = 9 * CK;        // weights per output channel
  constexpr int LDW = KW + 8;       // weight row pitch (halves): fragment reads conflict free
  constexpr int WQ = KW / 8;        // 16-byte pieces per weight row
  constexpr int P_IT = (PMAX * CQ + 255) / 256;
  constexpr int W_IT = (BN * WQ + 255) / 256;
  constexpr int L_PATCH = PMAX * CKP;
  constexpr int L_FRONT = L_PATCH > T::EPI ? L_PATCH : T::EPI;  // patch, then the epilogue tile
  __shared__ __attribute__((aligned(16))) _Float16 lds[L_FRONT + BN * LDW];
  _Float16 * const Ws = lds + L_FRONT;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int TH = p.th, TW = p.tw, PW = 2 * TW + 1, PP = (2 * TH + 1) * PW;
  const int tiles_x = (p.Wo + TW - 1) / TW, tiles_img = tiles_x * ((p.Ho + TH - 1) / TH);
  // XCD-aware order: each XCD owns a contiguous range of tiles (neighbours share patch rows)
  const int lin = xcd_tile(blockIdx.x, gridDim.x);
  const int img = lin / tiles_img, tr = lin - img * tiles_img;
  const int oy0 = (tr / tiles_x) * TH, ox0 = (tr % tiles_x) * TW;

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w), (short)0, BN * p.kpad * 2, kBufDword3);

  // the work-group's weight block [BN][9 CK], one 16-byte piece per slot, loaded once and
  // shared by the four waves
  h8 rw[W_IT];
#pragma unroll
  for (int i = 0; i < W_IT; ++i) {
    const int e = tid + i * 256, r = e / WQ;
    rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
        wr, r < BN ? (unsigned)((r * p.kpad + (e - r * WQ) * 8) * 2) : kBufOOB, 0, 0));
  }
  // patch: element e = tid + 256 i -> patch pixel e / CQ, piece e % CQ (= tid % CQ);
  // pixels outside the image load zeros (offset past the buffer range)
  const int q8 = (tid % CQ) * 8;
  const float inv_pw = __builtin_amdgcn_rcpf((float)PW);
  h8 rp[P_IT];
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int pp = (tid + i * 256) / CQ;
    unsigned off = kBufOOB;
    if (pp < PP) {
      const int py = idiv_small(pp, PW, inv_pw), px = pp - py * PW;
      const int iy = 2 * oy0 - 1 + py, ix = 2 * ox0 - 1 + px;
      if ((unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W)
        off = (unsigned)((img * (int)p.x.img + (iy * p.W + ix) * p.x.cs + q8) * 2);
    }
    rp[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < W_IT; ++i) {
    const int e = tid + i * 256, r = e / WQ;
    if (r < BN) *reinterpret_cast<h8 *>(Ws + r * LDW + (e - r * WQ) * 8) = rw[i];
  }
  // channels >= Cin of a ragged pixel are zeroed bitwise (their bits never reach the MFMAs)
  u16x8 keep;
#pragma unroll
  for (int k = 0; k < 8; ++k) keep[k] = q8 + k < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
  const bool ragged = p.Cin < CK;
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int e = tid + i * 256;
    if (e < PP * CQ) {
      h8 v = rp[i];
      if (ragged) v = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, v) & keep);
      *reinterpret_cast<h8 *>(lds + (e / CQ) * CKP + q8) = v;
    }
  }
  __syncthreads();

  // pixel fragment of this lane: output slot pl of the tile (slots past TH x TW read pixel
  // 0 and are discarded by the epilogue); weight fragment: row (lane & 31) of each block
  const int kq = F::kq(lane);
  int pl = wm * 32 + (lane & 31);
  if (pl >= TH * TW) pl = 0;
  const int ty = pl / TW, tx = pl - (pl / TW) * TW;
  const int bbase = (2 * ty * PW + 2 * tx) * CKP + kq;
  const int abase = (wn * TN * 32 + (lane & 31)) * LDW + kq;
  acc_t acc[TN][1];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int v = 0; v < F::NV; ++v) acc[tn][0][v] = 0.0f;
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const h8 fb = *reinterpret_cast<const h8 *>(lds + bbase + ((t / 3) * PW + t % 3) * CKP + j * 16);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const h8 fa = *reinterpret_cast<const h8 *>(Ws + abase + tn * 32 * LDW + t * CK + j * 16);
        acc[tn][0] = F::mma(fa, fb, acc[tn][0]);
      }
    }
  __syncthreads();  // every wave is done with the patch: the epilogue reuses its LDS

  tile_epilogue<32, WGM, WGN, 1, TN>(acc, p, lds, 0, 0, [&](int q, int & b, int & hw) {
    if (q >= TH * TW) return false;
    const int qy = q / TW, qx = q - qy * TW;
    const int oy = oy0 + qy, ox = ox0 + qx;
    if (oy >= p.Ho || ox >= p.Wo) return false;
    b = img;
    hw = oy * p.Wo + ox;
    return true;
  });
}

// ---------------------------------------------------------------- persistent kernel
//
// 3x3 stride-2 pad-1 convs of CK = 16 or 32 input channels (Cin <= CK), Cout <= 32 CB: the
// work-group's weights [32 CB][9 CK] stay in LDS for the whole launch, and the grid is
// persistent over TH x 16 output tiles (contiguous tile ranges, XCD-aware), the next
// tile's input patch in flight in registers while the current one is computed.
//
// The (2TH+1) x 33 input patch sits in LDS de-interleaved by column parity: every patch row
// holds its 17 even columns, then its 16 odd ones, so the three horizontal taps of a stride-2
// output row read consecutive pixels (dx = 0: even column tx, 1: odd column tx, 2: even
// column tx + 1).  gfx950 serves a ds_read_b128 in 16-lane groups (per half-wave, the quads
// of even and of odd bit parity) over 64 four-byte banks: a fragment of 32 pixels = two
// 16-wide output rows is conflict free when the pixel pitch is an odd number of 16-byte
// slots (48 bytes with 16 channels, 80 with 32) and two patch rows span a multiple of 256
// bytes (row pitch a multiple of 128 bytes), so that both output rows fall on one bank
// pattern.
//
// Waves: 4, each one 32-pixel block (two output rows) x one 32-channel block, K = 9 CK in
// slices of 16 on one accumulator (v_mfma_f32_32x32x16_f16).  With CB = 1 the tile is 8 x
// 16 (four pixel blocks), with CB = 2 it is 4 x 16.  Epilogue in registers: bias + act in
// fp32, one fp16 rounding, 8 consecutive channels per lane after a permlane32 swap, 16-byte
// stores (NHWC output, Cout padded to 8 by the view).
namespace {
template <int CK> struct S2P {
  static constexpr int CKP = CK + 8;                     // pixel pitch (halves): odd 16-byte slots
  static constexpr int ODD = 17 * CKP;                   // odd-column plane of a patch row
  static constexpr int RH = (33 * CKP + 63) / 64 * 64;   // row pitch (halves): multiple of 128 bytes
  static constexpr int LDW = 9 * CK + 8;                 // weight row pitch (halves): odd slots
};
}  // namespace

template <int CK, int CB, int PB, int ACT>
__global__ void __launch_bounds__(64 * PB * CB, CK == 16 ? 4 : 2) conv3x3s2_pk_kernel(const ConvParams p)
{
  using F = Mf<32>;
  using L = S2P<CK>;
  typedef F::acc_t acc_t;
  constexpr int NT = 64 * PB * CB;      // threads: a wave per (pixel block, channel block)
  constexpr int TH = 2 * PB, TW = 16;   // output tile
  constexpr int PR = 2 * TH + 1;        // patch rows
  constexpr int CQ = CK / 8;            // 16-byte pieces per pixel
  constexpr int NPC = PR * 33 * CQ;     // patch pieces
  constexpr int P_IT = (NPC + NT - 1) / NT;
  constexpr int BN = 32 * CB;
  constexpr int WQ = 9 * CK / 8;        // 16-byte pieces per weight row
  constexpr int W_IT = (BN * WQ + NT - 1) / NT;
  constexpr int NSL = 9 * CK / 16;      // K slices
  __shared__ __attribute__((aligned(16))) _Float16 Ws[BN * L::LDW];
  __shared__ __attribute__((aligned(16))) _Float16 Ps[PR * L::RH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pb = wave % PB, cb = wave / PB;
  const int co0 = blockIdx.y * BN;  // this work-group's output channels co0 .. co0 + BN - 1
  const int tiles_x = (p.Wo + TW - 1) / TW, tiles_y = (p.Ho + TH - 1) / TH;
  const int tiles_img = tiles_x * tiles_y, ntiles = p.batch * tiles_img;
  const int G = gridDim.x, r = xcd_tile(blockIdx.x, G);
  const int t_lo = (int)((long)r * ntiles / G), t_hi = (int)((long)(r + 1) * ntiles / G);
  const int ntl = t_hi - t_lo;
  if (ntl <= 0) return;

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.Ho * p.Wo - 1) * p.y.cs + (p.Cout + 7) / 8 * 8;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);

  // weights [BN][9 CK] (implicit-GEMM packing, k = tap * CK + ci), once per launch
  {
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(p.w + (long)co0 * p.kpad), (short)0, BN * p.kpad * 2, kBufDword3);
    h8 rw[W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, row = e / WQ;
      rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
          wr, row < BN ? (unsigned)((row * p.kpad + (e - row * WQ) * 8) * 2) : kBufOOB, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, row = e / WQ;
      if (row < BN) *reinterpret_cast<h8 *>(Ws + row * L::LDW + (e - row * WQ) * 8) = rw[i];
    }
  }
  // bias of the lane's 16 channel rows in its block
  float bv[16];
#pragma unroll
  for (int v4 = 0; v4 < 16; v4 += 4) {
    float4 b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (p.bias) b4 = *reinterpret_cast<const float4 *>(p.bias + co0 + cb * 32 + F::row(lane, v4));
    bv[v4] = b4.x;
    bv[v4 + 1] = b4.y;
    bv[v4 + 2] = b4.z;
    bv[v4 + 3] = b4.w;
  }

  // patch pieces of this thread: e = tid + NT i -> pixel e / CQ = (row py, column px) of
  // the (2TH+1) x 33 patch, piece e % CQ; packed as py << 8 | px (0xffff: none)
  const int q8 = (tid % CQ) * 8;
  int pyx[P_IT];
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int pp = (tid + i * NT) / CQ, py = pp / 33;
    pyx[i] = pp < PR * 33 ? (py << 8) | (pp - py * 33) : 0xffff;
  }
  // channels >= Cin of a ragged pixel are zeroed bitwise (their bits never reach the MFMAs)
  u16x8 keep;
#pragma unroll
  for (int k = 0; k < 8; ++k) keep[k] = q8 + k < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
  const bool ragged = p.Cin < CK;

  auto origin = [&](int t, int & b, int & oy0, int & ox0) __attribute__((always_inline)) {
    b = t / tiles_img;
    const int tr = t - b * tiles_img, ty = tr / tiles_x;
    oy0 = ty * TH;
    ox0 = (tr - ty * tiles_x) * TW;
  };
  const int xrow = p.W * p.x.cs;
  auto load_patch = [&](int t, h8 (&rp)[P_IT]) __attribute__((always_inline)) {
    int b, oy0, ox0;
    origin(t, b, oy0, ox0);
    const int iy0 = 2 * oy0 - 1, ix0 = 2 * ox0 - 1;
    const int base = b * (int)p.x.img + iy0 * xrow + ix0 * p.x.cs + q8;
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      const int py = pyx[i] >> 8, px = pyx[i] & 0xff;
      const bool ok = pyx[i] != 0xffff && (unsigned)(iy0 + py) < (unsigned)p.H && (unsigned)(ix0 + px) < (unsigned)p.W;
      const int off = base + py * xrow + px * p.x.cs;
      rp[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? (unsigned)off * 2u : kBufOOB, 0, 0));
    }
  };
  auto store_patch = [&](const h8 (&rp)[P_IT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i)
      if (pyx[i] != 0xffff) {
        const int py = pyx[i] >> 8, px = pyx[i] & 0xff;
        h8 v = rp[i];
        if (ragged) v = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, v) & keep);
        *reinterpret_cast<h8 *>(Ps + py * L::RH + ((px & 1) ? L::ODD : 0) + (px >> 1) * L::CKP + q8) = v;
      }
  };

  // fragments: B = pixel (lane & 31) of block pb = output row 2 pb + (lane & 31) / 16, column
  // (lane & 15); A = weight row cb * 32 + (lane & 31)
  const int kq = F::kq(lane);
  const int bl = (2 * (2 * pb + ((lane >> 4) & 1))) * L::RH + (lane & 15) * L::CKP + kq;
  const int al = (cb * 32 + (lane & 31)) * L::LDW + kq;

  h8 rp[P_IT];
  load_patch(t_lo, rp);
  __syncthreads();  // weights in LDS
  store_patch(rp);
  load_patch(t_lo + (ntl > 1 ? 1 : 0), rp);
  __syncthreads();  // first patch in LDS

  // fragments of K slice sl (tap sl / (CK / 16), channels 16 (sl % (CK / 16)) ..)
  auto frag = [&](int sl, h8 & fa, h8 & fb) __attribute__((always_inline)) {
    const int tap = sl / (CK / 16), j = sl % (CK / 16);
    const int dy = tap / 3, dx = tap % 3;
    const int boff = dy * L::RH + (dx == 1 ? L::ODD : (dx == 2 ? L::CKP : 0)) + 16 * j;
    fa = *reinterpret_cast<const h8 *>(Ws + al + tap * CK + 16 * j);
    fb = *reinterpret_cast<const h8 *>(Ps + bl + boff);
  };
  constexpr int D = CK == 16 ? 2 : 4;  // K slices whose fragments are in flight

  for (int i = 0; i < ntl; ++i) {
    // two accumulators (even and odd K slices): independent MFMA chains, summed at the end
    acc_t acc[2];
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][v] = acc[1][v] = 0.0f;
    h8 fa[D], fb[D];
#pragma unroll
    for (int sl = 0; sl < D && sl < NSL; ++sl) frag(sl, fa[sl], fb[sl]);
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      const h8 a0 = fa[sl % D], b0 = fb[sl % D];
      if (sl + D < NSL) frag(sl + D, fa[sl % D], fb[sl % D]);
      acc[sl & 1] = F::mma(a0, b0, acc[sl & 1]);
      __builtin_amdgcn_sched_barrier(0);  // keep the reads D slices ahead of their MFMAs
    }
    acc_t acc_s;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc_s[v] = acc[0][v] + acc[1][v];
    __syncthreads();  // every wave is done with the patch
    if (i + 1 < ntl) {
      store_patch(rp);  // tile i + 1
      load_patch(t_lo + (i + 2 < ntl ? i + 2 : i + 1), rp);
    }
    // epilogue of tile i: output pixel of the lane, 8-channel stores after the swap
    {
      int b, oy0, ox0;
      origin(t_lo + i, b, oy0, ox0);
      const int oy = oy0 + 2 * pb + ((lane >> 4) & 1), ox = ox0 + (lane & 15);
      const bool ok = oy < p.Ho && ox < p.Wo;
      const unsigned yo = ok ? ((unsigned)b * (unsigned)p.y.img + (unsigned)(oy * p.Wo + ox) * (unsigned)p.y.cs) * 2u : kBufOOB;
      auto vals = [&](int v4) __attribute__((always_inline)) {
        float o4[4] = {act_fast<ACT>(acc_s[v4] + bv[v4]), act_fast<ACT>(acc_s[v4 + 1] + bv[v4 + 1]),
                       act_fast<ACT>(acc_s[v4 + 2] + bv[v4 + 2]), act_fast<ACT>(acc_s[v4 + 3] + bv[v4 + 3])};
        h4 hv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __asm__("" : "+v"(o4[q]));  // fp32 result, then one fp16 rounding
          hv[q] = (_Float16)o4[q];
        }
        return hv;
      };
#pragma unroll
      for (int v4 = 0; v4 < 16; v4 += 8) {
        // runs v4 (channels c..c+3 / c+4..c+7 on lanes < 32 / >= 32) and v4 + 4 (c+8..c+11 /
        // c+12..c+15): swapped so every lane holds 8 consecutive channels
        const u2q lo = __builtin_bit_cast(u2q, vals(v4));
        const u2q hi = __builtin_bit_cast(u2q, vals(v4 + 4));
        const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], hi[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], hi[1], false, false);
        const u4q q = {s0[0], s1[0], s0[1], s1[1]};
        const int c = co0 + cb * 32 + F::row(lane, v4) - 4 * (lane >> 5) + 8 * (lane >> 5);
        if (c < p.Cout)
          __builtin_amdgcn_raw_buffer_store_b128(q, yr, yo == kBufOOB ? kBufOOB : yo + (unsigned)c * 2u, 0, 0);
      }
    }
    __syncthreads();  // patch of tile i + 1 in LDS
  }
}

// ---------------------------------------------------------------- host side

namespace {
struct S2Cfg {
  int ck, bm, bn, pmax;
};
// 0: 16 channels in, <= 32 out, 128-pixel tiles; 1: 16 in, <= 64 out, 64-pixel tiles.
// (With 32 channels in, the patch plus the 64 x 288 weight block leave two work-groups per
// CU, and the implicit GEMM is faster: measured 66 vs 47 us for 32->64 at 160x160, batch 64.)
constexpr S2Cfg kS2Cfg[2] = {{16, 128, 32, 600}, {16, 64, 64, 400}};
}  // namespace

int s2_patch(int th, int tw) { return (2 * th + 1) * (2 * tw + 1); }
int s2_cfg_bm(int cfg) { return kS2Cfg[cfg].bm; }
int s2_cfg_bn(int cfg) { return kS2Cfg[cfg].bn; }
int s2_cfg_ck(int cfg) { return kS2Cfg[cfg].ck; }
int s2_cfg_pmax(int cfg) { return kS2Cfg[cfg].pmax; }

// Config and output tile for a 3x3 stride-2 pad-1 conv; false: not this kernel's shape.
// The tile width is the one of 8 / 16 / 32 / 64 that wastes the fewest pixel slots on the
// ragged right and bottom edges (ties: 16, whose patch rows are 33 pixels).
bool s2_plan(int cin, int cout, int Ho, int Wo, int * cfg, int * th, int * tw)
{
  const int cin8 = (cin + 7) / 8 * 8;
  if (cin8 != 16 || cout > 64 || Ho < 1 || Wo < 1) return false;
  const int c = cout <= 32 ? 0 : 1;
  long best = -1;
  for (int w : {16, 8, 32, 64}) {
    const int h = kS2Cfg[c].bm / w;
    if (h < 1 || s2_patch(h, w) > kS2Cfg[c].pmax) continue;
    const long slots = (long)((Ho + h - 1) / h) * h * ((Wo + w - 1) / w) * w;
    if (best < 0 || slots < best) {
      best = slots;
      *th = h;
      *tw = w;
    }
  }
  if (best < 0) return false;
  *cfg = c;
  return true;
}

long s2_grid(const ConvParams & p)
{
  return (long)p.batch * ((p.Ho + p.th - 1) / p.th) * ((p.Wo + p.tw - 1) / p.tw);
}

// ---------------------------------------------------------------- persistent kernel, host side

namespace {
constexpr int kS2PkCUs = 256;
}  // namespace

// persistent configs: 2: 16 channels in, one 32-channel block, 8 x 16 tiles; 3: 16 in, two
// blocks, 4 x 16; 4, 5: the same with 32 channels in; 6: 64 channels in, two blocks, 8 x 16
// tiles, eight waves (Cout beyond 64 in further 64-channel blocks on grid.y)
int s2pk_ck(int cfg) { return cfg == 2 || cfg == 3 ? 16 : (cfg == 6 ? 64 : 32); }
int s2pk_cb(int cfg) { return cfg == 2 || cfg == 4 ? 1 : 2; }
int s2pk_pb(int cfg) { return cfg == 6 ? 4 : 4 / s2pk_cb(cfg); }
int s2pk_th(int cfg) { return 2 * s2pk_pb(cfg); }

bool s2pk_views_ok(const ConvParams & p)
{
  const View & y = p.y;
  if (y.layout != kNHWC || (y.cs % 8) || (y.img % 8) || (reinterpret_cast<uintptr_t>(y.ptr) % 16)) return false;
  if (p.Cout % 8 && p.ypad < 8 - p.Cout % 8) return false;
  const long ylast = (long)(p.batch - 1) * y.img + ((long)p.Ho * p.Wo - 1) * y.cs + (p.Cout + 7) / 8 * 8;
  const long xlast = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  return !p.r.ptr && ylast * 2 < (1L << 31) && xlast * 2 < (1L << 31) && (long)p.W * p.x.cs < (1L << 23) &&
         p.W < 65536 && p.H < 65536;
}

long s2pk_tiles(const ConvParams & p)
{
  const int th = s2pk_th(p.s2 - 1);
  return (long)p.batch * ((p.Ho + th - 1) / th) * ((p.Wo + 15) / 16);
}

template <int CK, int CB, int PB>
static void launch_s2pk_act(const ConvParams & p, hipStream_t s)
{
  // work-groups per CU: 4 with 16 channels (38 KB of LDS, <= 128 VGPRs), 2 with 32 (64 KB),
  // 1 with 64 (157 KB); output-channel blocks on grid.y share the CUs
  const long per_cu = CK == 16 ? 4 : (CK == 32 ? 2 : 1);
  const int ncb = (p.Cout + 32 * CB - 1) / (32 * CB);
  const long gx = std::min<long>(s2pk_tiles(p), std::max<long>(1, per_cu * kS2PkCUs / ncb));
  const dim3 grid((unsigned)gx, (unsigned)ncb), block(64 * PB * CB);
  switch (p.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3s2_pk_kernel<CK, CB, PB, kActSiLU>), grid, block, 0, s, p); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3s2_pk_kernel<CK, CB, PB, kActReLU>), grid, block, 0, s, p); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3s2_pk_kernel<CK, CB, PB, kActHSwish>), grid, block, 0, s, p); break;
  default: hipLaunchKernelGGL((conv3x3s2_pk_kernel<CK, CB, PB, kActNone>), grid, block, 0, s, p); break;
  }
}

static void launch_conv_s2pk(const ConvParams & p, hipStream_t s)
{
  switch (p.s2 - 1) {
  case 2: launch_s2pk_act<16, 1, 4>(p, s); break;
  case 3: launch_s2pk_act<16, 2, 2>(p, s); break;
  case 4: launch_s2pk_act<32, 1, 4>(p, s); break;
  case 5: launch_s2pk_act<32, 2, 2>(p, s); break;
  default: launch_s2pk_act<64, 2, 4>(p, s); break;
  }
}

void launch_conv_s2(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_s2(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  if (p.s2 > 2) {
    launch_conv_s2pk(p, s);
    return;
  }
  const dim3 grid((unsigned)s2_grid(p));
  switch (p.s2 - 1) {
  case 0: hipLaunchKernelGGL((conv3x3s2_kernel<16, 4, 1, 1, 600>), grid, dim3(256), 0, s, p); break;
  default: hipLaunchKernelGGL((conv3x3s2_kernel<16, 2, 2, 1, 400>), grid, dim3(256), 0, s, p); break;
  }
}

}  // namespace ivh
