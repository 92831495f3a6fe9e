// 3x3 stride-1 pad-1 convolution for wide layers (Cin >= 64) on gfx950 fp16 MFMA: one
// persistent work-group per CU that owns an exact share of the output pixels.
//
// Replaces, for channels-last layers with Cin % 32 == 0 and Cin >= 64, the reference's 3x3
// kernels conv3x3_ov (kernels/conv_ov.cl:133-297), conv3x3_blk (conv_blk.cl:118-296) and
// conv3x3_f16 (conv.cl:150-414):
//   y[co][p] = act(sum_{tap,ci} W[co][ci][tap] x[ci][p + tap] + b[co]) (+ r[co][p]).
//
// The batch is one tall image (image b at rows [b*(H+1), b*(H+1)+H), a zero separator row
// after each image) whose output pixels, row-major, are numbered as slots; slots form
// 32-slot blocks (one MFMA column block each).  Work-group (range, channel group) computes
// the blocks [blo, bhi) of its range -- an equal share of all blocks, so a layer whose pixel
// count is not a multiple of a tile still fills every CU -- for the BN output channels of
// its group.  The range is walked in passes of PB = WGM * TM blocks; a pass is a stream of
// 16-channel input chunks, and a chunk is one LDS stage holding
//   * the chunk's weights for all nine taps (9 x BN x 16 fp16, each 32 x 16 MFMA A fragment
//     as 1 KB in lane order: conflict-free reads), and
//   * the pass's input patch for the chunk: the rows of the tall image the pass's slots
//     touch plus one above and below, each row W + 2 pixels (zero columns at both ends), a
//     pixel three 16-byte slots (two 8-channel pieces and a pad slot); the row pitch is
//     3 W + 16 slots, so modulo 16 slots every pixel sits where it would if rows were laid
//     out without their two zero columns: the 32 lanes of a B fragment (32 consecutive
//     output slots, also across a row wrap) hit 16 distinct 16-byte bank groups.
// Both parts are copied by buffer loads with the LDS flag (no VGPR round trip) into the
// stage the previous chunk freed, while the current chunk's 9 x TN x TM MFMAs run on the
// other stage: one barrier per chunk.  Pixels outside the image, separator rows, pad slots
// and channel pieces at or past Cin read from past the buffer range, which the hardware
// answers with zeros.  After a pass's last chunk the epilogue (bias, activation in fp32,
// one fp16 rounding, residual, 8-channel stores through v_permlane32_swap) runs from the
// accumulators while the next pass's first chunk is in flight.
// Wave layout: WGN waves split the BN channels (TN 32-channel blocks each), WGM waves the
// pass's blocks (TM each); the accumulators (TN x TM x 16 fp32 per lane) live in AGPRs with
// one wave per SIMD.
#include <algorithm>
#include <type_traits>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned u2w __attribute__((ext_vector_type(2)));
typedef unsigned u4w __attribute__((ext_vector_type(4)));

// 16 bytes per lane from byte offset voff + soff (soff wave-uniform) into 64 consecutive
// 16-byte LDS slots from lds
__device__ __forceinline__ void dma16w(__amdgpu_buffer_rsrc_t r, _Float16 * lds, unsigned voff, int soff)
{
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, (int)voff, soff, 0, 0);
}
}  // namespace

// Host-resolved geometry of one launch.
struct WideGeom {
  int rp;       // patch row pitch in 16-byte slots (3 W + 16)
  int nslot;    // output slots of the tall image (rows * W)
  int nblk;     // 32-slot blocks
  int gx;       // pixel ranges
  int ncg;      // channel groups of BN channels
  int nchunks;  // 16-channel input chunks
};

// Patch slots of an LDS stage (a multiple of 256: whole DMA instructions of every wave).
template <int BN> struct WideLds {
  static constexpr int PSL = BN == 128 ? 2048 : 3840;
};

template <int TM, int TN, int WGM, int WGN, int ACT, bool RES>
__global__ void __launch_bounds__(256, 1) conv3x3_wide_kernel(const ConvParams p, const WideGeom g)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  static_assert(WGM * WGN == 4, "four waves");
  constexpr int BN = WGN * TN * 32;
  constexpr int NCB = BN / 32;               // 32-channel blocks of the group
  constexpr int PB = WGM * TM;               // blocks per pass
  constexpr int PSL = WideLds<BN>::PSL;
  constexpr int NWF = 9 * NCB;               // weight fragments (DMA instructions) per chunk
  constexpr int NWQ = (NWF + 3) / 4;         // ... per wave
  constexpr int NPQ = PSL / 256;             // patch DMA instructions per wave, at most
  __shared__ __attribute__((aligned(16))) _Float16 W0[NWF * 512];
  __shared__ __attribute__((aligned(16))) _Float16 W1[NWF * 512];
  __shared__ __attribute__((aligned(16))) _Float16 P0[PSL * 8];
  __shared__ __attribute__((aligned(16))) _Float16 P1[PSL * 8];
  __shared__ __attribute__((aligned(16))) float BIAS[BN];

  // the wave index as a scalar: copy bookkeeping and LDS destinations stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WGM, wn = wave / WGM;
  const int W = p.W, RP = g.rp, Hs = p.H + 1;
  const float inv_w = __builtin_amdgcn_rcpf((float)W), inv_hs = __builtin_amdgcn_rcpf((float)Hs);
  const float inv_rp = __builtin_amdgcn_rcpf((float)RP);

  // this work-group's pixel range and channel group (XCD-aware: the channel groups of a
  // range, and neighbouring ranges, which share input rows, run on one XCD)
  const int id = xcd_tile(blockIdx.x, gridDim.x);
  const int xr = id / g.ncg, cg = id - xr * g.ncg;
  const int blo = (int)((long)xr * g.nblk / g.gx), bhi = (int)((long)(xr + 1) * g.nblk / g.gx);
  if (bhi <= blo) return;
  const int npass = (bhi - blo + PB - 1) / PB;
  const int n0 = cg * BN;

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr_ = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w), (short)0, g.ncg * g.nchunks * NWF * 1024, kBufDword3);

  // ---- weight copies: the packing holds each chunk's fragments in LDS order (fragment
  // f = tap * NCB + channel block, 1 KB each, lane order), so copy f = u * 4 + wave reads
  // 1 KB from (group, chunk) block offset f * 1024: one contiguous range per chunk
  auto copy_w = [&](_Float16 * buf, int c16) __attribute__((always_inline)) {
    const int cs = (cg * g.nchunks + c16) * NWF * 1024;
#pragma unroll
    for (int u = 0; u < NWQ; ++u)
      if (u * 4 + wave < NWF) dma16w(wr, buf + (u * 4 + wave) * 512, (unsigned)((u * 4 + wave) * 1024 + lane * 16), cs);
  };

  // ---- patch copies: instruction j = u * 4 + wave covers slots 64 j .. 64 j + 63; a lane's
  // slot is (row pr, pixel px, piece pc); goff: the byte offset of its piece for chunk 0 in
  // the current pass (kBufOOB: a slot no input fills; Cin % 16 == 0, so every piece of a
  // pixel is inside the channels)
  unsigned goff[NPQ];
  // slot -> (tall row, column)
  auto slot_rc = [&](int f, int & r, int & c) __attribute__((always_inline)) {
    r = idiv_small(f, W, inv_w);
    c = f - r * W;
  };
  // goff for pass ps; returns the pass's patch DMA instruction count
  auto pass_patch = [&](int ps) __attribute__((always_inline)) {
    const int pb = blo + ps * PB, pe = min(pb + PB, bhi);
    const int r0 = idiv_small(pb * 32, W, inv_w);
    const int r1 = idiv_small(min(pe * 32, g.nslot) - 1, W, inv_w);
    const int nrows = r1 - r0 + 3;
#pragma unroll
    for (int u = 0; u < NPQ; ++u) {
      // recomputed per pass rather than hoisted and kept live for the whole kernel
      int e = (u * 4 + wave) * 64 + lane;
      __asm__ volatile("" : "+v"(e));
      const int pr = idiv_small(e, RP, inv_rp), rem = e - pr * RP;
      const int px = (int)(((unsigned)rem * 43691u) >> 17), pc = rem - px * 3;  // rem / 3, exact below 98304
      const int tr = r0 - 1 + pr;
      const int b = idiv_small(max(tr, 0), Hs, inv_hs), yy = tr - b * Hs;
      const bool ok = (tr >= 0) & (pr < nrows) & (px >= 1) & (px <= W) & (pc < 2) & (yy < p.H) & (b < p.batch);
      goff[u] = ok ? (unsigned)(b * (int)p.x.img + (yy * W + px - 1) * p.x.cs + pc * 8) * 2u : kBufOOB;
    }
    return (nrows * RP + 63) >> 6;
  };
  auto copy_p = [&](_Float16 * buf, int c16, int npi) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NPQ; ++u)
      if (u * 4 + wave < npi) dma16w(xr_, buf + (u * 4 + wave) * 512, goff[u], c16 * 32);
  };

  // ---- B fragment addresses of pass ps (halves): lane -> slot of its block's column, its
  // K piece; slots past the range or the image read a valid patch pixel and are not stored
  int bl[TM];
  auto pass_frags = [&](int ps) __attribute__((always_inline)) {
    const int pb = blo + ps * PB, pe = min(pb + PB, bhi);
    const int r0 = idiv_small(pb * 32, W, inv_w);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int blk = pb + wm * TM + tm;
      int f = blk * 32 + (lane & 31);
      if (blk >= pe || f >= g.nslot) f = pb * 32;
      int r, c;
      slot_rc(f, r, c);
      bl[tm] = ((r - r0) * RP + c * 3 + (lane >> 5)) * 8;
    }
  };

  // ---- epilogue: outputs straight from the accumulators, 8 channels (16 bytes) a store
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.H * p.W - 1) * p.y.cs + ((p.Cout + 7) & ~7);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);
  const long r_last = RES ? (long)(p.batch - 1) * p.r.img + ((long)p.H * p.W - 1) * p.r.cs + p.Cout : 0;
  const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(RES ? p.r.ptr : p.y.ptr, (short)0,
                                                                        (int)(r_last * 2), kBufDword3);
  const int cl0 = wn * TN * 32 + 4 * (lane >> 5);  // lane's first channel of a block, within BN
  auto coff = [&](unsigned base, int cl) { return n0 + cl < p.Cout ? base + (unsigned)cl * 2u : kBufOOB; };
  // one epilogue step of pass ps: block tm, channel block tn, half e -- the lane's value
  // groups 2e and 2e + 1 (channels cl0 + 16 e .. + 3 and + 8 .. + 11 of the block): bias,
  // activation in fp32, one fp16 rounding, (+ residual), one 16-byte store
  auto epi_step = [&](acc_t (&acc)[TN][TM], int ps, int tm, int tn, int e) __attribute__((always_inline)) {
    const int pb = blo + ps * PB, pe = min(pb + PB, bhi);
    const int blk = pb + wm * TM + tm;
    const int f = blk * 32 + (lane & 31);
    int r, c;
    slot_rc(min(f, g.nslot - 1), r, c);
    const int b = idiv_small(r, Hs, inv_hs), yy = r - b * Hs;
    const bool ok = blk < pe && f < g.nslot && yy < p.H;
    const unsigned hw = (unsigned)(yy * W + c);
    const unsigned yo = ok ? ((unsigned)b * (unsigned)p.y.img + hw * (unsigned)p.y.cs + (unsigned)n0) * 2u : kBufOOB;
    h4 rv[2];
    if (RES) {
      const unsigned ro = ok ? ((unsigned)b * (unsigned)p.r.img + hw * (unsigned)p.r.cs + (unsigned)n0) * 2u : kBufOOB;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        rv[k] = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rres, coff(ro, tn * 32 + cl0 + 8 * (2 * e + k)), 0, 0));
    }
    auto vals = [&](int k) __attribute__((always_inline)) {
      const int q = 2 * e + k;
      const float4 b4 = *reinterpret_cast<const float4 *>(BIAS + tn * 32 + cl0 + 8 * q);
      float o[4] = {act_fast<ACT>(acc[tn][tm][4 * q + 0] + b4.x), act_fast<ACT>(acc[tn][tm][4 * q + 1] + b4.y),
                    act_fast<ACT>(acc[tn][tm][4 * q + 2] + b4.z), act_fast<ACT>(acc[tn][tm][4 * q + 3] + b4.w)};
      h4 hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __asm__("" : "+v"(o[i]));  // fp32 result, then one fp16 rounding (no fused convert)
        hv[i] = (_Float16)o[i];
      }
      if (RES) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hv[i] = (_Float16)((float)hv[i] + (float)rv[k][i]);
      }
      return hv;
    };
    // groups 2e and 2e + 1: channels c..c+3 / c+8..c+11 (lanes < 32) and c+4..c+7 /
    // c+12..c+15 (lanes >= 32) of one pixel; swapped so every lane holds 8 consecutive ones
    const u2w a = __builtin_bit_cast(u2w, vals(0));
    const u2w bq = __builtin_bit_cast(u2w, vals(1));
    const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], bq[0], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], bq[1], false, false);
    const u4w v = {s0[0], s1[0], s0[1], s1[1]};
    __builtin_amdgcn_raw_buffer_store_b128(v, yr, coff(yo, tn * 32 + cl0 + 16 * e + 4 * (lane >> 5)), 0, 0);
  };
  // a whole pass's epilogue, one step after another (scheduling barriers keep the compiler
  // from interleaving all blocks, which would hold every block's values live at once)
  auto epilogue = [&](acc_t (&acc)[TN][TM], int ps) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < TM * TN * 2; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      epi_step(acc, ps, k / (TN * 2), (k / 2) % TN, k % 2);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue: the bias into LDS, pass 0's first chunk, pass 0's fragment addresses
  for (int c = tid; c < BN; c += 256) BIAS[c] = p.bias ? p.bias[n0 + c] : 0.0f;
  int npi = pass_patch(0);
  copy_p(P0, 0, npi);
  copy_w(W0, 0);
  pass_frags(0);
  const int rp8 = RP * 8;

  // one chunk (c) of pass ps: wait for its copies, publish them, start the next chunk's
  // copies (the next pass's first one after the last chunk) into the other stage, then the
  // 9 taps' MFMAs; FIRST: the pass's first chunk, whose first MFMAs start from zero
  auto chunk = [&](auto first_t, int ps, int c, const _Float16 * WC, const _Float16 * PC, _Float16 * WN,
                   _Float16 * PN, acc_t (&acc)[TN][TM]) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_t)::value;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kVmWait0);
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's copies visible; the other stage is free
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < g.nchunks) {
      copy_p(PN, c + 1, npi);
      copy_w(WN, c + 1);
    } else if (ps + 1 < npass) {
      npi = pass_patch(ps + 1);
      copy_p(PN, 0, npi);
      copy_w(WN, 0);
    }
    // A fragments double-buffered per tap; each B fragment register is refilled with the
    // next tap's fragment right after its last MFMA of this tap, so a read has the tap's
    // remaining MFMAs plus the next tap's earlier ones (about TM MFMAs) to land, with one
    // register set instead of two.  Scheduling barriers keep this order: the compiler would
    // otherwise move each read down to its MFMA (exposing the LDS latency on every MFMA with
    // one wave per SIMD) or hoist all reads up (two live sets).
    h8 fa[2][TN], fb[TM];
    auto read_a = [&](int tap, h8 (&a)[TN]) __attribute__((always_inline)) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        a[tn] = *reinterpret_cast<const h8 *>(WC + ((tap * NCB + wn * TN + tn) * 64 + lane) * 8);
    };
    // the tap offset is materialised per tap (one add per fragment read) rather than hoisted
    // out of the loop as 9 x TM live addresses
    auto tap_off = [&](int tap) __attribute__((always_inline)) {
      int toff = (tap / 3) * rp8 + (tap % 3) * 24;
      __asm__ volatile("" : "+s"(toff));
      return toff;
    };
    read_a(0, fa[0]);
    {
      const int toff = tap_off(0);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) fb[tm] = *reinterpret_cast<const h8 *>(PC + bl[tm] + toff);
    }
    // taps and blocks as compile-time loops: every index below folds
    static_for<0, 9>([&](auto tap_c) __attribute__((always_inline)) {
      constexpr int tap = decltype(tap_c)::value;
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (tap + 1 < 9) read_a(tap + 1, fa[(tap + 1) & 1]);
      const int toff = tap + 1 < 9 ? tap_off(tap + 1) : 0;
      static_for<0, TM>([&](auto tm_c) __attribute__((always_inline)) {
        constexpr int tm = decltype(tm_c)::value;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tn][tm] = F::mma(fa[tap & 1][tn], fb[tm], FIRST && tap == 0 ? acc_t{} : acc[tn][tm]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (tap + 1 < 9) fb[tm] = *reinterpret_cast<const h8 *>(PC + bl[tm] + toff);
      });
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  using first_c = std::integral_constant<bool, true>;
  using next_c = std::integral_constant<bool, false>;
  // a pass: chunk 0 on stage 0 (an even number of chunks per pass: every pass starts there),
  // then pairs on stages 1 / 0 and the last chunk on stage 1, then the pass's epilogue
  for (int ps = 0; ps < npass; ++ps) {
    acc_t acc[TN][TM];
    chunk(first_c{}, ps, 0, W0, P0, W1, P1, acc);
    for (int c = 1; c + 1 < g.nchunks; c += 2) {
      chunk(next_c{}, ps, c, W1, P1, W0, P0, acc);
      chunk(next_c{}, ps, c + 1, W0, P0, W1, P1, acc);
    }
    chunk(next_c{}, ps, g.nchunks - 1, W1, P1, W0, P0, acc);
    epilogue(acc, ps);
    if (ps + 1 < npass) pass_frags(ps + 1);
  }
  // every copy has landed before the work-group ends
  __builtin_amdgcn_s_waitcnt(kVmWait0);
}

// ---------------------------------------------------------------- host side

namespace {
// blocks per wave and pass (accumulators: TM x 16 per lane, in AGPRs)
constexpr int kWideTMs[] = {2, 4, 7, 10, 13};
constexpr int kWideBN = 128;                 // output channels per work-group
constexpr int kWidePSL = WideLds<kWideBN>::PSL;
constexpr int kWideCUs = 256;
}  // namespace

static int wide_rp(int W) { return 3 * W + 16; }

// Patch rows a pass of pb blocks can touch: the rows its 32 * pb slots span (starting
// anywhere in a row) plus one above and below.
static int wide_rows(int W, int pb) { return (W - 1 + 32 * pb - 1) / W + 1 + 2; }

bool wide_tm_ok(int tm)
{
  for (int t : kWideTMs)
    if (t == tm) return true;
  return false;
}

// Blocks per wave and pass (tm) and pixel ranges (gx) of a layer: per work-group an equal
// share of the 32-slot blocks; tm minimising the critical path of a work-group in MFMA-times
// -- passes x tm blocks of 9 x chunks MFMAs, a per-pass cost and the epilogue (~24
// MFMA-times a block) -- within the LDS patch.
// Used for Cin >= 128 (measured on MI355X at batch 64 against the kernels it replaces:
// 128 -> 128 at 40x40 41.8 vs 43.2 us, 256 -> 256 at 20x20 42.6 vs 45.8 us); with 64 input
// channels (four chunks per pass) the first chunk's copies are not covered and the
// resident-weight kernel stays faster (64 -> 64 at 80x80: 44.7 us).
bool wide_plan(int cin, int cout, int H, int W, int batch, int act, int * tm, int * gx)
{
  if (cin < 128 || cin % 32 || cout <= 64 || cout > 256 || H < 3 || W < 2 || W >= (1 << 14)) return false;
  if (act != kActSiLU) return false;
  const long htot = (long)batch * (H + 1) - 1, nslot = htot * W;
  if (nslot >= (1L << 22) - 64) return false;
  const int ncg = (cout + kWideBN - 1) / kWideBN;
  const long nblk = (nslot + 31) / 32;
  const int g = (int)std::min<long>(std::max(1, kWideCUs / ncg), nblk);
  const long nb = (nblk + g - 1) / g;  // blocks of the largest range
  const int nchunks = cin / 16;
  double best = 1e30;
  for (int t : kWideTMs) {
    if ((long)wide_rows(W, t) * wide_rp(W) > kWidePSL) continue;
    const long passes = (nb + t - 1) / t;
    const double cost = (double)passes * (t * (9.0 * nchunks + 24.0) + 200.0);
    if (cost < best) {
      best = cost;
      *tm = t;
    }
  }
  if (best >= 1e30) return false;
  *gx = g;
  return true;
}

static WideGeom wide_geom(const ConvParams & p)
{
  WideGeom g;
  g.rp = wide_rp(p.W);
  g.nslot = (int)(((long)p.batch * (p.H + 1) - 1) * p.W);
  g.nblk = (g.nslot + 31) / 32;
  g.gx = p.tw;
  g.ncg = (p.Cout + kWideBN - 1) / kWideBN;
  g.nchunks = (p.Cin + 15) / 16;
  return g;
}

long wide_grid(const ConvParams & p) { return (long)p.tw * wide_geom(p).ncg; }

template <int TM, int TN, int WGM, int WGN, bool RES>
static void launch_wide_t(const ConvParams & p, const WideGeom & g, hipStream_t s)
{
  const dim3 grid((unsigned)(g.gx * g.ncg)), block(256);
  hipLaunchKernelGGL((conv3x3_wide_kernel<TM, TN, WGM, WGN, kActSiLU, RES>), grid, block, 0, s, p, g);
}

template <bool RES>
static void launch_wide_tm(const ConvParams & p, const WideGeom & g, hipStream_t s)
{
  switch (p.th) {
  case 2: launch_wide_t<2, 1, 1, 4, RES>(p, g, s); break;
  case 4: launch_wide_t<4, 1, 1, 4, RES>(p, g, s); break;
  case 7: launch_wide_t<7, 1, 1, 4, RES>(p, g, s); break;
  case 10: launch_wide_t<10, 1, 1, 4, RES>(p, g, s); break;
  default: launch_wide_t<13, 1, 1, 4, RES>(p, g, s); break;
  }
}

void launch_conv_wide(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_wide(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  const WideGeom g = wide_geom(p);
  if (p.r.ptr) launch_wide_tm<true>(p, g, s);
  else launch_wide_tm<false>(p, g, s);
}

}  // namespace ivh
