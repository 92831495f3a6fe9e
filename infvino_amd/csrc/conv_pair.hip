// Two chained 3x3 stride-1 convs of 16 or 32 channels (the C2f / C3k2 bottleneck: conv ->
// conv, optionally + the first conv's input) as one kernel on gfx950 fp16 MFMA.
//
// The reference runs them as two conv3x3 nodes (kernels/conv_ov.cl:133-297 each, the add
// folded into the second: src/PlanModel.cpp:667-740): the intermediate t goes to memory and
// is read back, and the residual x is read again.  Here a work-group keeps t in LDS:
//   t = round(act1(conv1(x) + b1))                          on the tile plus a 1-pixel ring
//   y = round(round(act2(conv2(t) + b2)) + x)               on the tile
// with every rounding point of the two nodes kept, and zeros for t outside the image (the
// second conv's padding).  HBM sees x once (with a 2-pixel halo) and y once.
//
// Geometry as the other 3x3 kernels: the batch is one tall image with a zero separator row
// after each image; a TH x TW output tile needs a (TH+4) x (TW+4) input patch and a
// (TH+2) x (TW+2) ring of t, which must fit the eight waves' MFMA pixel blocks
// ((TH+2)(TW+2) <= 512: two 32-pixel blocks per wave with 32 channels, four 16-pixel blocks
// with 16): a wave's blocks share every weight fragment and are independent MFMA chains, so
// none waits on another's accumulator.  The grid is persistent (one work-group of eight
// waves per CU with 32 channels, two with 16) over contiguous tile ranges; both convs'
// weights stay in LDS, the next tiles' patches are in flight in registers two tiles ahead
// (as in conv_res.hip), and every patch or t read is an MFMA fragment of 8 channels of a
// block's pixels in a pixel-major layout whose rows are padded so that fragments which wrap
// a row stay bank-conflict free.
#include <algorithm>
#include <type_traits>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef unsigned u2q __attribute__((ext_vector_type(2)));
typedef unsigned u4q __attribute__((ext_vector_type(4)));

// Per channel count: MFMA shape, 16-byte LDS layouts and tile limits.
//   32 channels: v_mfma_f32_32x32x16_f16, blocks of 32 pixels, two per wave, K = 9 taps x 32
//                in 18 slices of 16; one work-group (137 KB of LDS) per CU
//   16 channels: v_mfma_f32_16x16x32_f16, blocks of 16 pixels, four per wave, K = 10 taps x 16
//                (a zero tenth tap, the 16-channel halo packing) in 5 slices of 32, a slice's
//                two taps split between the lane halves; two work-groups (61 KB) per CU
template <int C> struct PairT;
template <> struct PairT<32> {
  static constexpr int MB = 32, NB = 2, KP = 288, NSL = 18, WGS_PER_CU = 1;
};
template <> struct PairT<16> {
  static constexpr int MB = 16, NB = 4, KP = 160, NSL = 5, WGS_PER_CU = 2;
};
// LDS layouts.  gfx950 serves a ds_read_b128 in four cycles of 16 lanes: in each half-wave
// the lanes of the quads (lane / 4) of even bit parity, then those of odd parity (lanes 0-3,
// 12-15, 20-27 together; 4-11, 16-19, 28-31 together), 64 banks of 4 bytes; measured with
// SQ_LDS_BANK_CONFLICT on single-pattern probes.  A fragment is conflict free when those 16
// lanes fall on 16 distinct 16-byte slots of a 256-byte window:
//   32 channels: 32 consecutive pixels at an 80-byte pitch (5 slots: a bijection of
//                lane mod 16, which each cycle's lanes cover once); weight rows of 592 bytes
//   16 channels: 16 pixels x 2 channel halves: lanes l and l + 16 read one pixel at +0 and
//                +16 bytes, so a cycle holds pixels {0-3, 12-15} at +0 and {4-11} at +16;
//                a 32-byte pitch (2 slots: even slots +0, odd +16) keeps them apart, where
//                48 bytes (3 slots) collides.  Weights slice-major: [K slice][K half of 16]
//                [16 rows][16 halves], the same 32-byte pitch across a fragment's rows.
template <int C> struct PairL {
  static constexpr int CKP = C == 32 ? 40 : 16;   // pixel pitch (halves)
  static constexpr int LDK = PairT<C>::KP + 8;    // weight row pitch (halves, 32 channels)
  static constexpr int WSZ = C == 32 ? 32 * LDK : PairT<C>::KP * 16;  // weight buffer (halves)
  static constexpr int RING = 8 * PairT<C>::NB * PairT<C>::MB;  // ring / tile pixels
  static constexpr int PMAX = 640;               // patch pixels ((TH+4)(TW+4)) a tile may need
  static constexpr int MAXROWS = 36;             // patch rows (TH + 4)
  // rows padded so each starts where a linear layout of the tile's pixels would, modulo 256
  // bytes (-2 pixels mod 256 B): see conv_res.hip
  static constexpr int PADH = ((256 - (4 * CKP) % 256) % 256) / 2;
};
constexpr int kPairCUs = 256;
}  // namespace

struct PairGeom {
  int th, tw, tiles_x, ntiles;
};

template <int C, int ACT1, int ACT2, bool RES>
__global__ void __launch_bounds__(512, 2 * PairT<C>::WGS_PER_CU) conv3x3_pair_kernel(const ConvParams a, const ConvParams b,
                                                                                const PairGeom g)
{
  using T = PairT<C>;
  using L = PairL<C>;
  using F = Mf<T::MB>;
  typedef typename F::acc_t acc_t;
  constexpr int NT = 512, NB = T::NB, BLK = T::MB, CKP = L::CKP;
  constexpr int CQ = C / 8;                            // 16-byte pieces per pixel
  constexpr int P_IT = (L::PMAX * CQ + NT - 1) / NT;    // patch pieces per thread
  constexpr int WQ = T::KP / 8;
  constexpr int W_IT = (2 * C * WQ + NT - 1) / NT;
  constexpr int L_P = L::PMAX * CKP + L::MAXROWS * L::PADH;
  constexpr int L_T = L::RING * CKP + L::MAXROWS * L::PADH;
  __shared__ __attribute__((aligned(16))) _Float16 WA[L::WSZ];
  __shared__ __attribute__((aligned(16))) _Float16 WB[L::WSZ];
  // LDS place of the 8 halves q (K = 8 q .. 8 q + 7) of weight row `row`
  auto wslot = [&](int row, int q) {
    return C == 32 ? row * L::LDK + q * 8 : (q >> 2) * 512 + ((q >> 1) & 1) * 256 + row * 16 + (q & 1) * 8;
  };
  // one zero pixel after the patch and after the ring: the 16-channel K's tenth tap reads it
  // (its weights are zero; a real pixel could hold an infinity)
  __shared__ __attribute__((aligned(16))) _Float16 Ps[L_P + C];
  __shared__ __attribute__((aligned(16))) _Float16 Ts[L_T + C];
  __shared__ __attribute__((aligned(16))) float BA[C], BB[C];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int TH = g.th, TW = g.tw;
  const int PWd = TW + 4, EW = TW + 2;                 // patch and ring widths
  const int RPH = PWd * CKP + L::PADH;                 // patch row pitch (halves)
  const int RTH = EW * CKP + L::PADH;                  // ring row pitch (halves)
  const int Hs = a.H + 1;
  const int G = gridDim.x;
  const int r = xcd_tile(blockIdx.x, G);
  const int t_lo = (int)((long)r * g.ntiles / G), t_hi = (int)((long)(r + 1) * g.ntiles / G);
  const int ntl = t_hi - t_lo;
  if (ntl <= 0) return;

  const long x_last = (long)(a.batch - 1) * a.x.img + ((long)a.H * a.W - 1) * a.x.cs + C;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(a.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const long y_last = (long)(b.batch - 1) * b.y.img + ((long)b.H * b.W - 1) * b.y.cs + C;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(b.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);

  // ---- weights and bias of both convs into LDS (rows [co][tap][C] of the halo packing)
  {
    const __amdgpu_buffer_rsrc_t wra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(a.w), (short)0, C * a.kpad * 2, kBufDword3);
    const __amdgpu_buffer_rsrc_t wrb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(b.w), (short)0, C * b.kpad * 2, kBufDword3);
    h8 rw[W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, m = e / (C * WQ), rem = e - m * C * WQ;
      const int row = rem / WQ, q = rem - row * WQ;
      const unsigned off = e < 2 * C * WQ ? (unsigned)((row * (m ? b.kpad : a.kpad) + q * 8) * 2) : kBufOOB;
      rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(m ? wrb : wra, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, m = e / (C * WQ), rem = e - m * C * WQ;
      const int row = rem / WQ, q = rem - row * WQ;
      if (e < 2 * C * WQ) *reinterpret_cast<h8 *>((m ? WB : WA) + wslot(row, q)) = rw[i];
    }
    if (tid < C) BA[tid] = a.bias ? a.bias[tid] : 0.0f;
    else if (tid < 2 * C) BB[tid - C] = b.bias ? b.bias[tid - C] : 0.0f;
    if (C == 16 && tid >= 64 && tid < 64 + 2 * CQ)
      *reinterpret_cast<h8 *>((tid < 64 + CQ ? Ps + L_P : Ts + L_T) + (tid % CQ) * 8) = h8{};
  }

  // ---- patch pieces: element e = tid + NT i -> patch pixel e / CQ (row << 16 | column,
  // 0x7fff0000 past the patch), piece e % CQ
  const int q8 = (tid % CQ) * 8;
  const int PP = (TH + 4) * PWd;
  const float inv_pw = __builtin_amdgcn_rcpf((float)PWd);
  int pyx[P_IT];
#pragma unroll
  for (int i = 0; i < P_IT; ++i) {
    const int pp = (tid + i * NT) / CQ;
    const int py = idiv_small(pp, PWd, inv_pw);
    pyx[i] = pp < PP ? (py << 16) | (pp - py * PWd) : 0x7fff0000;
  }
  auto tile_origin = [&](int t, int & b0, int & r0, int & ox0) __attribute__((always_inline)) {
    const int ty = t / g.tiles_x;
    const int oy0 = ty * TH;
    b0 = oy0 / Hs;
    r0 = oy0 - b0 * Hs;
    ox0 = (t - ty * g.tiles_x) * TW;
  };
  const int xcs = a.x.cs, xwcs = a.W * a.x.cs;
  const int xdelta = (int)a.x.img - Hs * xwcs;
  // patch of tile t (rows oy0 - 2 .. oy0 + TH + 1, columns ox0 - 2 .. ox0 + TW + 1) into
  // registers; pixels outside the image read zeros from past the buffer range
  auto load_patch = [&](int t, h8 (&rp)[P_IT]) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
    int rb = r0 - 2, bb = b0;  // first patch row: 2 rows up (into the previous image's separator)
    if (rb < 0 && bb > 0) {
      rb += Hs;
      --bb;
    }
    const bool next_ok = bb + 1 < a.batch;
    const int base = bb * (int)a.x.img + (rb * a.W + ox0 - 2) * xcs + q8;
#pragma unroll
    for (int i = 0; i < P_IT; ++i) {
      const int py = pyx[i] >> 16, px = pyx[i] & 0xffff;
      const int rr = rb + py;
      const bool wrap = rr >= Hs;
      const int rw = wrap ? rr - Hs : rr;
      const int ix = ox0 - 2 + px;
      const bool ok = (unsigned)rw < (unsigned)a.H && (unsigned)ix < (unsigned)a.W && (!wrap || next_ok) && py < TH + 4;
      const int off = base + __umul24(py, xwcs) + __umul24(px, xcs) + (wrap ? xdelta : 0);
      rp[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? (unsigned)off * 2u : kBufOOB, 0, 0));
    }
  };
  auto store_patch = [&](const h8 (&rp)[P_IT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P_IT; ++i)
      if (pyx[i] != 0x7fff0000)
        *reinterpret_cast<h8 *>(Ps + (pyx[i] >> 16) * RPH + (pyx[i] & 0xffff) * CKP + q8) = rp[i];
  };

  // ---- this wave's pixel blocks (blocks wave + 8 k): ring pixels (conv1) and output pixels
  // (conv2) of the lane, clamped to pixel 0 past the ring / tile (computed, discarded)
  const float inv_ew = __builtin_amdgcn_rcpf((float)EW), inv_tw = __builtin_amdgcn_rcpf((float)TW);
  const int EP = (TH + 2) * EW, OP = TH * TW;
  const int kq = F::kq(lane);
  // the lane's channels within a pixel for its B fragments (C = 16: the K offset's channel
  // part; its tap part, lane half 0 or 1, selects the slice's first or second tap)
  const int kc = kq % C;
  const int khalf = C == 16 ? (kq >= 16 ? 1 : 0) : 0;
  // ring pixel (row, column) of block k's lane, and output pixel (row, column): recomputed in
  // the epilogues rather than held across the tile loop
  auto ring_px = [&](int k, int & y, int & x) __attribute__((always_inline)) {
    const int e = (wave + 8 * k) * BLK + (lane % BLK), ec = e < EP ? e : 0;
    y = idiv_small(ec, EW, inv_ew);
    x = ec - y * EW;
  };
  auto out_px = [&](int k, int & y, int & x) __attribute__((always_inline)) {
    const int o = (wave + 8 * k) * BLK + (lane % BLK), oc = o < OP ? o : 0;
    y = idiv_small(oc, TW, inv_tw);
    x = oc - y * TW;
  };
  // per block: patch fragment base of the ring pixel (low 16 bits) and ring fragment base of
  // the output pixel (high 16 bits), in halves (both buffers are under 64 Ki halves)
  static_assert(L_P + C < 65536 && L_T + C < 65536, "16-bit LDS bases");
  unsigned bases[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    int y, x;
    ring_px(k, y, x);
    const int b1 = y * RPH + x * CKP + kc;
    out_px(k, y, x);
    const int b2 = y * RTH + x * CKP + kc;
    bases[k] = (unsigned)b1 | ((unsigned)b2 << 16);
  }
  const int arow = wslot(lane % BLK, kq / 8);  // A fragment of K slice 0 (slice sl: + sl * astep)
  constexpr int astep = C == 32 ? F::KD : 512;

  // patches in flight: two tiles ahead with one work-group per CU (32 channels), one tile
  // ahead with two (16 channels: the other work-group hides the latency, and the registers
  // are needed)
  constexpr int AHEAD = PairT<C>::WGS_PER_CU == 1 ? 2 : 1;
  h8 rpA[P_IT], rpB[AHEAD == 2 ? P_IT : 1];
  load_patch(t_lo, rpA);
  __syncthreads();  // weights in LDS
  store_patch(rpA);
  load_patch(t_lo + (1 < ntl ? 1 : 0), rpA);
  if constexpr (AHEAD == 2) load_patch(t_lo + (2 < ntl ? 2 : 0), rpB);
  __syncthreads();  // first patch in LDS

  // active blocks of this wave (wave-uniform): ring blocks for conv1, tile blocks for conv2
  auto active = [&](int px) {
    const int nblk = (px + BLK - 1) / BLK;
    return __builtin_amdgcn_readfirstlane(wave < nblk ? std::min((nblk - wave + 7) / 8, NB) : 0);
  };
  const int na1 = active(EP), na2 = active(OP);

  // the convs of this wave's first NA blocks (fragment bases of half 0 or 1) over an LDS source
  // (patch or ring) with weights W: one weight fragment feeds the NA MFMAs of a K slice
  auto conv = [&](auto na_c, const _Float16 * W, const _Float16 * S, int half, int rowpitch, int zoff,
                  acc_t (&acc)[NB]) __attribute__((always_inline)) {
    constexpr int NA = decltype(na_c)::value;
    // fragment bases, taken out of the packed registers here (opaque to the compiler, so it
    // does not hold every tap's address of every block across the tile loop); with 16
    // channels the lane halves' taps differ by one pixel (tap pairs 0-1, 4-5, 6-7) or by a
    // row less two pixels (2-3), folded into two bases per block
    int base[NA], baseA[NA], baseB[NA];
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      base[k] = (int)((bases[k] >> (16 * half)) & 0xffffu);
      __asm__ volatile("" : "+v"(base[k]));
      if constexpr (C == 16) {
        baseA[k] = base[k] + (khalf ? CKP : 0);
        baseB[k] = base[k] + (khalf ? rowpitch - 2 * CKP : 0);
      }
    }
    auto toff = [&](int tap) { return (tap / 3) * rowpitch + (tap % 3) * CKP; };
#pragma unroll
    for (int k = 0; k < NA; ++k)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) acc[k][v] = 0.0f;
#pragma unroll
    for (int sl = 0; sl < T::NSL; ++sl) {
      const h8 fa = *reinterpret_cast<const h8 *>(W + arow + sl * astep);
#pragma unroll
      for (int k = 0; k < NA; ++k) {
        int addr;
        if constexpr (C == 32) {
          addr = base[k] + toff(sl / 2) + (sl % 2) * 16;  // tap sl / 2, channels 16 (sl % 2) ..
        } else if (2 * sl + 1 < 9) {
          // taps 2 sl (lane half 0) and 2 sl + 1 (half 1)
          addr = (sl == 1 ? baseB[k] : baseA[k]) + toff(2 * sl);
        } else {
          addr = khalf ? zoff + kc : base[k] + toff(2 * sl);  // tap 8 and the zero tenth tap
        }
        const h8 fb = *reinterpret_cast<const h8 *>(S + addr);
        acc[k] = F::mma(fa, fb, acc[k]);
      }
    }
  };
  // output channel runs of a lane: 4 consecutive channels per run, F::NV / 4 runs per block
  auto run_ch = [&](int v4) { return F::row(lane, v4); };

  // ---- conv1 on the ring: t = round(act1(acc + b1)); zero outside the image
  auto phase1 = [&](auto na_c, int b0, int r0, int ox0) __attribute__((always_inline)) {
    constexpr int NA = decltype(na_c)::value;
    acc_t acc[NB];
    conv(na_c, WA, Ps, 0, RPH, L_P, acc);
    float4 bvs[F::NV / 4];  // bias of the lane's channel runs (the same for every block)
#pragma unroll
    for (int v4 = 0; v4 < F::NV; v4 += 4) bvs[v4 / 4] = *reinterpret_cast<const float4 *>(BA + run_ch(v4));
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      const int e = (wave + 8 * k) * BLK + (lane % BLK);
      int ey, ex;
      ring_px(k, ey, ex);
      // tall-image row / column of this lane's ring pixel
      int rr = r0 - 1 + ey, bb = b0;
      if (rr < 0 && bb > 0) {
        rr += Hs;
        --bb;
      }
      if (rr >= Hs) {
        rr -= Hs;
        ++bb;
      }
      const int cx = ox0 - 1 + ex;
      const bool inside = e < EP && rr >= 0 && rr < a.H && bb < a.batch && cx >= 0 && cx < a.W;
#pragma unroll
      for (int v4 = 0; v4 < F::NV; v4 += 4) {
        const int c = run_ch(v4);  // 4 consecutive channels c .. c + 3
        const float4 bv = bvs[v4 / 4];
        float o[4] = {act_fast<ACT1>(acc[k][v4] + bv.x), act_fast<ACT1>(acc[k][v4 + 1] + bv.y),
                      act_fast<ACT1>(acc[k][v4 + 2] + bv.z), act_fast<ACT1>(acc[k][v4 + 3] + bv.w)};
        h4 hv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __asm__("" : "+v"(o[q]));  // fp32 result, then one fp16 rounding (no fused convert)
          hv[q] = inside ? (_Float16)o[q] : (_Float16)0.0f;
        }
        if (e < EP) *reinterpret_cast<h4 *>(Ts + ey * RTH + ex * CKP + c) = hv;
      }
    }
  };
  // ---- conv2 on the tile, + x, stores of 8 (C = 32) or 4 (C = 16) channels per lane
  auto phase2 = [&](auto na_c, int b0, int r0, int ox0) __attribute__((always_inline)) {
    constexpr int NA = decltype(na_c)::value;
    acc_t acc[NB];
    conv(na_c, WB, Ts, 1, RTH, L_T, acc);
    float4 bvs[F::NV / 4];
#pragma unroll
    for (int v4 = 0; v4 < F::NV; v4 += 4) bvs[v4 / 4] = *reinterpret_cast<const float4 *>(BB + run_ch(v4));
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      const int o = (wave + 8 * k) * BLK + (lane % BLK);
      int oy, ox;
      out_px(k, oy, ox);
      int rr = r0 + oy, bb = b0;
      if (rr >= Hs) {
        rr -= Hs;
        ++bb;
      }
      const int cx = ox0 + ox;
      const bool ok = o < OP && rr < a.H && bb < a.batch && cx < a.W;
      const unsigned yo = ok ? ((unsigned)bb * (unsigned)b.y.img + (unsigned)(rr * a.W + cx) * (unsigned)b.y.cs) * 2u : kBufOOB;
      auto vals = [&](int v4) __attribute__((always_inline)) {
        const int c = run_ch(v4);
        const float4 bv = bvs[v4 / 4];
        float o4[4] = {act_fast<ACT2>(acc[k][v4] + bv.x), act_fast<ACT2>(acc[k][v4 + 1] + bv.y),
                       act_fast<ACT2>(acc[k][v4 + 2] + bv.z), act_fast<ACT2>(acc[k][v4 + 3] + bv.w)};
        h4 hv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __asm__("" : "+v"(o4[q]));
          hv[q] = (_Float16)o4[q];
        }
        if (RES) {  // x at this output pixel: the patch's centre (row oy + 2, column ox + 2)
          const h4 xv = *reinterpret_cast<const h4 *>(Ps + (oy + 2) * RPH + (ox + 2) * CKP + c);
#pragma unroll
          for (int q = 0; q < 4; ++q) hv[q] = (_Float16)((float)hv[q] + (float)xv[q]);
        }
        return hv;
      };
      if constexpr (C == 32) {
#pragma unroll
        for (int v4 = 0; v4 < F::NV; v4 += 8) {
          // runs v4 (channels c..c+3 / c+4..c+7 on lanes < 32 / >= 32) and v4 + 4
          // (c+8..c+11 / c+12..c+15): swapped so every lane holds 8 consecutive channels
          const u2q lo = __builtin_bit_cast(u2q, vals(v4));
          const u2q hi = __builtin_bit_cast(u2q, vals(v4 + 4));
          const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], hi[0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], hi[1], false, false);
          const u4q q = {s0[0], s1[0], s0[1], s1[1]};
          const int c = run_ch(v4) - 4 * (lane >> 5) + 8 * (lane >> 5);
          __builtin_amdgcn_raw_buffer_store_b128(q, yr, yo == kBufOOB ? kBufOOB : yo + (unsigned)c * 2u, 0, 0);
        }
      } else {
        // one run of 4 channels per lane: lanes l, l + 16, l + 32, l + 48 write one pixel
        const int c = run_ch(0);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2q, vals(0)), yr,
                                              yo == kBufOOB ? kBufOOB : yo + (unsigned)c * 2u, 0, 0);
      }
    }
  };
  // a phase over the wave's active block count (0: nothing to do)
  auto dispatch = [&](auto phase, int na, int b0, int r0, int ox0) __attribute__((always_inline)) {
    static_assert(NB == 2 || NB == 4, "blocks per wave");
    if (na == NB) phase(std::integral_constant<int, NB>{}, b0, r0, ox0);
    else if (na == 1) phase(std::integral_constant<int, 1>{}, b0, r0, ox0);
    else if constexpr (NB == 4) {
      if (na == 2) phase(std::integral_constant<int, 2>{}, b0, r0, ox0);
      else if (na == 3) phase(std::integral_constant<int, 3>{}, b0, r0, ox0);
    }
  };

  auto tile = [&](h8 (&rp)[P_IT], int i) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(t_lo + i, b0, r0, ox0);
    dispatch(phase1, na1, b0, r0, ox0);
    __syncthreads();  // the ring of t complete
    dispatch(phase2, na2, b0, r0, ox0);
    __syncthreads();  // patch and ring consumed
    if (i + 1 < ntl) {
      store_patch(rp);  // tile i + 1
      load_patch(t_lo + (i + 1 + AHEAD < ntl ? i + 1 + AHEAD : i + 1), rp);
      __syncthreads();  // next patch in LDS
    }
  };
  if constexpr (AHEAD == 2) {
    for (int i = 0; i < ntl; i += 2) {
      tile(rpA, i);
      if (i + 1 < ntl) tile(rpB, i + 1);
    }
  } else {
    for (int i = 0; i < ntl; ++i) tile(rpA, i);
  }
}

// ---------------------------------------------------------------- host side

// Tile of a layer: (TH + 2)(TW + 2) <= 512 ring pixels (the eight waves' conv1 blocks),
// (TH + 4)(TW + 4) <= the patch buffer, TH + 4 <= H + 1 (at most one image boundary inside a
// patch).  The choice minimises the critical path: rounds of tiles over the persistent grid
// times the per-tile cost (MFMA block rounds of conv1 and conv2 over the eight waves).
template <int C>
static bool pair_plan_c(int H, int W, int batch, int * th, int * tw)
{
  using L = PairL<C>;
  constexpr int WGS = kPairCUs * PairT<C>::WGS_PER_CU, BLKS = 8 * PairT<C>::MB;
  if (H < 4 || W < 2 || (long)batch * (H + 1) >= (1L << 22) || W >= (1 << 14)) return false;
  const long Htot = (long)batch * (H + 1) - 1;
  double best = 1e30;
  for (int w = 1; w <= W && w + 2 <= L::RING; ++w) {
    const int hmax = std::min({L::RING / (w + 2) - 2, L::RING / w, H - 3, L::MAXROWS - 4, L::PMAX / (w + 4) - 4});
    if (hmax < 1) continue;
    const int h = (int)std::min<long>(hmax, Htot);
    const long ty = (Htot + h - 1) / h, tx = (W + w - 1) / w;
    const int hh = (int)((Htot + ty - 1) / ty), ww = (int)((W + tx - 1) / tx);  // balanced
    const long n = ty * tx;
    const long rounds = (n + WGS - 1) / WGS;
    // per tile: conv1 over the ring's blocks, conv2 over the tile's, both spread over 8 waves
    const int per = ((hh + 2) * (ww + 2) + BLKS - 1) / BLKS + (hh * ww + BLKS - 1) / BLKS;
    // ties: more tiles while they fit one round (more CUs share a small layer), else fewer
    const double cost = (double)rounds * per + (n <= WGS ? -1e-6 * (double)n : 1e-6 * (double)n);
    if (cost < best) {
      best = cost;
      *th = hh;
      *tw = ww;
    }
  }
  return best < 1e30;
}

bool pair_plan(int C, int H, int W, int batch, int * th, int * tw)
{
  if (C == 32) return pair_plan_c<32>(H, W, batch, th, tw);
  if (C == 16) return pair_plan_c<16>(H, W, batch, th, tw);
  return false;
}

bool pair_tile_ok(int C, int th, int tw)
{
  if (C != 16 && C != 32) return false;
  const int ring = 512, pmax = 640, maxrows = 36;  // PairL<16> and PairL<32> agree
  static_assert(PairL<16>::RING == 512 && PairL<32>::RING == 512 && PairL<16>::PMAX == 640 &&
                PairL<32>::PMAX == 640 && PairL<16>::MAXROWS == 36 && PairL<32>::MAXROWS == 36,
                "pair tile limits");
  return th >= 1 && tw >= 1 && (th + 2) * (tw + 2) <= ring && (th + 4) * (tw + 4) <= pmax && th + 4 <= maxrows;
}

long pair_tiles(int H, int W, int batch, int th, int tw)
{
  const long Htot = (long)batch * (H + 1) - 1;
  return ((Htot + th - 1) / th) * ((W + tw - 1) / tw);
}

template <int C, int ACT1, bool RES>
static void launch_pair_a2(const ConvParams & a, const ConvParams & b, const PairGeom & g, hipStream_t s)
{
  const dim3 grid((unsigned)std::min(g.ntiles, kPairCUs * PairT<C>::WGS_PER_CU)), block(512);
  switch (b.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3_pair_kernel<C, ACT1, kActSiLU, RES>), grid, block, 0, s, a, b, g); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3_pair_kernel<C, ACT1, kActReLU, RES>), grid, block, 0, s, a, b, g); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3_pair_kernel<C, ACT1, kActHSwish, RES>), grid, block, 0, s, a, b, g); break;
  default: hipLaunchKernelGGL((conv3x3_pair_kernel<C, ACT1, kActNone, RES>), grid, block, 0, s, a, b, g); break;
  }
}

template <int C, bool RES>
static void launch_pair_res(const ConvParams & a, const ConvParams & b, const PairGeom & g, hipStream_t s)
{
  switch (a.act) {
  case kActSiLU: launch_pair_a2<C, kActSiLU, RES>(a, b, g, s); break;
  case kActReLU: launch_pair_a2<C, kActReLU, RES>(a, b, g, s); break;
  case kActHSwish: launch_pair_a2<C, kActHSwish, RES>(a, b, g, s); break;
  default: launch_pair_a2<C, kActNone, RES>(a, b, g, s); break;
  }
}

void launch_conv_pair(const ConvParams & a, const ConvParams & b, hipStream_t s)
{
  const int bc = conv_batch_chunk(b);
  if (bc < b.batch) {
    for (int b0 = 0; b0 < b.batch; b0 += bc) {
      const int nb = std::min(bc, b.batch - b0);
      launch_conv_pair(conv_batch_slice(a, b0, nb), conv_batch_slice(b, b0, nb), s);
    }
    return;
  }
  PairGeom g;
  g.th = b.th;
  g.tw = b.tw;
  g.tiles_x = (b.W + b.tw - 1) / b.tw;
  g.ntiles = (int)pair_tiles(b.H, b.W, b.batch, b.th, b.tw);
  if (a.Cin == 16) {
    if (b.r.ptr) launch_pair_res<16, true>(a, b, g, s);
    else launch_pair_res<16, false>(a, b, g, s);
  } else {
    if (b.r.ptr) launch_pair_res<32, true>(a, b, g, s);
    else launch_pair_res<32, false>(a, b, g, s);
  }
}

}  // namespace ivh
