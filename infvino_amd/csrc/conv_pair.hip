// Two chained 3x3 stride-1 convs of 32 channels (the C2f / C3k2 bottleneck: conv -> conv,
// optionally + the first conv's input) as one kernel on gfx950 fp16 MFMA.
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
// (TH+2) x (TW+2) ring of t, which must fit the eight waves' 32-pixel MFMA blocks, two per
// wave ((TH+2)(TW+2) <= 512): a wave's two blocks share every weight fragment and are two
// independent MFMA chains, so neither waits on the other's accumulator.  The grid is persistent (one work-group of eight waves per CU)
// over contiguous tile ranges; both convs' weights (2 x 32 x 288 fp16) stay in LDS, the next
// tiles' patches are in flight in registers two tiles ahead (as in conv_res.hip), and every
// patch or t read is an MFMA fragment of 32 pixels x 8 channels in a pixel-major layout
// whose rows are padded so that fragments which wrap a row stay bank-conflict free.
#include <algorithm>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef unsigned u2q __attribute__((ext_vector_type(2)));
typedef unsigned u4q __attribute__((ext_vector_type(4)));
constexpr int kPairC = 32;          // channels of x, t and y
constexpr int kPairK = 9 * kPairC;  // K of each conv
constexpr int kPairLDK = kPairK + 8;
constexpr int kPairCKP = kPairC + 8;  // pixel pitch (halves)
constexpr int kPairNB = 2;            // 32-pixel blocks per wave (conv1 ring, conv2 tile)
constexpr int kPairRing = 8 * kPairNB * 32;  // ring / tile pixels of the eight waves
constexpr int kPairPMax = 640;        // patch pixels ((TH+4)(TW+4)) a tile may need
constexpr int kPairMaxRows = 36;      // patch rows (TH + 4)
constexpr int kPairWGs = 256;
// rows padded so each starts where a linear layout of the previous row's pixels would end
// plus 2 pixels, modulo 256 bytes (-2 pixels mod 256 B): see conv_res.hip
constexpr int kPairPadH = ((256 - (4 * kPairCKP) % 256) % 256) / 2;
}  // namespace

struct PairGeom {
  int th, tw, tiles_x, ntiles;
};

template <int ACT1, int ACT2, bool RES>
__global__ void __launch_bounds__(512, 1) conv3x3_pair_kernel(const ConvParams a, const ConvParams b, const PairGeom g)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  constexpr int NT = 512;
  constexpr int CQ = kPairC / 8;                       // 16-byte pieces per pixel
  constexpr int P_IT = (kPairPMax * CQ + NT - 1) / NT;  // patch pieces per thread
  constexpr int WQ = kPairK / 8;
  constexpr int W_IT = (2 * kPairC * WQ + NT - 1) / NT;
  constexpr int L_P = kPairPMax * kPairCKP + kPairMaxRows * kPairPadH;
  constexpr int L_T = kPairRing * kPairCKP + kPairMaxRows * kPairPadH;
  constexpr int NB = kPairNB;
  __shared__ __attribute__((aligned(16))) _Float16 WA[kPairC * kPairLDK];
  __shared__ __attribute__((aligned(16))) _Float16 WB[kPairC * kPairLDK];
  __shared__ __attribute__((aligned(16))) _Float16 Ps[L_P];
  __shared__ __attribute__((aligned(16))) _Float16 Ts[L_T];
  __shared__ __attribute__((aligned(16))) float BA[kPairC], BB[kPairC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int TH = g.th, TW = g.tw;
  const int PWd = TW + 4, EW = TW + 2;                 // patch and ring widths
  const int RPH = PWd * kPairCKP + kPairPadH;          // patch row pitch (halves)
  const int RTH = EW * kPairCKP + kPairPadH;           // ring row pitch (halves)
  const int Hs = a.H + 1;
  const int G = gridDim.x;
  const int r = xcd_tile(blockIdx.x, G);
  const int t_lo = (int)((long)r * g.ntiles / G), t_hi = (int)((long)(r + 1) * g.ntiles / G);
  const int ntl = t_hi - t_lo;
  if (ntl <= 0) return;

  const long x_last = (long)(a.batch - 1) * a.x.img + ((long)a.H * a.W - 1) * a.x.cs + kPairC;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(a.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const long y_last = (long)(b.batch - 1) * b.y.img + ((long)b.H * b.W - 1) * b.y.cs + kPairC;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(b.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);

  // ---- weights and bias of both convs into LDS (rows [co][tap][32] of the halo packing)
  {
    const __amdgpu_buffer_rsrc_t wra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(a.w), (short)0, kPairC * a.kpad * 2, kBufDword3);
    const __amdgpu_buffer_rsrc_t wrb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(b.w), (short)0, kPairC * b.kpad * 2, kBufDword3);
    h8 rw[W_IT];
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, m = e / (kPairC * WQ), rem = e - m * kPairC * WQ;
      const int row = rem / WQ, q = rem - row * WQ;
      const unsigned off = e < 2 * kPairC * WQ ? (unsigned)((row * (m ? b.kpad : a.kpad) + q * 8) * 2) : kBufOOB;
      rw[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(m ? wrb : wra, off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < W_IT; ++i) {
      const int e = tid + i * NT, m = e / (kPairC * WQ), rem = e - m * kPairC * WQ;
      const int row = rem / WQ, q = rem - row * WQ;
      if (e < 2 * kPairC * WQ) *reinterpret_cast<h8 *>((m ? WB : WA) + row * kPairLDK + q * 8) = rw[i];
    }
    if (tid < kPairC) BA[tid] = a.bias ? a.bias[tid] : 0.0f;
    else if (tid < 2 * kPairC) BB[tid - kPairC] = b.bias ? b.bias[tid - kPairC] : 0.0f;
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
        *reinterpret_cast<h8 *>(Ps + (pyx[i] >> 16) * RPH + (pyx[i] & 0xffff) * kPairCKP + q8) = rp[i];
  };

  // ---- this wave's pixel blocks (blocks wave and wave + 8): ring pixels (conv1) and output
  // pixels (conv2) of the lane, clamped to pixel 0 past the ring / tile (computed, discarded)
  const float inv_ew = __builtin_amdgcn_rcpf((float)EW), inv_tw = __builtin_amdgcn_rcpf((float)TW);
  const int EP = (TH + 2) * EW, OP = TH * TW;
  const int kq = F::kq(lane);
  int ey[NB], ex[NB], b1[NB], oy[NB], ox[NB], b2[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int e = (wave + 8 * k) * 32 + (lane & 31), ec = e < EP ? e : 0;
    ey[k] = idiv_small(ec, EW, inv_ew);
    ex[k] = ec - ey[k] * EW;
    b1[k] = ey[k] * RPH + ex[k] * kPairCKP + kq;  // patch fragment base of the ring pixel
    const int o = (wave + 8 * k) * 32 + (lane & 31), oc = o < OP ? o : 0;
    oy[k] = idiv_small(oc, TW, inv_tw);
    ox[k] = oc - oy[k] * TW;
    b2[k] = oy[k] * RTH + ox[k] * kPairCKP + kq;  // ring fragment base of the output pixel
  }
  const int arow = (lane & 31) * kPairLDK + kq;
  const int cl0 = 4 * (lane >> 5);                 // lane's first channel of each run of 4

  h8 rpA[P_IT], rpB[P_IT];
  load_patch(t_lo, rpA);
  __syncthreads();  // weights in LDS
  store_patch(rpA);
  load_patch(t_lo + (1 < ntl ? 1 : 0), rpA);
  load_patch(t_lo + (2 < ntl ? 2 : 0), rpB);
  __syncthreads();  // first patch in LDS

  // the convs of this wave's blocks (fragment bases base[k]) over an LDS source (patch or
  // ring) with weights W: one weight fragment feeds the NB MFMAs of a K slice
  auto conv = [&](const _Float16 * W, const _Float16 * S, const int (&base)[NB], int rowpitch, acc_t (&acc)[NB])
      __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NB; ++k)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) acc[k][v] = 0.0f;
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int toff = (tap / 3) * rowpitch + (tap % 3) * kPairCKP;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const h8 fa = *reinterpret_cast<const h8 *>(W + arow + tap * kPairC + j * 16);
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          const h8 fb = *reinterpret_cast<const h8 *>(S + base[k] + toff + j * 16);
          acc[k] = F::mma(fa, fb, acc[k]);
        }
      }
    }
  };

  auto tile = [&](h8 (&rp)[P_IT], int i) __attribute__((always_inline)) {
    const int t = t_lo + i;
    int b0, r0, ox0;
    tile_origin(t, b0, r0, ox0);
    // ---- conv1 on the ring: t = round(act1(acc + b1)); zero outside the image
    {
      acc_t acc[NB];
      conv(WA, Ps, b1, RPH, acc);
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const int e = (wave + 8 * k) * 32 + (lane & 31);
        // tall-image row / column of this lane's ring pixel
        int rr = r0 - 1 + ey[k], bb = b0;
        if (rr < 0 && bb > 0) {
          rr += Hs;
          --bb;
        }
        if (rr >= Hs) {
          rr -= Hs;
          ++bb;
        }
        const int cx = ox0 - 1 + ex[k];
        const bool inside = e < EP && rr >= 0 && rr < a.H && bb < a.batch && cx >= 0 && cx < a.W;
#pragma unroll
        for (int v4 = 0; v4 < F::NV; v4 += 4) {
          const int c = F::row(lane, v4);  // 4 consecutive channels c .. c + 3
          const float4 bv = *reinterpret_cast<const float4 *>(BA + c);
          float o[4] = {act_fast<ACT1>(acc[k][v4] + bv.x), act_fast<ACT1>(acc[k][v4 + 1] + bv.y),
                        act_fast<ACT1>(acc[k][v4 + 2] + bv.z), act_fast<ACT1>(acc[k][v4 + 3] + bv.w)};
          h4 hv;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            __asm__("" : "+v"(o[q]));  // fp32 result, then one fp16 rounding (no fused convert)
            hv[q] = inside ? (_Float16)o[q] : (_Float16)0.0f;
          }
          if (e < EP) *reinterpret_cast<h4 *>(Ts + ey[k] * RTH + ex[k] * kPairCKP + c) = hv;
        }
      }
    }
    __syncthreads();  // the ring of t complete
    // ---- conv2 on the tile, + x, stores of 8 channels per lane
    if (wave * 32 < OP) {  // wave-uniform: the wave has at least one block of the tile
      acc_t acc[NB];
      conv(WB, Ts, b2, RTH, acc);
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const int o = (wave + 8 * k) * 32 + (lane & 31);
        int rr = r0 + oy[k], bb = b0;
        if (rr >= Hs) {
          rr -= Hs;
          ++bb;
        }
        const int cx = ox0 + ox[k];
        const bool ok = o < OP && rr < a.H && bb < a.batch && cx < a.W;
        const unsigned yo = ok ? ((unsigned)bb * (unsigned)b.y.img + (unsigned)(rr * a.W + cx) * (unsigned)b.y.cs) * 2u : kBufOOB;
        auto vals = [&](int v4) __attribute__((always_inline)) {
          const int c = F::row(lane, v4);
          const float4 bv = *reinterpret_cast<const float4 *>(BB + c);
          float o4[4] = {act_fast<ACT2>(acc[k][v4] + bv.x), act_fast<ACT2>(acc[k][v4 + 1] + bv.y),
                         act_fast<ACT2>(acc[k][v4 + 2] + bv.z), act_fast<ACT2>(acc[k][v4 + 3] + bv.w)};
          h4 hv;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            __asm__("" : "+v"(o4[q]));
            hv[q] = (_Float16)o4[q];
          }
          if (RES) {  // x at this output pixel: the patch's centre (row oy + 2, column ox + 2)
            const h4 xv = *reinterpret_cast<const h4 *>(Ps + (oy[k] + 2) * RPH + (ox[k] + 2) * kPairCKP + c);
#pragma unroll
            for (int q = 0; q < 4; ++q) hv[q] = (_Float16)((float)hv[q] + (float)xv[q]);
          }
          return hv;
        };
#pragma unroll
        for (int v4 = 0; v4 < F::NV; v4 += 8) {
          // runs v4 (channels c..c+3 / c+4..c+7 on lanes < 32 / >= 32) and v4 + 4 (c+8..c+11 /
          // c+12..c+15): swapped so every lane holds 8 consecutive channels of its pixel
          const u2q lo = __builtin_bit_cast(u2q, vals(v4));
          const u2q hi = __builtin_bit_cast(u2q, vals(v4 + 4));
          const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], hi[0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], hi[1], false, false);
          const u4q q = {s0[0], s1[0], s0[1], s1[1]};
          const int c = F::row(lane, v4) - cl0 + 8 * (lane >> 5);
          __builtin_amdgcn_raw_buffer_store_b128(q, yr, yo == kBufOOB ? kBufOOB : yo + (unsigned)c * 2u, 0, 0);
        }
      }
    }
    __syncthreads();  // patch and ring consumed
    if (i + 1 < ntl) {
      store_patch(rp);  // tile i + 1
      load_patch(t_lo + (i + 3 < ntl ? i + 3 : i + 1), rp);
      __syncthreads();  // next patch in LDS
    }
  };
  for (int i = 0; i < ntl; i += 2) {
    tile(rpA, i);
    if (i + 1 < ntl) tile(rpB, i + 1);
  }
}

// ---------------------------------------------------------------- host side

// Tile of a layer: (TH + 2)(TW + 2) <= 512 ring pixels (the eight waves' conv1 blocks, two
// per wave), (TH + 4)(TW + 4) <= the patch buffer, TH + 4 <= H + 1 (at most one image
// boundary inside a patch).  The choice minimises the critical path: rounds of tiles over
// the persistent grid times the per-tile cost (MFMA block rounds of conv1 and conv2 over the
// eight waves).
bool pair_plan(int H, int W, int batch, int * th, int * tw)
{
  if (H < 4 || W < 2 || (long)batch * (H + 1) >= (1L << 22) || W >= (1 << 14)) return false;
  const long Htot = (long)batch * (H + 1) - 1;
  double best = 1e30;
  for (int w = 1; w <= W && w + 2 <= kPairRing; ++w) {
    const int hmax = std::min({kPairRing / (w + 2) - 2, kPairRing / w, H - 3, kPairMaxRows - 4, kPairPMax / (w + 4) - 4});
    if (hmax < 1) continue;
    const int h = (int)std::min<long>(hmax, Htot);
    const long ty = (Htot + h - 1) / h, tx = (W + w - 1) / w;
    const int hh = (int)((Htot + ty - 1) / ty), ww = (int)((W + tx - 1) / tx);  // balanced
    const long n = ty * tx;
    const long rounds = (n + kPairWGs - 1) / kPairWGs;
    // per tile: conv1 over the ring's blocks, conv2 over the tile's, both spread over 8 waves
    const int per = ((hh + 2) * (ww + 2) + 255) / 256 + (hh * ww + 255) / 256;
    // ties: more tiles while they fit one round (more CUs share a small layer), else fewer
    const double cost = (double)rounds * per + (n <= kPairWGs ? -1e-6 * (double)n : 1e-6 * (double)n);
    if (cost < best) {
      best = cost;
      *th = hh;
      *tw = ww;
    }
  }
  return best < 1e30;
}

long pair_tiles(int H, int W, int batch, int th, int tw)
{
  const long Htot = (long)batch * (H + 1) - 1;
  return ((Htot + th - 1) / th) * ((W + tw - 1) / tw);
}

template <int ACT1, bool RES>
static void launch_pair_a2(const ConvParams & a, const ConvParams & b, const PairGeom & g, hipStream_t s)
{
  const dim3 grid((unsigned)std::min(g.ntiles, kPairWGs)), block(512);
  switch (b.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3_pair_kernel<ACT1, kActSiLU, RES>), grid, block, 0, s, a, b, g); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3_pair_kernel<ACT1, kActReLU, RES>), grid, block, 0, s, a, b, g); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3_pair_kernel<ACT1, kActHSwish, RES>), grid, block, 0, s, a, b, g); break;
  default: hipLaunchKernelGGL((conv3x3_pair_kernel<ACT1, kActNone, RES>), grid, block, 0, s, a, b, g); break;
  }
}

template <bool RES>
static void launch_pair_res(const ConvParams & a, const ConvParams & b, const PairGeom & g, hipStream_t s)
{
  switch (a.act) {
  case kActSiLU: launch_pair_a2<kActSiLU, RES>(a, b, g, s); break;
  case kActReLU: launch_pair_a2<kActReLU, RES>(a, b, g, s); break;
  case kActHSwish: launch_pair_a2<kActHSwish, RES>(a, b, g, s); break;
  default: launch_pair_a2<kActNone, RES>(a, b, g, s); break;
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
  if (b.r.ptr) launch_pair_res<true>(a, b, g, s);
  else launch_pair_res<false>(a, b, g, s);
}

}  // namespace ivh
