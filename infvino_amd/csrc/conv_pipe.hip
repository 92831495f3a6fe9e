// 3x3 stride-1 pad-1 convolution on gfx950 fp16 MFMA with a DMA-fed LDS pipeline.
//
// Replaces, for channels-last layers with Cin % 8 == 0 and Cin >= 32, the reference's 3x3
// kernels conv3x3_ov (kernels/conv_ov.cl:133-297), conv3x3_blk (conv_blk.cl:118-296) and
// conv3x3_f16 (conv.cl:150-414):
//   y[co][p] = act(sum_{tap,ci} W[co][ci][tap] x[ci][p + tap] + b[co]) (+ r[co][p]).
//
// Work items are (output tile, channel block) pairs of the batch-as-one-tall-image (image b
// at rows [b*(H+1), b*(H+1)+H), a zero separator row after each image).  The grid is
// persistent: two work-groups per CU, each walking a contiguous range of items, and the K
// loop of consecutive items runs as one uninterrupted stream of steps.  A step is one tap of
// a 32-channel input chunk: 2 x 16-deep MFMA K slices on v_mfma_f32_32x32x16_f16.
//
// No operand passes through registers on its way to LDS.  Buffer loads with the LDS flag
// (buffer_load_dwordx4 ... lds) copy 16-byte pieces straight into
//   * a ring of three weight slots, one step each (BN rows x 32 K), filled two steps ahead;
//   * two input-patch buffers, (TH+2) x (TW+2) pixels x 32 channels each: the next chunk's
//     patch is copied during the first seven steps of the current chunk.
// A DMA instruction writes 64 consecutive 16-byte LDS slots (one per lane), so layouts are
// chosen per slot and every lane fetches the piece its slot holds: weight slots hold each
// 32 x 16 MFMA A fragment as 1 KB in lane order (conflict-free reads); a patch pixel is five
// slots (four 8-channel pieces and one pad slot that a lane fills with zeros) and each
// patch row is padded so that, modulo 16 slots, every pixel sits where it would in a
// pad-free tile-width layout: the 32 lanes of a B fragment (consecutive output pixels, also
// across a tile row wrap) then hit 16 distinct 16-byte bank groups.  Pixels outside the
// image, pad slots and channel pieces at or past Cin read from past the buffer range, which
// the hardware answers with zeros.
//
// Synchronisation: each wave issues the same number of DMA instructions every step (extra
// ones are dummies into a scratch slot), so the number of its DMA instructions younger than
// a step's weights is a compile-time count; the wave waits with s_waitcnt vmcnt(count),
// then one s_barrier per step makes every wave's copies visible and retires the ring slot
// and patch buffer the next copies overwrite.  The ring slots and patch buffers are separate
// LDS objects, so the compiler's own wait analysis sees that reading one does not depend on
// copies into another.  The epilogue (bias, activation in fp32, one fp16 rounding, residual,
// 8-channel stores through v_permlane32_swap) runs straight from the accumulators after an
// item's last step while the next item's first copies are in flight.
#include <algorithm>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned u2p __attribute__((ext_vector_type(2)));
typedef unsigned u4p __attribute__((ext_vector_type(4)));

constexpr int kPipeNW = 3;        // weight ring slots: a step's weights are copied two steps ahead
constexpr int kPipePS = 10 - kPipeNW;  // steps of a chunk that copy the next chunk's patch
constexpr int kPipeWGs = 512;     // persistent grid: two work-groups on each of 256 CUs

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, _Float16 * lds, unsigned voff, int soff)
{
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, (int)voff, soff, 0, 0);
}
}  // namespace

// Host-resolved geometry of one launch.
struct PipeGeom {
  int th, tw;           // output tile
  int rp;               // patch row pitch in 16-byte slots (5 * tw + 16)
  int npi;              // patch DMA instructions per chunk (64 slots each)
  int tiles_x;          // tiles across a row band
  int ntiles;           // pixel tiles
  int nitems;           // ntiles * channel blocks
  int nchunks;          // 32-channel input chunks
};

// Slots of a patch buffer (a multiple of 64: whole DMA instructions stay inside).
template <int BN> struct PipeLds {
  static constexpr int PSL = BN == 128 ? 1728 : 2112;
};

// PRE: the tile-independent part of every patch copy is kept in registers (2 x NPQ VGPRs)
template <int TM, int TN, int WGM, int WGN, int Q, bool PRE, int ACT, bool RES>
__global__ void __launch_bounds__(256, 2) conv3x3_pipe_kernel(const ConvParams p, const PipeGeom g)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  static_assert(WGM * WGN == 4, "four waves");
  constexpr int BN = WGN * TN * 32;
  constexpr int WI = BN / 64;                 // weight DMA instructions per wave and step
  constexpr int PSL = PipeLds<BN>::PSL;
  constexpr int NPQ = kPipePS * Q;            // patch DMA instructions per wave and chunk
  static_assert(NPQ * 4 * 64 >= PSL, "patch copy capacity");
  __shared__ __attribute__((aligned(16))) _Float16 W0[BN * 32];
  __shared__ __attribute__((aligned(16))) _Float16 W1[BN * 32];
  __shared__ __attribute__((aligned(16))) _Float16 W2[BN * 32];
  __shared__ __attribute__((aligned(16))) _Float16 P0[PSL * 8];
  __shared__ __attribute__((aligned(16))) _Float16 P1[PSL * 8];
  __shared__ __attribute__((aligned(16))) _Float16 DUM[512];
  __shared__ __attribute__((aligned(16))) float BIAS[256];  // the bias of every channel block

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int TH = g.th, TW = g.tw, RP = g.rp;
  const int Hs = p.H + 1;

  // this work-group's items (XCD-aware contiguous ranges)
  const int G = gridDim.x;
  const int rr = xcd_tile(blockIdx.x, G);
  const int i_lo = (int)((long)rr * g.nitems / G), i_hi = (int)((long)(rr + 1) * g.nitems / G);
  const int nit = i_hi - i_lo;
  if (nit <= 0) return;
  const int nk = nit * g.nchunks;             // chunks in this work-group's stream

  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const int wrows = (p.Cout + 127) / 128 * 128;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.w), (short)0, (int)((long)wrows * p.kpad * 2), kBufDword3);

  // ---- weight copies: fragment f = wave * WI + i of a step (1 KB, lane order) holds rows
  // (f / 2) * 32 + lane % 32 of the block, K pieces 2 * (f % 2) + lane / 32 of the step
  auto wl = [&](int i) __attribute__((always_inline)) {
    const int f = wave * WI + i;
    const int co = (f >> 1) * 32 + (lane & 31), piece = 2 * (f & 1) + (lane >> 5);
    return (unsigned)((co * p.kpad + piece * 8) * 2);
  };
  // copies of step s (K range 32 s .. 32 s + 31) of channel block blk into ring slot buf
  // (!live: past the stream, dummies reading zeros)
  auto copy_w = [&](_Float16 * buf, int blk, int s, bool live) __attribute__((always_inline)) {
    const int soff = live ? (blk * BN * p.kpad + s * 32) * 2 : 0;
#pragma unroll
    for (int i = 0; i < WI; ++i) dma16(wr, buf + (wave * WI + i) * 512, live ? wl(i) : kBufOOB, soff);
  };

  // ---- patch copies: this wave's instruction j = u * 4 + wave (u = t * Q + q) of a chunk
  // covers slots 64 j .. 64 j + 63; a lane's slot is (row py, pixel px, piece pc), pc 4 being
  // the pad slot
  const int prow = TH + 2, pcol = TW + 2;
  const float inv_rp = __builtin_amdgcn_rcpf((float)RP);
  const int xcs = p.x.cs, xwcs = p.W * p.x.cs;
  const int xdelta = (int)p.x.img - Hs * xwcs;  // (b, r + Hs) -> (b + 1, r)
  // origin of item `it`'s tile: first output row (image b0, row r0) and column ox0
  auto tile_origin = [&](int it, int & b0, int & r0, int & ox0) __attribute__((always_inline)) {
    const int tile = it % g.ntiles;
    const int ty = tile / g.tiles_x;
    const int oy0 = ty * TH;
    b0 = oy0 / Hs;
    r0 = oy0 - b0 * Hs;
    ox0 = (tile - ty * g.tiles_x) * TW;
  };
  // chunk-stream index kc -> item and chunk; per-lane copy state of that chunk's patch
  struct PatchSrc {
    int base, rb, c0;
    bool next_ok, live;
    int ox0;
  };
  auto patch_src = [&](int kc) __attribute__((always_inline)) {
    PatchSrc ps;
    ps.live = kc < nk;
    const int it = i_lo + (ps.live ? kc / g.nchunks : 0);
    ps.c0 = (ps.live ? kc % g.nchunks : 0) * 32;
    int b0, r0, ox0;
    tile_origin(it, b0, r0, ox0);
    int rb = r0 - 1, bb = b0;
    if (rb < 0 && bb > 0) {
      rb += Hs;
      --bb;
    }
    ps.rb = rb;
    ps.ox0 = ox0;
    ps.next_ok = bb + 1 < p.batch;
    ps.base = bb * (int)p.x.img + (rb * p.W + ox0 - 1) * xcs + ps.c0;
    return ps;
  };
  // Tile-independent part of copy u: packed row / pixel / piece (py << 16 | px << 3 | pc) and
  // the offset of that piece from the patch origin, -1 for a slot no input fills (pad
  // slots, slots past the patch).  With PRE it is kept in registers for the whole K loop,
  // otherwise recomputed at every copy.
  auto pdesc_of = [&](int u, int & yxc, int & soff) __attribute__((always_inline)) {
    const int j = u * 4 + wave;
    int e = j * 64 + lane;
    if (!PRE) __asm__ volatile("" : "+v"(e));  // not hoisted out of the K loop
    const int py = idiv_small(e, RP, inv_rp), rem = e - py * RP;
    const int px = (rem * 13108) >> 16, pc = rem - px * 5;  // rem / 5 (exact for rem < 16384)
    yxc = (py << 16) | (px << 3) | pc;
    soff = ((py < prow) & (px < pcol) & (pc < 4)) ? (int)(__umul24(py, xwcs) + __umul24(px, xcs)) + pc * 8 : -1;
  };
  int pre_yxc[PRE ? NPQ : 1], pre_off[PRE ? NPQ : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int u = 0; u < NPQ; ++u) pdesc_of(u, pre_yxc[u], pre_off[u]);
  }
  auto copy_p = [&](_Float16 * buf, const PatchSrc & ps, int u) __attribute__((always_inline)) {
    const int j = u * 4 + wave;
    int yxc, soff;
    if constexpr (PRE) {
      yxc = pre_yxc[u];
      soff = pre_off[u];
    } else {
      pdesc_of(u, yxc, soff);
    }
    const int py = yxc >> 16, px = (yxc >> 3) & 0x1fff, pc = yxc & 7;
    const int rrw = ps.rb + py;
    const bool wrap = rrw >= Hs;
    const int rw = wrap ? rrw - Hs : rrw;
    const int ix = ps.ox0 - 1 + px;
    // bitwise: no branches in the copy
    const bool ok = (soff >= 0) & ps.live & (ps.c0 + pc * 8 < p.Cin) & ((unsigned)rw < (unsigned)p.H) &
                    ((unsigned)ix < (unsigned)p.W) & (!wrap | ps.next_ok);
    const int off = ps.base + soff + (wrap ? xdelta : 0);
    // instructions past the chunk's patch go to the scratch slot
    _Float16 * dst = j < g.npi ? buf + j * 512 : DUM;
    dma16(xr, dst, ok ? (unsigned)off * 2u : kBufOOB, 0);
  };

  // ---- per-lane fragment addresses
  int bl[TM];
  const float inv_tw = __builtin_amdgcn_rcpf((float)TW);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    int o = wm * TM * 32 + tm * 32 + (lane & 31);
    if (o >= TH * TW) o = 0;  // slot past the tile: computed on pixel 0, never stored
    const int ty = idiv_small(o, TW, inv_tw), tx = o - ty * TW;
    bl[tm] = (ty * RP + tx * 5 + (lane >> 5)) * 8;  // halves
  }
  const int al = ((wn * TN) * 2 * 64 + lane) * 8;  // A fragment (tn 0, slice 0) of this wave, halves

  // ---- epilogue: outputs straight from the accumulators, 8 channels (16 bytes) a store
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.H * p.W - 1) * p.y.cs + ((p.Cout + 7) & ~7);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);
  const long r_last = RES ? (long)(p.batch - 1) * p.r.img + ((long)p.H * p.W - 1) * p.r.cs + p.Cout : 0;
  const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(RES ? p.r.ptr : p.y.ptr, (short)0,
                                                                        (int)(r_last * 2), kBufDword3);
  const int cl0 = wn * TN * 32 + 4 * (lane >> 5);  // lane's first channel of a block, within BN
  auto epilogue = [&](acc_t (&acc)[TN][TM], int it) __attribute__((always_inline)) {
    int b0, r0, ox0;
    tile_origin(it, b0, r0, ox0);
    const int n0 = (it / g.ntiles) * BN;
    unsigned yo[TM], ro[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int o = wm * TM * 32 + tm * 32 + (lane & 31);
      const int ty = idiv_small(o, TW, inv_tw), tx = o - ty * TW;
      int r = r0 + ty, b = b0;
      if (r >= Hs) {  // TH + 2 <= Hs: at most one image boundary inside a tile
        r -= Hs;
        ++b;
      }
      const int ox = ox0 + tx;
      const bool ok = o < TH * TW && r < p.H && b < p.batch && ox < p.W;
      const unsigned hw = (unsigned)(r * p.W + ox);
      yo[tm] = ok ? ((unsigned)b * (unsigned)p.y.img + hw * (unsigned)p.y.cs + (unsigned)n0) * 2u : kBufOOB;
      ro[tm] = RES && ok ? ((unsigned)b * (unsigned)p.r.img + hw * (unsigned)p.r.cs + (unsigned)n0) * 2u : kBufOOB;
    }
    auto coff = [&](unsigned base, int cl) { return n0 + cl < p.Cout ? base + (unsigned)cl * 2u : kBufOOB; };
    // two blocks (one tn, tm and tm + 1) at a time: their residual values, then their outputs
    constexpr int TM2 = TM >= 2 ? 2 : 1;
#pragma unroll
    for (int bb = 0; bb < TN * TM / TM2; ++bb) {
      const int tn = bb / (TM / TM2), tmb = (bb % (TM / TM2)) * TM2;
      h4 rv[TM2 * 4];
      if (RES) {
#pragma unroll
        for (int q = 0; q < TM2 * 4; ++q) {
          const int tm = tmb + q / 4, v4 = (q % 4) * 4;
          rv[q] = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rres, coff(ro[tm], tn * 32 + cl0 + 2 * v4), 0, 0));
        }
      }
      auto vals = [&](int q) __attribute__((always_inline)) {
        const int tm = tmb + q / 4, v4 = (q % 4) * 4;
        const int cl = tn * 32 + cl0 + 2 * v4;
        const float4 b4 = *reinterpret_cast<const float4 *>(BIAS + n0 + cl);
        float o[4] = {act_fast<ACT>(acc[tn][tm][v4 + 0] + b4.x), act_fast<ACT>(acc[tn][tm][v4 + 1] + b4.y),
                      act_fast<ACT>(acc[tn][tm][v4 + 2] + b4.z), act_fast<ACT>(acc[tn][tm][v4 + 3] + b4.w)};
        h4 hv;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          __asm__("" : "+v"(o[k]));  // fp32 result, then one fp16 rounding (no fused convert)
          hv[k] = (_Float16)o[k];
        }
        if (RES) {
#pragma unroll
          for (int k = 0; k < 4; ++k) hv[k] = (_Float16)((float)hv[k] + (float)rv[q][k]);
        }
        return hv;
      };
#pragma unroll
      for (int e = 0; e < TM2 * 2; ++e) {
        // groups 2e and 2e + 1: channels c..c+3 / c+8..c+11 (lanes < 32) and c+4..c+7 /
        // c+12..c+15 (lanes >= 32) of one pixel; swapped so every lane holds 8 consecutive ones
        const int q = 2 * e;
        const int tm = tmb + q / 4, v4 = (q % 4) * 4;
        const u2p a = __builtin_bit_cast(u2p, vals(q));
        const u2p b = __builtin_bit_cast(u2p, vals(q + 1));
        const auto s0 = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
        const u4p v = {s0[0], s1[0], s0[1], s1[1]};
        const int cl = tn * 32 + cl0 + 2 * v4 + 4 * (lane >> 5);
        __builtin_amdgcn_raw_buffer_store_b128(v, yr, coff(yo[tm], cl), 0, 0);
      }
    }
  };

  acc_t acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int v = 0; v < F::NV; ++v) acc[a][b][v] = 0.0f;

  // ---- prologue: the bias into LDS, chunk 0's patch, then the first two steps' weights
  for (int c = tid; c < 256; c += 256) BIAS[c] = p.bias && c < wrows ? p.bias[c] : 0.0f;
  __syncthreads();
  {
    const PatchSrc ps = patch_src(0);
#pragma unroll
    for (int u = 0; u < NPQ; ++u) copy_p(P0, ps, u);
  }
  copy_w(W0, i_lo / g.ntiles, 0, true);
  copy_w(W1, i_lo / g.ntiles, 1, true);

  // one chunk of the stream: nine steps on patch buffer PC while the next chunk's patch goes
  // to PN; step t reads ring slot t % 3 and refills slot (t + 2) % 3 with step t + 2
  auto chunk = [&](int kc, _Float16 * PC, _Float16 * PN) __attribute__((always_inline)) {
    const PatchSrc nxt = patch_src(kc + 1);
    // channel block and chunk of this chunk and of the next one (whose first two steps'
    // weights the last two steps copy)
    const int blk_c = (i_lo + kc / g.nchunks) / g.ntiles, c_c = kc % g.nchunks;
    const bool live_n = kc + 1 < nk;
    const int kn = live_n ? kc + 1 : kc;
    const int blk_n = (i_lo + kn / g.nchunks) / g.ntiles, c_n = kn % g.nchunks;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      _Float16 * const wc = t % 3 == 0 ? W0 : (t % 3 == 1 ? W1 : W2);
      _Float16 * const wf = t % 3 == 0 ? W2 : (t % 3 == 1 ? W0 : W1);
      // the previous step's fragment reads and MFMAs stay before the barrier (its reads of
      // ring slot (t+2)%3 are complete before any wave refills it)
      __builtin_amdgcn_sched_barrier(0);
      // this step's weights (and, at t = 0, this chunk's patch) have landed for this wave
      if (t >= 1 && t <= kPipePS) __builtin_amdgcn_s_waitcnt(vm_wait(WI + Q));
      else __builtin_amdgcn_s_waitcnt(vm_wait(WI));
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();  // every wave's copies visible; slot (t+2)%3 and PN free
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if (t + 2 < 9) copy_w(wf, blk_c, c_c * 9 + t + 2, true);
      else copy_w(wf, blk_n, c_n * 9 + t - 7, live_n);
      const int toff = ((t / 3) * RP + (t % 3) * 5) * 8;  // tap offset in halves
      h8 fa[TN], fb[TM];
      auto frags = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) fa[tn] = *reinterpret_cast<const h8 *>(wc + al + (tn * 2 + j) * 512);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) fb[tm] = *reinterpret_cast<const h8 *>(PC + bl[tm] + toff + j * 16);
      };
      auto mmas = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = F::mma(fa[tn], fb[tm], acc[tn][tm]);
      };
      // slice 0's fragment reads, then the patch copies (their address arithmetic fills the
      // LDS latency), then the MFMAs; slice 1 likewise without copies
      frags(0);
      __builtin_amdgcn_sched_barrier(0);
      if (t < kPipePS) {
#pragma unroll
        for (int q = 0; q < Q; ++q) copy_p(PN, nxt, t * Q + q);
      }
      __builtin_amdgcn_sched_barrier(0);
      mmas();
      frags(1);
      mmas();
    }
    if (kc % g.nchunks == g.nchunks - 1) {
      epilogue(acc, i_lo + kc / g.nchunks);
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b)
#pragma unroll
          for (int v = 0; v < F::NV; ++v) acc[a][b][v] = 0.0f;
    }
  };
  for (int kc = 0; kc < nk; kc += 2) {
    chunk(kc, P0, P1);
    if (kc + 1 < nk) chunk(kc + 1, P1, P0);
  }
  // every copy has landed before the work-group ends (the last ones are dummies)
  __builtin_amdgcn_s_waitcnt(vm_wait(0));
}

// ---------------------------------------------------------------- host side

namespace {
struct PipeCfgDesc {
  int bm, bn, psl;
};
// 0: BN 128 (2 x 2 waves of 4 x 2 blocks), 1: BN 64 (4 x 1 waves of 2 x 2 blocks); BM 256
constexpr PipeCfgDesc kPipeCfg[2] = {{256, 128, PipeLds<128>::PSL}, {256, 64, PipeLds<64>::PSL}};
}  // namespace

int pipe_bn(int cfg) { return kPipeCfg[cfg].bn; }

static int pipe_rp(int tw) { return 5 * tw + 16; }

// Config and tile of a layer: BN by Cout; the tile (TH x TW <= BM, patch within the buffer,
// TH + 2 <= H + 1) with the fewest rounds of items over the persistent grid, then the
// fewest MFMA slots plus patch fill.
bool pipe_plan(int cin, int cout, int H, int W, int batch, int act, int * cfg, int * th, int * tw)
{
  if (cin < 32 || cin % 8 || H < 3 || W < 2 || (long)batch * (H + 1) >= (1L << 22) || W >= (1 << 14)) return false;
  if (act != kActNone && act != kActSiLU && act != kActReLU && act != kActHSwish) return false;
  const int c = cout > 64 ? 0 : 1;
  const PipeCfgDesc & d = kPipeCfg[c];
  const long nblk = (cout + d.bn - 1) / d.bn;
  const long Htot = (long)batch * (H + 1) - 1;
  long best_rounds = 1L << 40;
  double best = 1e30;
  for (int w = 1; w <= W && w <= d.bm; ++w) {
    int h = std::min(d.bm / w, H - 1);
    h = (int)std::min<long>(h, Htot);
    while (h >= 1 && (long)(h + 2) * pipe_rp(w) > d.psl) --h;
    if (h < 1) continue;
    const long ty = (Htot + h - 1) / h, tx = (W + w - 1) / w;
    const int hh = (int)((Htot + ty - 1) / ty), ww = (int)((W + tx - 1) / tx);  // balanced
    if ((long)(hh + 2) * pipe_rp(ww) > d.psl) continue;
    const long n = ty * tx * nblk;
    const long rounds = (n + kPipeWGs - 1) / kPipeWGs;
    const double work = (double)n * (d.bm + 0.15 * (hh + 2) * (ww + 2));
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

static PipeGeom pipe_geom(const ConvParams & p)
{
  PipeGeom g;
  g.th = p.th;
  g.tw = p.tw;
  g.rp = pipe_rp(p.tw);
  g.npi = (int)(((long)(p.th + 2) * g.rp + 63) / 64);
  const long Htot = (long)p.batch * (p.H + 1) - 1;
  g.tiles_x = (p.W + p.tw - 1) / p.tw;
  g.ntiles = (int)(((Htot + p.th - 1) / p.th) * g.tiles_x);
  g.nitems = g.ntiles * ((p.Cout + pipe_bn(p.pipe - 1) - 1) / pipe_bn(p.pipe - 1));
  g.nchunks = (p.Cin + 31) / 32;
  return g;
}

long pipe_items(const ConvParams & p) { return pipe_geom(p).nitems; }

bool pipe_views_ok(const ConvParams & p)
{
  if (p.x.layout != kNHWC || (p.x.cs % 8) || (p.x.img % 8) || (reinterpret_cast<uintptr_t>(p.x.ptr) % 16)) return false;
  if ((long)p.W * p.x.cs >= (1L << 23) || p.Cin % 8 || p.cin8 != p.Cin) return false;
  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  if (x_last * 2 >= (1L << 31)) return false;
  return res_views_ok(p) && res_store_width(p) == 8;
}

template <int TM, int TN, int WGM, int WGN, int Q, bool PRE, bool RES>
static void launch_pipe_act(const ConvParams & p, const PipeGeom & g, hipStream_t s)
{
  const dim3 grid((unsigned)std::min(g.nitems, kPipeWGs)), block(256);
  switch (p.act) {
  case kActSiLU: hipLaunchKernelGGL((conv3x3_pipe_kernel<TM, TN, WGM, WGN, Q, PRE, kActSiLU, RES>), grid, block, 0, s, p, g); break;
  case kActReLU: hipLaunchKernelGGL((conv3x3_pipe_kernel<TM, TN, WGM, WGN, Q, PRE, kActReLU, RES>), grid, block, 0, s, p, g); break;
  case kActHSwish: hipLaunchKernelGGL((conv3x3_pipe_kernel<TM, TN, WGM, WGN, Q, PRE, kActHSwish, RES>), grid, block, 0, s, p, g); break;
  default: hipLaunchKernelGGL((conv3x3_pipe_kernel<TM, TN, WGM, WGN, Q, PRE, kActNone, RES>), grid, block, 0, s, p, g); break;
  }
}

void launch_conv_pipe(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_pipe(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  const PipeGeom g = pipe_geom(p);
  if (p.pipe == 1) {
    if (p.r.ptr) launch_pipe_act<4, 2, 2, 2, 1, false, true>(p, g, s);
    else launch_pipe_act<4, 2, 2, 2, 1, false, false>(p, g, s);
  } else {
    if (p.r.ptr) launch_pipe_act<2, 2, 4, 1, 2, true, true>(p, g, s);
    else launch_pipe_act<2, 2, 4, 1, 2, true, false>(p, g, s);
  }
}

}  // namespace ivh
