// The stem (3x3 stride-2 conv of the 3-channel image) and the stride-2 3x3 conv that reads
// it, as one kernel: the stem's output never goes to HBM.
//
// Replaces, for the YOLO input pair "3 -> 16 s2, SiLU" then "16 -> 32 s2, SiLU", two launches
// of the reference's conv3x3_cin3 (kernels/conv_cin3.cl:67-118) and conv3x3_ov with stride 2
// (kernels/conv_ov.cl:133-297), whose 16-channel intermediate (210 MB at batch 64 and 640x640)
// is written and read back.  Both convs keep the arithmetic of their stand-alone kernels here:
// the stem's MFMA formulation and fp32 epilogue of conv_stem_rows_kernel, rounded to fp16 as
// the stored tensor would be; the second conv as fp16 MFMAs over k = tap * 16 + ci with an
// fp32 epilogue.
//
// A work-group owns a band of output rows of one image and walks down it.  Output row r
// needs stem rows 2r-1 .. 2r+1, and stem rows 2r, 2r+1 need input rows 4r-1 .. 4r+3:
//   * those five input rows (all columns, channels interleaved as 4 halves per pixel) are
//     staged in LDS;
//   * stem rows are computed from them (16-pixel blocks, two 16x16x32 MFMAs each) into a
//     ring of stem rows in LDS;
//   * output row r is computed from the ring: 16-pixel x 16-channel blocks, five 16x16x32
//     MFMAs over the 144-deep K (nine taps of 16 channels, a tenth of zeros).
// Ring rows store their columns split by parity (even columns, then odd): the stride-2 taps
// of 16 consecutive output pixels then read 16 consecutive ring pixels.  A ring pixel is 32
// bytes (16 channels); its two 8-channel halves trade places on every other group of 8
// pixels, so 16 lanes reading the same half of 16 consecutive pixels hit distinct banks.
// Steps are pipelined with one barrier each: step r computes the stem rows of output row
// r + 1 (a ring of five stem rows) from one of two input-row buffers, and output row r from
// rows the previous step finished; the next input rows go to the other buffer, and their
// loads are issued two steps ahead.  Within a step the 8 waves' stem work (SiLU, VALU bound)
// and output-row work (LDS fragment reads) overlap.
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef _Float16 h4t __attribute__((ext_vector_type(4)));
typedef float f4t __attribute__((ext_vector_type(4)));
typedef unsigned u2v __attribute__((ext_vector_type(2)));

constexpr int kSsThreads = 512;        // 8 waves
constexpr int kSsInRows = 5;           // input rows staged per output row
constexpr int kSsPS = 16;              // ring pixel pitch (halves): 16 channels, 8-channel
                                       // halves swapped on every other group of 8 pixels
constexpr int kSsLDW = 168;            // second conv's weight row pitch (halves): 160 K + 8
constexpr int kSsMaxW0 = 640;          // widest input the static LDS holds
constexpr int kSsRing = 5;             // stem rows in the ring
}  // namespace

// Staged input rows hold 4 halves (3 channels + 0) per column, columns c = image column + 2,
// with 8 halves of padding after every 8 image columns: a lane stores one 8-column group (64
// bytes), so 16 lanes store at an 80-byte stride, bank-conflict free.  Offset of column c:
static constexpr __host__ __device__ inline int ss_pcol(int c) { return c * 4 + ((c + 6) >> 3) * 8; }

// LDS layout (halves) for an input width W0 and stem width W1
struct StemS2Lds {
  int lw, in_sz, ring_off, plane, ring_row, ring_sz, w_off, total;
};
static constexpr __host__ __device__ inline StemS2Lds stem_s2_lds(int W0, int W1)
{
  StemS2Lds L{};
  L.lw = ss_pcol(W0 + 4);                         // row pitch: 2 zero columns each side
  L.in_sz = kSsInRows * L.lw;                     // one of two input-row buffers
  L.ring_off = 2 * L.in_sz;
  L.plane = ((W1 + 2) / 2 + 1) * kSsPS;           // columns -1 .. W1 split by parity
  L.ring_row = 2 * L.plane;
  L.ring_sz = kSsRing * L.ring_row;
  L.w_off = L.ring_off + L.ring_sz;
  L.total = L.w_off + 32 * kSsLDW;
  return L;
}

template <int ACT1, int ACT2>
__global__ void __launch_bounds__(kSsThreads, 2) conv_stem_s2_kernel(const StemS2Params q)
{
  __shared__ __attribute__((aligned(16))) _Float16 lds[stem_s2_lds(kSsMaxW0, kSsMaxW0 / 2).total];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const StemS2Lds L = stem_s2_lds(q.W0, q.W1);
  // LDS regions are addressed as offsets into `lds` (a pointer picked at run time from an
  // array would lose the LDS address space: flat instead of ds instructions)
  _Float16 * const IN = lds;
  _Float16 * const RING = lds + L.ring_off;
  _Float16 * const W2s = lds + L.w_off;
  // XCD-aware order over (band, image): neighbouring bands share an input row
  const int lin = xcd_tile(blockIdx.x, gridDim.x);
  const int b = lin / q.nb, band = lin - b * q.nb;
  const int r0 = (int)((long)band * q.H2 / q.nb), r1 = (int)((long)(band + 1) * q.H2 / q.nb);
  if (r0 >= r1) return;
  const _Float16 * const xb = reinterpret_cast<const _Float16 *>(q.x.ptr) + (long)b * q.x.img;

  // ---- one-time set-up: zero pad columns of the input rows and of the ring, second conv's
  // weights into LDS (K 144 .. 167 zero)
  for (int e = tid; e < 2 * kSsInRows * 4; e += kSsThreads) {  // both buffers' rows
    const int lr = e >> 2, c = e & 3;
    const int col = c < 2 ? c : q.W0 + c;
    *reinterpret_cast<h4t *>(IN + lr * L.lw + ss_pcol(col)) = h4t{};
  }
  for (int e = tid; e < kSsRing * 2 * 2; e += kSsThreads) {  // slot, {column -1, column W1}, half
    const int slot = e >> 2, side = (e >> 1) & 1, hh = e & 1;
    const int cp = side ? q.W1 + 1 : 0;                  // ring column index c' = c + 1
    *reinterpret_cast<h8 *>(RING + slot * L.ring_row + (cp & 1) * L.plane + (cp >> 1) * kSsPS + 8 * hh) = h8{};
  }
  // ring offset of 8-channel half h of pixel pos within a plane
  auto rhalf = [](int pos, int h) __attribute__((always_inline)) { return pos * kSsPS + ((h ^ ((pos >> 3) & 1)) << 3); };
  for (int e = tid; e < 32 * (kSsLDW / 8); e += kSsThreads) {
    const int co = e / (kSsLDW / 8), k8 = (e - co * (kSsLDW / 8)) * 8;
    h8 v = h8{};
    if (co < q.C2 && k8 < 144) v = *reinterpret_cast<const h8 *>(reinterpret_cast<const _Float16 *>(q.w2) + (long)co * q.kpad2 + k8);
    *reinterpret_cast<h8 *>(W2s + co * kSsLDW + k8) = v;
  }

  // ---- input rows [base, base + 5) into registers / LDS (zeros outside the image)
  const int G = q.W0 >> 3;                                // 8-pixel groups per input row
  constexpr int UIT = 2;                                  // host: 5 * W0 / 8 <= 2 * 512
  h8 cin[UIT][3];
  auto load_in = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < UIT; ++i) {
      const int u = tid + kSsThreads * i;
      const int lr = u / G, g = u - lr * G;
      const int iy = base + lr;
      const bool ok = u < kSsInRows * G && iy >= 0 && iy < q.H0;
#pragma unroll
      for (int ci = 0; ci < 3; ++ci)
        cin[i][ci] = (ok && ci < q.Cin) ? *reinterpret_cast<const h8 *>(xb + (long)ci * q.x.cs + (long)iy * q.W0 + 8 * g) : h8{};
    }
  };
  auto store_in = [&](int buf) __attribute__((always_inline)) {  // buffer 0 / 1
#pragma unroll
    for (int i = 0; i < UIT; ++i) {
      const int u = tid + kSsThreads * i;
      if (u >= kSsInRows * G) continue;
      const int lr = u / G, g = u - lr * G;
      _Float16 * dst = lds + buf * L.in_sz + lr * L.lw + ss_pcol(8 * g + 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        h8 v;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          v[4 * h + 0] = cin[i][0][2 * j + h];
          v[4 * h + 1] = cin[i][1][2 * j + h];
          v[4 * h + 2] = cin[i][2][2 * j + h];
          v[4 * h + 3] = (_Float16)0.0f;
        }
        *reinterpret_cast<h8 *>(dst + 8 * j) = v;
      }
    }
  };

  // ---- stem: lane = pixel (lane & 15) of a 16-pixel block, K group kg = lane >> 4 (taps 2kg
  // and 2kg + 1; kg == 0 also tap 8 for the second MFMA); D = channels 4kg .. 4kg+3
  const int px = lane & 15, kg = lane >> 4;
  const _Float16 * W4 = reinterpret_cast<const _Float16 *>(q.w1);
  const h8 a1 = *reinterpret_cast<const h8 *>(W4 + px * 64 + 8 * kg);
  const h8 a2 = *reinterpret_cast<const h8 *>(W4 + px * 64 + 32 + 8 * kg);
  float sb[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) sb[v] = (q.b1 && 4 * kg + v < q.C1) ? q.b1[4 * kg + v] : 0.0f;
  // this lane's taps: 2kg, 2kg + 1 and 8 (row, column offsets of the 3x3 window)
  const int ty0 = (2 * kg) / 3, tx0 = (2 * kg) % 3, ty1 = (2 * kg + 1) / 3, tx1 = (2 * kg + 1) % 3;
  const int SB = (q.W1 + 15) >> 4;                        // 16-pixel stem blocks per row
  // stem row sr from the input rows in LDS buffer `buf`, whose first row is input row `base`:
  // this wave's blocks cb = blk0 + 8 i (at most three at 320 stem columns), issued together
  // so their LDS reads and MFMAs overlap; blocks past the row compute on a clamped block and
  // store nothing
  auto stem_row = [&](int sr, int buf, int base, int blk0) __attribute__((always_inline)) {
    constexpr int IT = 3;
    const int ring = L.ring_off + ((sr + kSsRing) % kSsRing) * L.ring_row;
    const _Float16 * const rb = lds + buf * L.in_sz + (2 * sr - 1 - base) * L.lw;
    f4t acc[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int ox = (blk0 + 8 * i) * 16 + px;
      // window corner: image column 2 ox - 1, staged column 2 ox + 1
      const int c0 = 2 * (ox < q.W1 ? ox : q.W1 - 1) + 1;
      const h4t t0 = *reinterpret_cast<const h4t *>(rb + ty0 * L.lw + ss_pcol(c0 + tx0));
      const h4t t1 = *reinterpret_cast<const h4t *>(rb + ty1 * L.lw + ss_pcol(c0 + tx1));
      // tap 8 feeds the second MFMA from K group 0 only; the other groups' weights there are
      // zero, so they read the same (finite or not, the same pixel's) values unmasked
      const h4t t8 = *reinterpret_cast<const h4t *>(rb + 2 * L.lw + ss_pcol(c0 + 2));
      h8 b1v, b2v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        b1v[e] = t0[e];
        b1v[4 + e] = t1[e];
        b2v[e] = t8[e];
        b2v[4 + e] = (_Float16)0.0f;
      }
      acc[i] = f4t{0.0f, 0.0f, 0.0f, 0.0f};
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1v, acc[i], 0, 0, 0);
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b2v, acc[i], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int cb = blk0 + 8 * i, ox = cb * 16 + px;
      h4t hv;
      // channels >= C1 have zero weights and zero bias (the packing's zero rows): act(0) = 0
#pragma unroll
      for (int v = 0; v < 4; ++v) hv[v] = (_Float16)act_fast<ACT1>(acc[i][v] + sb[v]);
      const int cp = ox + 1;
      if (cb < SB && ox < q.W1)
        *reinterpret_cast<h4t *>(lds + ring + (cp & 1) * L.plane + rhalf(cp >> 1, kg >> 1) + 4 * (kg & 1)) = hv;
    }
  };
  // a stem row outside the image: its ring slot is all zero
  auto zero_row = [&](int sr) __attribute__((always_inline)) {
    _Float16 * const ring = RING + ((sr + kSsRing) % kSsRing) * L.ring_row;
    for (int e = tid; e < L.ring_row / 8; e += kSsThreads) *reinterpret_cast<h8 *>(ring + 8 * e) = h8{};
  };

  // ---- second conv: blocks of 16 output pixels x 16 channels; lane = pixel (lane & 15), K
  // group kg: K slice s covers taps 2s + (kg >> 1), channels 8 (kg & 1) .. +7
  const int PB = (q.W2 + 15) >> 4, CB = (q.C2 + 15) >> 4, NBLK = PB * CB;
  float b2v[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int co = 16 * c + 4 * kg + v;
      b2v[c][v] = (q.b2 && co < q.C2) ? q.b2[co] : 0.0f;
    }
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      q.y.ptr, (short)0, (int)(((long)(q.batch - 1) * q.y.img + ((long)q.H2 * q.W2 - 1) * q.y.cs + q.C2) * 2), kBufDword3);
  // this wave's blocks blk = wave + 8 i (at most three at 160 columns and 32 channels), issued
  // together; blocks past the row compute on a clamped block and store nothing
  auto out_row = [&](int r) __attribute__((always_inline)) {
    constexpr int IT = 3;
    int rows[3];
#pragma unroll
    for (int ty = 0; ty < 3; ++ty) rows[ty] = L.ring_off + ((2 * r - 1 + ty + kSsRing) % kSsRing) * L.ring_row;
    f4t acc[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int blk = wave + 8 * i, blkc = blk < NBLK ? blk : NBLK - 1;
      const int pb = blkc % PB, cb = blkc / PB;
      const int ox = 16 * pb + px, oxc = ox < q.W2 ? ox : q.W2 - 1;
      const _Float16 * wa = W2s + (16 * cb + px) * kSsLDW + 8 * kg;
      acc[i] = f4t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 5; ++s) {
        // K slice 4's upper half is a tenth tap of zero weights: it reads tap 8's pixel again
        const int tap = min(2 * s + (kg >> 1), 8);
        const int ty = tap / 3, tx = tap - 3 * ty;
        const h8 fb = *reinterpret_cast<const h8 *>(lds + rows[ty] + (tx & 1) * L.plane + rhalf(oxc + (tx >> 1), kg & 1));
        const h8 fa = *reinterpret_cast<const h8 *>(wa + 32 * s);
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa, fb, acc[i], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int blk = wave + 8 * i;
      const int pb = blk % PB, cb = blk / PB;
      const int ox = 16 * pb + px, co = 16 * cb + 4 * kg;
      h4t hv;
#pragma unroll
      for (int v = 0; v < 4; ++v) hv[v] = (_Float16)act_fast<ACT2>(acc[i][v] + b2v[cb & 1][v]);
      const bool ok = blk < NBLK && ox < q.W2 && co < q.C2;
      const unsigned off = ok ? (unsigned)(((long)b * q.y.img + ((long)r * q.W2 + ox) * q.y.cs + co) * 2) : kBufOOB;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, hv), yr, off, 0, 0);
    }
  };

  // stem rows 2p and 2p+1 from input buffer p & 1 (input rows 4p-1 .. 4p+3); a row past the
  // stem's last is all zero; the second row's blocks start at wave 4, so a wave with a third
  // block of one row has two of the other
  auto stem_pair = [&](int pr) __attribute__((always_inline)) {
    stem_row(2 * pr, pr & 1, 4 * pr - 1, wave);
    if (2 * pr + 1 < q.H1) stem_row(2 * pr + 1, pr & 1, 4 * pr - 1, (wave + 4) & 7);
    else zero_row(2 * pr + 1);
  };

  // ---- prologue: stem row 2 r0 - 1 and rows 2 r0, 2 r0 + 1 into the ring; input rows of
  // pair r0 + 1 into LDS and of pair r0 + 2 into registers
  load_in(4 * r0 - 3);
  store_in((r0 + 1) & 1);
  load_in(4 * r0 - 1);
  store_in(r0 & 1);
  __syncthreads();
  if (2 * r0 - 1 >= 0) stem_row(2 * r0 - 1, (r0 + 1) & 1, 4 * r0 - 3, wave);
  else zero_row(2 * r0 - 1);
  stem_pair(r0);
  if (r0 + 1 < r1) load_in(4 * (r0 + 1) - 1);
  __syncthreads();  // the prologue's input rows consumed
  if (r0 + 1 < r1) store_in((r0 + 1) & 1);
  if (r0 + 2 < r1) load_in(4 * (r0 + 2) - 1);
  // ---- step r: stem rows of pair r + 1 (input buffer (r + 1) & 1, ring slots last read by
  // output row r - 1) and output row r (ring rows 2r-1 .. 2r+1); one barrier per step
  for (int r = r0; r < r1; ++r) {
    __syncthreads();  // ring rows 2r-1 .. 2r+1 and pair r + 1's input rows in LDS
    if (r + 1 < r1) stem_pair(r + 1);
    out_row(r);
    if (r + 2 < r1) store_in(r & 1);           // pair r + 2: its buffer's last reader was pair r
    if (r + 3 < r1) load_in(4 * (r + 3) - 1);
  }
}

// ---------------------------------------------------------------- host side

long stem_s2_lds_bytes(int W0, int W1) { return (long)stem_s2_lds(W0, W1).total * 2; }

bool stem_s2_supported(const StemS2Params & q)
{
  auto al = [](const void * p, int n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; };
  // C1 in (8, 16]: the second conv's packing has 16 channels per tap (k = tap * 16 + ci)
  return q.Cin >= 1 && q.Cin <= 3 && q.C1 > 8 && q.C1 <= 16 && q.C2 >= 4 && q.C2 <= 32 && q.C2 % 4 == 0 &&
         q.W0 % 8 == 0 && q.W0 <= kSsMaxW0 && q.H0 >= 2 && q.W0 >= 8 &&
         (q.W1 + 15) / 16 <= 24 && ((q.W2 + 15) / 16) * ((q.C2 + 15) / 16) <= 24 &&  // <= 3 blocks a wave
         q.H1 == (q.H0 - 1) / 2 + 1 && q.W1 == (q.W0 - 1) / 2 + 1 && q.H2 == (q.H1 - 1) / 2 + 1 &&
         q.W2 == (q.W1 - 1) / 2 + 1 && q.kpad2 >= 144 && kSsInRows * (q.W0 / 8) <= 2 * kSsThreads &&
         stem_s2_lds_bytes(q.W0, q.W1) <= 160 * 1024 && q.x.layout == kNCHW && q.y.layout == kNHWC &&
         (q.x.cs % 8) == 0 && (q.x.img % 8) == 0 && al(q.x.ptr, 16) && (q.y.cs % 4) == 0 && (q.y.img % 4) == 0 &&
         al(q.y.ptr, 8) && al(q.w1, 16) && al(q.w2, 16) && (q.kpad2 % 8) == 0 &&
         ((long)(q.batch - 1) * q.y.img + (long)q.H2 * q.W2 * q.y.cs) * 2 < (1L << 31);
}

// bands per image: one work-group per CU over the batch, at least one output row per band
int stem_s2_bands(int batch, int H2) { return std::max(1, std::min(H2, (256 + batch - 1) / batch)); }

template <int A1, int A2>
static void launch_ss(const StemS2Params & q, hipStream_t s)
{
  hipLaunchKernelGGL((conv_stem_s2_kernel<A1, A2>), dim3((unsigned)(q.batch * q.nb)), dim3(kSsThreads), 0, s, q);
}

bool stem_s2_act_ok(int a1, int a2) { return a1 == a2 && (a1 == kActSiLU || a1 == kActReLU || a1 == kActHSwish || a1 == kActNone); }

void launch_stem_s2(const StemS2Params & q, hipStream_t s)
{
  switch (q.act1) {
  case kActSiLU: launch_ss<kActSiLU, kActSiLU>(q, s); break;
  case kActReLU: launch_ss<kActReLU, kActReLU>(q, s); break;
  case kActHSwish: launch_ss<kActHSwish, kActHSwish>(q, s); break;
  default: launch_ss<kActNone, kActNone>(q, s); break;
  }
}

}  // namespace ivh
