// Pointwise (1x1, stride 1) convolution with Cout <= 128 on gfx950 fp16 MFMA, streaming.
//
// Replaces, for the channels-last 1x1 convs of the C2f / C3k2 blocks and the heads, the
// reference's conv1x1 / gemm kernels (kernels/conv1x1.cl, gemm.cl:468-472, 644-650;
// dispatch src/PlanModel.cpp:3688-3933):
//   y[p][co] = act(sum_ci W[co][ci] x[p][ci] + b[co])
// At Cout <= 128 these layers carry 1-4 bytes of HBM traffic per FLOP: the bound is HBM, and
// the kernel is built to keep the HBM stream full rather than to stage tiles:
//   * the work-group's weights [32 CB][K] and bias sit in LDS, loaded once per launch;
//   * every wave is an independent stream over 32-pixel blocks (grid-stride over the
//     batch's pixels): the MFMA B fragment of a block -- pixel (lane & 31), channels
//     8 (lane / 32) .. +7 of a 16-channel K slice -- is one 16-byte load straight from the
//     NHWC input into registers, so there is no LDS staging and no barrier after the first;
//   * the K dimension runs in chunks of NSL 16-channel slices (2 for 32 input channels, 3
//     for 48, else 4), and the loads of the next R - 1 (block, chunk) steps are in flight
//     while one is multiplied (an R-deep register ring: 5, 4 or 3 steps for 2, 3 or 4
//     slices), which keeps 4-8 KB per wave in flight;
//   * epilogue in registers: bias + activation in fp32, one fp16 rounding, a permlane32 swap
//     so each lane holds 8 consecutive channels of its pixel, 16-byte stores.
// Weight rows in LDS have a pitch of an odd number of 16-byte slots, so the A fragments
// (32 rows x 16 bytes per half-wave) are bank-conflict free.
#include <algorithm>
#include <map>
#include <mutex>

#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef unsigned u2q __attribute__((ext_vector_type(2)));
typedef unsigned u4q __attribute__((ext_vector_type(4)));
constexpr int kPwCUs = 256;
constexpr int kPwMaxK = 512;
}  // namespace

struct PwGeom {
  int nch;       // K chunks of 16 NSL channels
  int ldw;       // LDS weight row pitch (halves) = 16 NSL nch + 8
  long nblk;     // 32-pixel blocks of the batch
  FastDiv d_hw;  // division by H * W
};

template <int CB, int NSL, int R, int ACT>
__global__ void __launch_bounds__(256, 2) conv1x1_pw_kernel(const ConvParams p, const PwGeom g)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  extern __shared__ __align__(16) unsigned char pw_lds[];
  _Float16 * const Ws = reinterpret_cast<_Float16 *>(pw_lds);                      // [32 CB][ldw]
  float * const Bs = reinterpret_cast<float *>(pw_lds + (size_t)CB * 32 * g.ldw * 2);  // [32 CB]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int KC = 16 * NSL;  // channels per chunk
  const int KP = KC * g.nch;

  // weights [32 CB][KP] (zero past Cout and past cin8) and bias, once per launch
  {
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(p.w), (short)0, CB * 32 * p.kpad * 2, kBufDword3);
    const int wq = KP / 8, n = CB * 32 * wq;
    for (int e = tid; e < n; e += 256) {
      const int row = e / wq, q = e - row * wq;
      const bool ok = row < p.Cout && q * 8 < p.cin8;
      const h8 v = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
          wr, ok ? (unsigned)((row * p.kpad + q * 8) * 2) : kBufOOB, 0, 0));
      *reinterpret_cast<h8 *>(Ws + row * g.ldw + q * 8) = v;
    }
    if (tid < CB * 32) Bs[tid] = p.bias && tid < p.Cout ? p.bias[tid] : 0.0f;
  }
  __syncthreads();

  const long M = (long)p.batch * p.H * p.W;
  const long x_last = (long)(p.batch - 1) * p.x.img + ((long)p.H * p.W - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const long y_last = (long)(p.batch - 1) * p.y.img + ((long)p.H * p.W - 1) * p.y.cs + (p.Cout + 7) / 8 * 8;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);

  const long nw = (long)gridDim.x * 4, w0 = (long)blockIdx.x * 4 + wave;
  const long my_blocks = w0 < g.nblk ? (g.nblk - 1 - w0) / nw + 1 : 0;
  const long nsteps = my_blocks * g.nch;
  const int kq = F::kq(lane);
  const unsigned hw_n = (unsigned)(p.H * p.W);

  // byte offset of the lane's pixel of block blk (kBufOOB past the batch)
  auto pix_off = [&](long blk) __attribute__((always_inline)) {
    const long px = blk * 32 + (lane & 31);
    if (px >= M) return kBufOOB;
    const unsigned img = fastdiv((unsigned)px, g.d_hw), hw = (unsigned)px - img * hw_n;
    return (img * (unsigned)p.x.img + hw * (unsigned)p.x.cs) * 2u;
  };
  // loads of step s (block w0 + (s / nch) nw, chunk s % nch): NSL 16-channel slices
  auto load = [&](long s, h8 (&b)[NSL]) __attribute__((always_inline)) {
    const long blk = w0 + (s / g.nch) * nw;
    const int ch = (int)(s % g.nch);
    const unsigned po = s < nsteps ? pix_off(blk) : kBufOOB;
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      const int k = ch * KC + sl * 16 + kq;
      const unsigned off = po == kBufOOB || k >= p.cin8 ? kBufOOB : po + (unsigned)k * 2u;
      b[sl] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    }
  };
  // Cin not a multiple of 8: the channels of the last 8-channel piece past Cin (a channels-
  // last view's padding, which need not hold finite values) are zeroed bitwise
  auto mask_ragged = [&](long s, h8 (&b)[NSL]) __attribute__((always_inline)) {
    const int ch = (int)(s % g.nch);
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
      const int k = ch * KC + sl * 16 + kq;
      if (k < p.Cin && k + 8 > p.Cin) {
        u16x8 keep;
#pragma unroll
        for (int e = 0; e < 8; ++e) keep[e] = k + e < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
        b[sl] = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, b[sl]) & keep);
      }
    }
  };
  const bool ragged = p.Cin != p.cin8;

  acc_t acc[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  const int arow = (lane & 31) * g.ldw + kq;

  auto epilogue = [&](long blk) __attribute__((always_inline)) {
    const long px = blk * 32 + (lane & 31);
    unsigned yo = kBufOOB;
    if (px < M) {
      const unsigned img = fastdiv((unsigned)px, g.d_hw), hw = (unsigned)px - img * hw_n;
      yo = (img * (unsigned)p.y.img + hw * (unsigned)p.y.cs) * 2u;
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      auto vals = [&](int v4) __attribute__((always_inline)) {
        const float4 bv = *reinterpret_cast<const float4 *>(Bs + c * 32 + F::row(lane, v4));
        float o4[4] = {act_fast<ACT>(acc[c][v4] + bv.x), act_fast<ACT>(acc[c][v4 + 1] + bv.y),
                       act_fast<ACT>(acc[c][v4 + 2] + bv.z), act_fast<ACT>(acc[c][v4 + 3] + bv.w)};
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
        // c+12..c+15): swapped so every lane holds 8 consecutive channels of its pixel
        const u2q lo = __builtin_bit_cast(u2q, vals(v4));
        const u2q hi = __builtin_bit_cast(u2q, vals(v4 + 4));
        const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], hi[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], hi[1], false, false);
        const u4q q = {s0[0], s1[0], s0[1], s1[1]};
        const int ch = c * 32 + F::row(lane, v4) - 4 * (lane >> 5) + 8 * (lane >> 5);
        if (ch + 8 <= p.Cout || (ch < p.Cout && p.ypad >= ch + 8 - p.Cout)) {
          __builtin_amdgcn_raw_buffer_store_b128(q, yr, yo == kBufOOB ? kBufOOB : yo + (unsigned)ch * 2u, 0, 0);
        } else if (ch < p.Cout && yo != kBufOOB) {  // ragged last piece: the channels below Cout
          const h8 hv = __builtin_bit_cast(h8, q);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (ch + e < p.Cout)
              __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, hv[e]), yr,
                                                    yo + (unsigned)(ch + e) * 2u, 0, 0);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
    }
  };
  auto step = [&](long s, h8 (&b)[NSL]) __attribute__((always_inline)) {
    if (ragged) mask_ragged(s, b);
    const int ch = (int)(s % g.nch);
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const h8 fa = *reinterpret_cast<const h8 *>(Ws + c * 32 * g.ldw + arow + ch * KC + sl * 16);
        acc[c] = F::mma(fa, b[sl], acc[c]);
      }
    if (ch == g.nch - 1) epilogue(w0 + (s / g.nch) * nw);
  };

  // R-deep ring: step s in registers, s + 1 .. s + R - 1 in flight
  h8 b[R][NSL];
#pragma unroll
  for (int i = 0; i < R - 1; ++i) load(i, b[i]);
  for (long s = 0; s < nsteps; s += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (s + j >= nsteps) break;
      load(s + j + R - 1, b[(j + R - 1) % R]);
      step(s + j, b[j]);
    }
  }
}

// Planar-output variant: y in NCHW channel planes (the plan's graph outputs, the heads'
// concat planes), x in NCHW planes (XT) or channels-last, Cin <= 64 and Cout <= 128 (NCB
// 32-channel blocks), the whole K range in one step.  The MFMA computes the transpose,
// D[pixel][co] = x^T W^T (operand A the pixel fragment, operand B the weight fragment), so a
// lane's accumulators are 4-pixel runs of its own channel plane; after the permlane32 swap a
// lane holds 8 consecutive pixels of one plane and writes them as one 16-byte store.  With
// XT a wave loads its block's 32 pixels as 16-byte pieces along the channel planes (8 pixels
// of one channel, lane / 4 the channel, lane % 4 the piece) and transposes them through its
// own LDS rows [pixel][channel] (pitch an odd number of 16-byte slots, as the weights), from
// which the pixel fragments are read; LDS operations of one wave complete in order, so the
// rows need no barrier, only a fence that keeps the compiler from reordering them.
template <int NCB, int NSL, int ACT, bool XT>
__global__ void __launch_bounds__(256, 2) conv1x1_pwt_kernel(const ConvParams p, const PwGeom g)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  constexpr int KP = 16 * NSL;   // K, zero padded
  constexpr int LDW = KP + 8;    // weight and pixel row pitch (halves)
  constexpr int R = 3;           // register ring: block s in use, s + 1 and s + 2 in flight
  extern __shared__ __align__(16) unsigned char pw_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  _Float16 * const Ws = reinterpret_cast<_Float16 *>(pw_lds);                         // [32 NCB][LDW]
  float * const Bs = reinterpret_cast<float *>(Ws + 32 * NCB * LDW);                   // [32 NCB]
  _Float16 * const Ts = reinterpret_cast<_Float16 *>(Bs + 32 * NCB) + wave * 32 * LDW;  // XT: [32][LDW]

  {
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half *>(p.w), (short)0, NCB * 32 * p.kpad * 2, kBufDword3);
    constexpr int wq = KP / 8, n = NCB * 32 * wq;
    for (int e = tid; e < n; e += 256) {
      const int row = e / wq, q = e - row * wq;
      const bool ok = row < p.Cout && q * 8 < p.cin8;
      const h8 v = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(
          wr, ok ? (unsigned)((row * p.kpad + q * 8) * 2) : kBufOOB, 0, 0));
      *reinterpret_cast<h8 *>(Ws + row * LDW + q * 8) = v;
    }
    if (tid < NCB * 32) Bs[tid] = p.bias && tid < p.Cout ? p.bias[tid] : 0.0f;
  }
  __syncthreads();

  const long M = (long)p.batch * p.H * p.W;
  const unsigned hw_n = (unsigned)(p.H * p.W);
  const long x_last = XT ? (long)(p.batch - 1) * p.x.img + (long)(p.Cin - 1) * p.x.cs + hw_n
                         : (long)(p.batch - 1) * p.x.img + ((long)hw_n - 1) * p.x.cs + p.cin8;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<__half *>(p.x.ptr), (short)0, (int)(x_last * 2), kBufDword3);
  const long y_last = (long)(p.batch - 1) * p.y.img + (long)(p.Cout - 1) * p.y.cs + hw_n;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(p.y.ptr, (short)0, (int)(y_last * 2), kBufDword3);

  const long nw = (long)gridDim.x * 4, w0 = (long)blockIdx.x * 4 + wave;
  const long nsteps = w0 < g.nblk ? (g.nblk - 1 - w0) / nw + 1 : 0;
  const int kq = F::kq(lane);

  // loads of block w0 + s nw: XT, NSL pieces (channel 16 j + lane / 4, pixels 8 (lane % 4) ..
  // + 7); channels-last, the NSL pixel fragments (pixel lane % 32, channels 16 j + kq ..)
  auto load = [&](long s, h8 (&b)[NSL]) __attribute__((always_inline)) {
    const long blk = w0 + s * nw;
    if (XT) {
      const long px = blk * 32 + (lane & 3) * 8;
      unsigned po = kBufOOB;
      if (s < nsteps && px < M) {
        const unsigned img = fastdiv((unsigned)px, g.d_hw), hw = (unsigned)px - img * hw_n;
        po = (img * (unsigned)p.x.img + hw) * 2u;
      }
#pragma unroll
      for (int j = 0; j < NSL; ++j) {
        const int ci = 16 * j + (lane >> 2);
        const unsigned off = po == kBufOOB || ci >= p.Cin ? kBufOOB : po + (unsigned)ci * (unsigned)p.x.cs * 2u;
        b[j] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
    } else {
      const long px = blk * 32 + (lane & 31);
      unsigned po = kBufOOB;
      if (s < nsteps && px < M) {
        const unsigned img = fastdiv((unsigned)px, g.d_hw), hw = (unsigned)px - img * hw_n;
        po = (img * (unsigned)p.x.img + hw * (unsigned)p.x.cs) * 2u;
      }
#pragma unroll
      for (int j = 0; j < NSL; ++j) {
        const int k = 16 * j + kq;
        const unsigned off = po == kBufOOB || k >= p.cin8 ? kBufOOB : po + (unsigned)k * 2u;
        b[j] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
      }
    }
  };
  const bool ragged = !XT && p.Cin != p.cin8;

  auto step = [&](long s, h8 (&b)[NSL]) __attribute__((always_inline)) {
    const long blk = w0 + s * nw;
    h8 xf[NSL];
    if (XT) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the previous block's reads first
      const int r0 = (lane & 3) * 8, c0 = lane >> 2;
#pragma unroll
      for (int j = 0; j < NSL; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) Ts[(r0 + e) * LDW + 16 * j + c0] = b[j][e];
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");  // the rows before the fragment reads
#pragma unroll
      for (int j = 0; j < NSL; ++j) xf[j] = *reinterpret_cast<const h8 *>(Ts + (lane & 31) * LDW + 16 * j + kq);
    } else {
#pragma unroll
      for (int j = 0; j < NSL; ++j) {
        xf[j] = b[j];
        const int k = 16 * j + kq;
        if (ragged && k < p.Cin && k + 8 > p.Cin) {
          u16x8 keep;
#pragma unroll
          for (int e = 0; e < 8; ++e) keep[e] = k + e < p.Cin ? (unsigned short)0xffff : (unsigned short)0;
          xf[j] = __builtin_bit_cast(h8, __builtin_bit_cast(u16x8, xf[j]) & keep);
        }
      }
    }
    // output pixels of the lane after the swap: 16 pr + 8 (lane / 32) .. + 7, pr = 0, 1
    unsigned yo[2];
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      const long px = blk * 32 + 16 * pr + 8 * (lane >> 5);
      yo[pr] = kBufOOB;
      if (px < M) {
        const unsigned img = fastdiv((unsigned)px, g.d_hw), hw = (unsigned)px - img * hw_n;
        yo[pr] = (img * (unsigned)p.y.img + hw) * 2u;
      }
    }
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      acc_t acc;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
      const int co = cb * 32 + (lane & 31);
#pragma unroll
      for (int j = 0; j < NSL; ++j) {
        const h8 wf = *reinterpret_cast<const h8 *>(Ws + co * LDW + 16 * j + kq);
        acc = F::mma(xf[j], wf, acc);
      }
      const float bco = Bs[co];
      auto vals = [&](int v4) __attribute__((always_inline)) {
        float o4[4] = {act_fast<ACT>(acc[v4] + bco), act_fast<ACT>(acc[v4 + 1] + bco),
                       act_fast<ACT>(acc[v4 + 2] + bco), act_fast<ACT>(acc[v4 + 3] + bco)};
        h4 hv;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          __asm__("" : "+v"(o4[q]));  // fp32 result, then one fp16 rounding
          hv[q] = (_Float16)o4[q];
        }
        return hv;
      };
      const unsigned cofs = (unsigned)co * (unsigned)p.y.cs * 2u;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        // pixel runs 16 pr + 4 (lane / 32) .. (v4 = 8 pr) and 16 pr + 8 + 4 (lane / 32) ..
        // (v4 + 4): swapped so a lane holds pixels 16 pr + 8 (lane / 32) .. + 7 of plane co
        const u2q lo = __builtin_bit_cast(u2q, vals(8 * pr));
        const u2q hi = __builtin_bit_cast(u2q, vals(8 * pr + 4));
        const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], hi[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], hi[1], false, false);
        const u4q q = {s0[0], s1[0], s0[1], s1[1]};
        const unsigned off = yo[pr] == kBufOOB || co >= p.Cout ? kBufOOB : yo[pr] + cofs;
        __builtin_amdgcn_raw_buffer_store_b128(q, yr, off, 0, 0);
      }
    }
  };

  h8 b[R][NSL];
#pragma unroll
  for (int i = 0; i < R - 1; ++i) load(i, b[i]);
  for (long s = 0; s < nsteps; s += R) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (s + j >= nsteps) break;
      load(s + j + R - 1, b[(j + R - 1) % R]);
      step(s + j, b[j]);
    }
  }
}

// ---------------------------------------------------------------- host side

size_t pw_lds_bytes(const ConvParams & p);

bool pw_views_ok(const ConvParams & p)
{
  auto nhwc16 = [](const View & v) {
    return v.layout == kNHWC && v.cs % 8 == 0 && v.img % 8 == 0 && (reinterpret_cast<uintptr_t>(v.ptr) % 16) == 0;
  };
  if (!nhwc16(p.x) || !nhwc16(p.y) || p.r.ptr || p.xt) return false;
  const long HW = (long)p.H * p.W;
  const long x_last = (long)(p.batch - 1) * p.x.img + (HW - 1) * p.x.cs + p.cin8;
  const long y_last = (long)(p.batch - 1) * p.y.img + (HW - 1) * p.y.cs + (p.Cout + 7) / 8 * 8;
  return x_last * 2 < (1L << 31) && y_last * 2 < (1L << 31) && (long)p.batch * HW < (1L << 31) &&
         p.x.img * 2 < (1L << 31) && p.y.img * 2 < (1L << 31);
}

bool pw_plan(const ConvParams & p)
{
  const bool act_ok = p.act == kActNone || p.act == kActSiLU || p.act == kActReLU || p.act == kActHSwish;
  return p.K == 1 && p.S == 1 && p.P == 0 && p.G == 1 && p.H == p.Ho && p.W == p.Wo && act_ok && p.Cout <= 128 &&
         p.cin8 <= kPwMaxK && p.kpad >= p.cin8 && pw_lds_bytes(p) <= 65536 && pw_views_ok(p);
}

long pw_blocks(const ConvParams & p) { return ((long)p.batch * p.H * p.W + 31) / 32; }

// 32-channel output blocks per wave: 1, 2 or 4
int pw_cb(const ConvParams & p) { return p.Cout > 64 ? 4 : (p.Cout > 32 ? 2 : 1); }

// K slices per chunk: 2 for up to 32 input channels, 3 for 48, else 4
int pw_nsl(const ConvParams & p) { return p.cin8 <= 32 ? 2 : (p.cin8 == 48 ? 3 : 4); }

size_t pw_lds_bytes(const ConvParams & p)
{
  const int cb = pw_cb(p), kc = 16 * pw_nsl(p), nch = (p.cin8 + kc - 1) / kc;
  return (size_t)cb * 32 * (kc * nch + 8) * 2 + (size_t)cb * 32 * 4;
}

// Persistent grid: as many work-groups as fit on the CUs at once (registers and LDS, from
// the runtime's occupancy query, kept per kernel and LDS size), no more than the blocks need.
template <int CB, int NSL, int ACT>
static void launch_pw_act(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  const size_t lds = pw_lds_bytes(p);
  static std::mutex mu;
  static std::map<size_t, int> occ;
  int per_cu = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = occ.find(lds);
    if (it == occ.end()) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv1x1_pw_kernel<CB, NSL, 7 - NSL, ACT>, 256, lds) !=
              hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      occ.emplace(lds, per_cu);
    } else {
      per_cu = it->second;
    }
  }
  const long wgs = std::min<long>((g.nblk + 3) / 4, (long)per_cu * kPwCUs);
  hipLaunchKernelGGL((conv1x1_pw_kernel<CB, NSL, 7 - NSL, ACT>), dim3((unsigned)wgs), dim3(256), lds, s, p, g);
}

template <int CB, int NSL>
static void launch_pw_nsl(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  switch (p.act) {
  case kActSiLU: launch_pw_act<CB, NSL, kActSiLU>(p, g, s); break;
  case kActReLU: launch_pw_act<CB, NSL, kActReLU>(p, g, s); break;
  case kActHSwish: launch_pw_act<CB, NSL, kActHSwish>(p, g, s); break;
  default: launch_pw_act<CB, NSL, kActNone>(p, g, s); break;
  }
}

template <int CB>
static void launch_pw_cb(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  switch (pw_nsl(p)) {
  case 2: launch_pw_nsl<CB, 2>(p, g, s); break;
  case 3: launch_pw_nsl<CB, 3>(p, g, s); break;
  default: launch_pw_nsl<CB, 4>(p, g, s); break;
  }
}

// ---- planar-output variant

static int pwt_ncb(const ConvParams & p) { return p.Cout <= 64 ? 2 : 4; }
static int pwt_nsl(const ConvParams & p) { return p.cin8 <= 32 ? 2 : 4; }

bool pwt_views_ok(const ConvParams & p)
{
  const long HW = (long)p.H * p.W;
  const View & x = p.x, & y = p.y;
  if (p.r.ptr || HW % 8) return false;
  if (y.layout != kNCHW || y.cs % 8 || y.cs < HW || y.img % 8 || (reinterpret_cast<uintptr_t>(y.ptr) % 16)) return false;
  if (p.xt) {
    if (x.layout != kNCHW || x.cs % 8 || x.cs < HW || x.img % 8 || (reinterpret_cast<uintptr_t>(x.ptr) % 16)) return false;
  } else if (x.layout != kNHWC || x.cs % 8 || x.img % 8 || (reinterpret_cast<uintptr_t>(x.ptr) % 16)) {
    return false;
  }
  const long x_last = p.xt ? (long)(p.batch - 1) * x.img + (long)(p.Cin - 1) * x.cs + HW
                           : (long)(p.batch - 1) * x.img + (HW - 1) * x.cs + p.cin8;
  const long y_last = (long)(p.batch - 1) * y.img + (long)(p.Cout - 1) * y.cs + HW;
  return x_last * 2 < (1L << 31) && y_last * 2 < (1L << 31) && (long)p.batch * HW < (1L << 31) &&
         x.img * 2 < (1L << 31) && y.img * 2 < (1L << 31) && (long)x.cs * 64 * 2 < (1L << 31) &&
         (long)y.cs * 128 * 2 < (1L << 31);
}

size_t pwt_lds_bytes(const ConvParams & p)
{
  const int ncb = pwt_ncb(p), ldw = 16 * pwt_nsl(p) + 8;
  return (size_t)ncb * 32 * ldw * 2 + (size_t)ncb * 32 * 4 + (p.xt ? (size_t)4 * 32 * ldw * 2 : 0);
}

bool pwt_plan(const ConvParams & p)
{
  const bool act_ok = p.act == kActNone || p.act == kActSiLU || p.act == kActReLU || p.act == kActHSwish;
  return p.K == 1 && p.S == 1 && p.P == 0 && p.G == 1 && p.H == p.Ho && p.W == p.Wo && act_ok && p.Cout >= 1 &&
         p.Cout <= 128 && p.Cin <= 64 && p.cin8 <= 64 && p.kpad >= p.cin8 && pwt_views_ok(p);
}

template <int NCB, int NSL, int ACT, bool XT>
static void launch_pwt_act(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  const size_t lds = pwt_lds_bytes(p);
  static int per_cu = 0;
  static std::once_flag once;
  std::call_once(once, [&] {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv1x1_pwt_kernel<NCB, NSL, ACT, XT>, 256, lds) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
  });
  const long wgs = std::min<long>((g.nblk + 3) / 4, (long)per_cu * kPwCUs);
  hipLaunchKernelGGL((conv1x1_pwt_kernel<NCB, NSL, ACT, XT>), dim3((unsigned)wgs), dim3(256), lds, s, p, g);
}

template <int NCB, int NSL, bool XT>
static void launch_pwt_nsl(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  switch (p.act) {
  case kActSiLU: launch_pwt_act<NCB, NSL, kActSiLU, XT>(p, g, s); break;
  case kActReLU: launch_pwt_act<NCB, NSL, kActReLU, XT>(p, g, s); break;
  case kActHSwish: launch_pwt_act<NCB, NSL, kActHSwish, XT>(p, g, s); break;
  default: launch_pwt_act<NCB, NSL, kActNone, XT>(p, g, s); break;
  }
}

template <bool XT>
static void launch_pwt_xt(const ConvParams & p, const PwGeom & g, hipStream_t s)
{
  const int ncb = pwt_ncb(p), nsl = pwt_nsl(p);
  if (ncb == 2 && nsl == 2) launch_pwt_nsl<2, 2, XT>(p, g, s);
  else if (ncb == 2) launch_pwt_nsl<2, 4, XT>(p, g, s);
  else if (nsl == 2) launch_pwt_nsl<4, 2, XT>(p, g, s);
  else launch_pwt_nsl<4, 4, XT>(p, g, s);
}

void launch_conv_pw(const ConvParams & p, hipStream_t s)
{
  PwGeom g;
  const int kc = 16 * pw_nsl(p);
  g.nch = (p.cin8 + kc - 1) / kc;
  g.ldw = kc * g.nch + 8;
  g.nblk = pw_blocks(p);
  g.d_hw = fastdiv_make((unsigned)(p.H * p.W));
  if (p.pw == 2) {
    if (p.xt) launch_pwt_xt<true>(p, g, s);
    else launch_pwt_xt<false>(p, g, s);
    return;
  }
  if (p.Cout > 64) launch_pw_cb<4>(p, g, s);
  else if (p.Cout > 32) launch_pw_cb<2>(p, g, s);
  else launch_pw_cb<1>(p, g, s);
}

}  // namespace ivh
