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
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

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

void launch_conv_s2(const ConvParams & p, hipStream_t s)
{
  const int bc = conv_batch_chunk(p);
  if (bc < p.batch) {
    for (int b0 = 0; b0 < p.batch; b0 += bc) launch_conv_s2(conv_batch_slice(p, b0, std::min(bc, p.batch - b0)), s);
    return;
  }
  const dim3 grid((unsigned)s2_grid(p));
  switch (p.s2 - 1) {
  case 0: hipLaunchKernelGGL((conv3x3s2_kernel<16, 4, 1, 1, 600>), grid, dim3(256), 0, s, p); break;
  default: hipLaunchKernelGGL((conv3x3s2_kernel<16, 2, 2, 1, 400>), grid, dim3(256), 0, s, p); break;
  }
}

}  // namespace ivh
