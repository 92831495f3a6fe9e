// Batched matrix product on gfx950 fp16 MFMA (v_mfma_f32_32x32x16_f16), fp32 accumulate:
// the reference's bmm (kernels/ops.cl:276-294, dispatch src/PlanModel.cpp:3935-3990), used by
// the YOLO11n C2PSA attention (q^T k over 400 tokens, v attn^T).
//
//   Y[bb][m][n] = sum_k A[bb][m][k] * B[bb][k][n]     per image, one rounding to fp16
//
// Either operand may be stored transposed -- A as [K][M] (TA), B as [N][K] (TB) -- which is
// how a permute of the last two dimensions feeding the product is folded away.  Tiles of
// 64 x 128 outputs, K steps of 32 staged in LDS as [row][k] (k contiguous: the MFMA fragment
// layout); an operand whose k is contiguous in memory is copied with 16-byte loads, the
// other is transposed on the way into LDS.  The output tile is staged in LDS and written
// as 16-byte row pieces.
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
constexpr int kBM = 64, kBN = 128, kBK = 32, kLDK = kBK + 8, kLDY = kBN + 8;

// 8 consecutive elements p[0..7] with bound `lim` (elements past it are zero); vector
// load when the whole piece is in range and 16-byte aligned.
__device__ __forceinline__ h8 load8(const _Float16 * p, int lim, bool vec)
{
  if (vec && lim >= 8) return *reinterpret_cast<const h8 *>(p);
  h8 v = h8{};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < lim) v[e] = p[e];
  return v;
}
}  // namespace

template <int TA, int TB>
__global__ void __launch_bounds__(256) bmm_mfma_kernel(const SmallParams q)
{
  using F = Mf<32>;
  __shared__ __attribute__((aligned(16))) _Float16 As[kBM * kLDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kBN * kLDK];
  __shared__ __attribute__((aligned(16))) _Float16 Ys[kBM * kLDY];
  const int BB = q.i0, M = q.i1, K = q.i2, N = q.i3;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;   // 2 x 2 waves: 32 rows x 64 columns each
  const int z = blockIdx.z, img = z / BB, hb = z - img * BB;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const _Float16 * A = reinterpret_cast<const _Float16 *>(q.a.ptr) + (long)img * q.a.img + (long)hb * M * K;
  const _Float16 * B = reinterpret_cast<const _Float16 *>(q.b.ptr) + (long)img * q.b.img + (long)hb * K * N;
  _Float16 * Y = reinterpret_cast<_Float16 *>(q.y.ptr) + (long)img * q.y.img + (long)hb * M * N;
  // 16-byte loads need the piece's start aligned: rows of the k-contiguous (or the
  // transposed) layout have a length that is a multiple of 8 and an aligned base
  const bool va = ((reinterpret_cast<uintptr_t>(A) & 15) == 0) && ((TA ? M : K) % 8 == 0);
  const bool vb = ((reinterpret_cast<uintptr_t>(B) & 15) == 0) && ((TB ? K : N) % 8 == 0);

  F::acc_t acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < F::NV; ++v) acc[t][v] = 0.0f;

  for (int k0 = 0; k0 < K; k0 += kBK) {
    __syncthreads();  // the previous step's fragments are read
    // A tile -> As[m][k]: 64 x 32 = 256 pieces of 8
    {
      if (!TA) {  // A [M][K]: piece = 8 consecutive k of one row
        const int r = tid >> 2, kq = (tid & 3) * 8, m = m0 + r, k = k0 + kq;
        const h8 v = m < M ? load8(A + (long)m * K + k, K - k, va) : h8{};
        *reinterpret_cast<h8 *>(As + r * kLDK + kq) = v;
      } else {    // A [K][M]: piece = 8 consecutive m of one k, transposed into As
        const int kk = tid >> 3, m8 = (tid & 7) * 8, k = k0 + kk, m = m0 + m8;
        const h8 v = k < K ? load8(A + (long)k * M + m, M - m, va) : h8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) As[(m8 + e) * kLDK + kk] = v[e];
      }
    }
    // B tile -> Bs[n][k]: 128 x 32 = 512 pieces, two per thread
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i;
      if (TB) {   // B [N][K]: piece = 8 consecutive k of one column
        const int r = e >> 2, kq = (e & 3) * 8, n = n0 + r, k = k0 + kq;
        const h8 v = n < N ? load8(B + (long)n * K + k, K - k, vb) : h8{};
        *reinterpret_cast<h8 *>(Bs + r * kLDK + kq) = v;
      } else {    // B [K][N]: piece = 8 consecutive n of one k, transposed into Bs
        const int kk = e >> 4, n8 = (e & 15) * 8, k = k0 + kk, n = n0 + n8;
        const h8 v = k < K ? load8(B + (long)k * N + n, N - n, vb) : h8{};
#pragma unroll
        for (int t = 0; t < 8; ++t) Bs[(n8 + t) * kLDK + kk] = v[t];
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kBK / 16; ++j) {
      const h8 fa = *reinterpret_cast<const h8 *>(As + (wm * 32 + (lane & 31)) * kLDK + j * 16 + F::kq(lane));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const h8 fb = *reinterpret_cast<const h8 *>(Bs + (wn * 64 + t * 32 + (lane & 31)) * kLDK + j * 16 + F::kq(lane));
        acc[t] = F::mma(fa, fb, acc[t]);
      }
    }
  }
  // D: lane holds column n = lane%32 of its block, rows m = F::row(lane, v)
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int v = 0; v < F::NV; ++v)
      Ys[(wm * 32 + F::row(lane, v)) * kLDY + wn * 64 + t * 32 + (lane & 31)] = (_Float16)acc[t][v];
  __syncthreads();
  const bool vy = ((reinterpret_cast<uintptr_t>(Y) & 15) == 0) && (N % 8 == 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid + 256 * i;
    const int r = e >> 4, n8 = (e & 15) * 8, m = m0 + r, n = n0 + n8;
    if (m >= M || n >= N) continue;
    const h8 v = *reinterpret_cast<const h8 *>(Ys + r * kLDY + n8);
    _Float16 * yp = Y + (long)m * N + n;
    if (vy && n + 8 <= N) *reinterpret_cast<h8 *>(yp) = v;
    else
      for (int c = 0; c < 8 && n + c < N; ++c) yp[c] = v[c];
  }
}

// q.op bit 0: A stored [K][M]; bit 1: B stored [N][K]
void launch_bmm_mfma(const SmallParams & q, hipStream_t s)
{
  const dim3 grid((unsigned)((q.i3 + kBN - 1) / kBN), (unsigned)((q.i1 + kBM - 1) / kBM), (unsigned)(q.batch * q.i0));
  switch (q.op & 3) {
  case 0: hipLaunchKernelGGL((bmm_mfma_kernel<0, 0>), grid, dim3(256), 0, s, q); break;
  case 1: hipLaunchKernelGGL((bmm_mfma_kernel<1, 0>), grid, dim3(256), 0, s, q); break;
  case 2: hipLaunchKernelGGL((bmm_mfma_kernel<0, 1>), grid, dim3(256), 0, s, q); break;
  default: hipLaunchKernelGGL((bmm_mfma_kernel<1, 1>), grid, dim3(256), 0, s, q); break;
  }
}

}  // namespace ivh
