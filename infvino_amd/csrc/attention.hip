// Fused attention core of ultralytics' Attention (the C2PSA block of YOLO11, position-
// sensitive attention over the H*W tokens of a 20x20 map) on gfx950 fp16 MFMA.
//
// The plan spells it as four nodes (scripts/onnx2plan.py lowering; kernels ops.cl:276-294
// bmm and ops.cl:181-197 softmax in the reference):
//   S = q^T k          bmm, per head [N x kd] x [kd x N], fp32 accumulation, fp16 store
//   T = S * scale      ew_binary mul by a scalar init, fp32, fp16 store
// (ultralytics 8.4 exports scale q^T instead, before the product: T = (q^T scale) k; the
// kernel takes either form, AttnParams::scale_q)
//   P = softmax(T)     over the last axis: m = max, s = sum exp(T - m), fp16(exp(T - m) / s)
//   O = v P^T          bmm, per head [hd x N] x [N x N]^T, fp32 accumulation, fp16 store
// which moves the N x N score matrix through HBM five times.  Here one work-group owns an
// (image, head, 128 queries) triple: k (transposed to key rows), v and the queries' q
// (transposed to query rows) are staged in LDS once; each wave computes S^T = k^T q for its 32
// queries with v_mfma_f32_32x32x16_f16 (A = 32 keys x 16 channels, B = 16 channels x 32
// queries), so a lane holds one query's scores for 16 of every 32 keys and the row max and
// sum are lane-local plus one exchange with the partner lane (lane ^ 32).  The fp16 rounding
// points of the four nodes are kept (S, T and P are rounded to fp16 where the nodes store),
// and the probabilities go from the score registers straight into the B operand of the P v^T
// MFMAs: v_permlane32_swap turns the two 4-key runs a lane holds of a 16-key slice (and the
// two its partner holds) into the 8 consecutive keys of the B-fragment layout.
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef unsigned u2v __attribute__((ext_vector_type(2)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
}  // namespace

// NB: key blocks of 32 held per lane (N <= 32 NB); 4 waves x 32 queries per work-group.
template <int NB>
__global__ void __launch_bounds__(256) attn_kernel(const AttnParams a)
{
  using F = Mf<32>;
  typedef F::acc_t acc_t;
  constexpr int KD = kAttnKD, HD = kAttnHD;
  constexpr int NP = NB * 32;    // keys padded to whole blocks
  constexpr int KTP = KD + 8;    // key / query row pitch (halves): 16-byte fragment reads conflict free
  constexpr int VP = NP + 8;     // v row pitch (halves)
  constexpr int QW = 128;        // queries per work-group
  __shared__ __attribute__((aligned(16))) _Float16 Kt[NP * KTP];
  __shared__ __attribute__((aligned(16))) _Float16 Vs[HD * VP];
  __shared__ __attribute__((aligned(16))) _Float16 Qt[QW * KTP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y, b = blockIdx.z, N = a.n;
  const int q0 = blockIdx.x * QW;
  const _Float16 * qp = reinterpret_cast<const _Float16 *>(a.q.ptr) + (long)b * a.q.img + (long)h * a.q.cs;
  const _Float16 * kp = reinterpret_cast<const _Float16 *>(a.k.ptr) + (long)b * a.k.img + (long)h * a.k.cs;
  const _Float16 * vp = reinterpret_cast<const _Float16 *>(a.v.ptr) + (long)b * a.v.img + (long)h * a.v.cs;
  _Float16 * op = reinterpret_cast<_Float16 *>(a.y.ptr) + (long)b * a.y.img + (long)h * a.y.cs;

  // ---- stage k^T, v and q^T in LDS.  k and q go in transposed (token rows): a lane loads
  // channels 2c and 2c + 1 of 8 consecutive tokens (two 16-byte loads) and writes the 8
  // channel pairs as dwords, so 16 consecutive lanes fill 64 consecutive bytes of a token
  // row (a per-channel transpose would put consecutive lanes 8 rows apart: a 32-way LDS bank
  // conflict).  v goes in as is.  Every load is issued before the first LDS write, so the
  // work-group waits for one memory latency; tokens (and queries) past N are zero.
  constexpr int KPC = (KD / 2) * (NP / 8), VPC = HD * NP / 8, QPC = (KD / 2) * (QW / 8);  // pieces
  constexpr int KI = (KPC + 255) / 256, VI = (VPC + 255) / 256, QI = (QPC + 255) / 256;
  h8 kr[KI][2], vr[VI], qr[QI][2];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int e = tid + 256 * i, c = e % (KD / 2), j = (e / (KD / 2)) * 8;
    const bool ok = e < KPC && j < N;
#pragma unroll
    for (int u = 0; u < 2; ++u) kr[i][u] = ok ? *reinterpret_cast<const h8 *>(kp + (long)(2 * c + u) * N + j) : h8{};
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int e = tid + 256 * i, d = e / (NP / 8), j = (e - d * (NP / 8)) * 8;
    vr[i] = (e < VPC && j < N) ? *reinterpret_cast<const h8 *>(vp + (long)d * N + j) : h8{};
  }
#pragma unroll
  for (int i = 0; i < QI; ++i) {
    const int e = tid + 256 * i, c = e % (KD / 2), qi = (e / (KD / 2)) * 8;
    const bool ok = e < QPC && q0 + qi < N;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      qr[i][u] = ok ? *reinterpret_cast<const h8 *>(qp + (long)(2 * c + u) * N + q0 + qi) : h8{};
  }
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int e = tid + 256 * i, c = e % (KD / 2), j = (e / (KD / 2)) * 8;
    if (e < KPC) {
#pragma unroll
      for (int t = 0; t < 8; ++t) *reinterpret_cast<h2v *>(Kt + (j + t) * KTP + 2 * c) = h2v{kr[i][0][t], kr[i][1][t]};
    }
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int e = tid + 256 * i, d = e / (NP / 8), j = (e - d * (NP / 8)) * 8;
    if (e < VPC) *reinterpret_cast<h8 *>(Vs + d * VP + j) = vr[i];
  }
  // scale_q: the plan multiplies q^T by the scale (an ew_binary node: fp32 product, fp16
  // store) before the product; the product of two fp16 values is exact in fp32, so one fp16
  // multiply rounds it the same way
  const _Float16 sc16 = (_Float16)a.scale;  // an fp16 value (the plan's init)
  const h2v sc2 = {sc16, sc16};
  const h2v qs2 = a.scale_q ? sc2 : h2v{(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
  for (int i = 0; i < QI; ++i) {
    const int e = tid + 256 * i, c = e % (KD / 2), qi = (e / (KD / 2)) * 8;
    if (e < QPC) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        *reinterpret_cast<h2v *>(Qt + (qi + t) * KTP + 2 * c) = h2v{qr[i][0][t], qr[i][1][t]} * qs2;
    }
  }
  __syncthreads();
  const int qw = q0 + wave * 32;  // this wave's first query
  if (qw >= N) return;            // no barrier follows

  // ---- T^T = fp16(fp16(k^T q) * scale) (or fp16(k^T q) of the scaled q), one query per lane
  // (column), 16 keys per block.  One packed fp16 multiply rounds the exact product as the
  // ew_binary node (fp32 multiply, fp16 store) does.
  const int nb = (N + 31) / 32;
  const h2v ss2 = a.scale_q ? h2v{(_Float16)1.0f, (_Float16)1.0f} : sc2;
  const _Float16 ninf = (_Float16)(-__builtin_inff());
  const int hi = lane >> 5;
  h2v T[NB][8];  // (keys of v = 2j, 2j + 1) of each block: scores, then probabilities
  h2v mx = {ninf, ninf};
  const int qrow = (wave * 32 + (lane & 31)) * KTP + 8 * hi;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    if (kb >= nb) continue;  // (a guard, not a break: the loop stays fully unrolled)
    acc_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < KD / 16; ++s) {
      const h8 fa = *reinterpret_cast<const h8 *>(Kt + (kb * 32 + (lane & 31)) * KTP + 8 * hi + 16 * s);
      const h8 fb = *reinterpret_cast<const h8 *>(Qt + qrow + 16 * s);
      acc = F::mma(fa, fb, acc);
    }
    const bool tail = kb * 32 + 32 > N;  // keys past N in this block: -inf (probability 0)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const h2v s2 = {(_Float16)acc[2 * j], (_Float16)acc[2 * j + 1]};
      h2v t2 = s2 * ss2;
      if (tail) {
        if (kb * 32 + F::row(lane, 2 * j) >= N) t2[0] = ninf;
        if (kb * 32 + F::row(lane, 2 * j + 1) >= N) t2[1] = ninf;
      }
      T[kb][j] = t2;
      mx = __builtin_elementwise_max(mx, t2);
    }
  }
  // ---- softmax over the keys: lane-local, then with the partner lane holding the other 16.
  // exp(T - m) = exp2((T - m) log2e): the difference first, in fp32 (exact for the scores
  // near the maximum, which carry the probability mass), then one multiply and one v_exp_f32
  // per score; the exponentials stay in fp32 registers for the probabilities (the softmax
  // node evaluates them twice).  Folding m log2e into one fma would round m log2e to fp32,
  // an exponent error of ulp(m log2e) that exceeds fp16's half ulp once |m| is large.
  float m = fmaxf((float)mx[0], (float)mx[1]);
  m = fmaxf(m, __shfl_xor(m, 32));
  constexpr float kLog2e = 1.4426950408889634f;
  float e[NB][16];
  float sum = 0.0f;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    if (kb >= nb) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      e[kb][v] = __builtin_amdgcn_exp2f(((float)T[kb][v / 2][v % 2] - m) * kLog2e);
      sum += e[kb][v];
    }
  }
  sum += __shfl_xor(sum, 32);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    if (kb >= nb) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) T[kb][j] = h2v{(_Float16)(e[kb][2 * j] * inv), (_Float16)(e[kb][2 * j + 1] * inv)};
  }

  // ---- O = v P^T: A = 32 channels x 16 keys of v, B = 16 keys x 32 queries of P
  acc_t o[HD / 32];
#pragma unroll
  for (int db = 0; db < HD / 32; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.0f;
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    if (kb >= nb) continue;  // (a guard, not a break: the loop stays fully unrolled)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      // keys 16 hh + 0..3 / 8..11 (lanes < 32) and + 4..7 / 12..15 (lanes >= 32) -> each lane
      // the 8 consecutive keys 16 hh + 8 * (lane >= 32) + 0..7 of its query
      const u2v lo = {__builtin_bit_cast(unsigned, T[kb][4 * hh + 0]), __builtin_bit_cast(unsigned, T[kb][4 * hh + 1])};
      const u2v up = {__builtin_bit_cast(unsigned, T[kb][4 * hh + 2]), __builtin_bit_cast(unsigned, T[kb][4 * hh + 3])};
      const auto s0 = __builtin_amdgcn_permlane32_swap(lo[0], up[0], false, false);
      const auto s1 = __builtin_amdgcn_permlane32_swap(lo[1], up[1], false, false);
      const u4v pq = {s0[0], s1[0], s0[1], s1[1]};
      const h8 fb = __builtin_bit_cast(h8, pq);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) {
        const h8 fa = *reinterpret_cast<const h8 *>(Vs + (db * 32 + (lane & 31)) * VP + kb * 32 + 16 * hh + 8 * hi);
        o[db] = F::mma(fa, fb, o[db]);
      }
    }
  }
  // ---- store O[d][query] (fp16): for each accumulator value, 32 lanes write 32 consecutive queries
  const int qi = qw + (lane & 31);
  if (qi < N) {
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) op[(long)(db * 32 + F::row(lane, v)) * N + qi] = (_Float16)o[db][v];
  }
}

int attn_key_blocks(int n)
{
  const int nb = (n + 31) / 32;
  return nb <= 4 ? 4 : nb <= 8 ? 8 : nb <= 13 ? 13 : 0;
}

void launch_attention(const AttnParams & a, hipStream_t s)
{
  const dim3 grid((unsigned)((a.n + 127) / 128), (unsigned)a.heads, (unsigned)a.batch), blk(256);
  switch (attn_key_blocks(a.n)) {
  case 4: hipLaunchKernelGGL(attn_kernel<4>, grid, blk, 0, s, a); break;
  case 8: hipLaunchKernelGGL(attn_kernel<8>, grid, blk, 0, s, a); break;
  case 13: hipLaunchKernelGGL(attn_kernel<13>, grid, blk, 0, s, a); break;
  default: throw std::runtime_error("fused attention: more than 416 tokens");
  }
}

}  // namespace ivh
