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
// which moves the N x N score matrix through HBM five times.
//
// Here a work-group of 12 waves (three per SIMD) owns the 16-query blocks of one (image,
// head) (or a share of them when batch x heads is below the CU count), a wave one block at a
// time.  k
// (transposed to key rows) and v are staged in LDS once per work-group (80 KB at 416 keys);
// v is copied by DMA straight into LDS and lands while the waves compute their first
// scores; each wave holds its 16 queries' q^T fragment in registers for the key loop.
//   * S^T = k^T q on v_mfma_f32_16x16x32_f16: one MFMA per 16 keys (kd = 32 is one K
//     slice).  The A operand's row r of the two MFMAs of a 32-key slice j is key
//     32 j + 8 (r / 4) + 4 h + r % 4 (h = 0, 1), so a lane of group g = lane / 16 ends up
//     holding the scores of keys 32 j + 8 g + 0..7 of its query (column lane % 16): exactly
//     the B-operand layout of the P v^T MFMA for that slice, so probabilities go from the
//     score registers into the second product with no lane exchange.
//   * Softmax per query: lane-local max / sum over the lane's keys, then two exchanges across
//     the four lane groups (xor 16, xor 32).  The fp16 rounding points of the nodes are kept
//     (S, T and P are rounded where the nodes store them); exp(T - m) is one v_fma_mix_f32
//     and one v_exp_f32 per score; the exponentials stay in fp32 registers between the sum
//     and the probabilities, which are rounded to fp16 straight from e * (1 / sum).
//   * O = v P^T on the same MFMA shape: A = 16 channels x 32 keys of v (one 16-byte LDS read
//     each), B = the 32 probabilities of the slice; the four 16-channel blocks of hd = 64
//     accumulate in registers.
// LDS layouts (conflict-free 16-byte fragment reads under gfx950's service order of
// ds_read_b128, four cycles of 16 lanes grouped by quad parity): k^T rows of 64 bytes with
// 16-byte chunk c of key k stored at chunk position c ^ (2 * bit 3 of k); v rows of N + 16
// halves (N rounded up to 32 keys).
#include "conv_common.hpp"
#include "kernels.hpp"

namespace ivh {

namespace {
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kAttnWaves = 12;  // waves per work-group (three per SIMD)
}  // namespace

// fp16 pair {a * s, b * s}, each product rounded once to fp16 (v_fma_mixlo / mixhi_f16 on
// fp32 operands: the exact product a * s + 0 rounded to the fp16 half)
__device__ __forceinline__ unsigned mul_pack(float a, float b, float s)
{
  unsigned r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(s));
  asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(r) : "v"(b), "v"(s));
  return r;
}

// Packed fp16 maximum.  Written out because the compiler otherwise canonicalises both
// operands of every maximum first (two more v_pk_max_f16); the scores are never signalling
// NaNs.
__device__ __forceinline__ h2v pk_max(h2v a, h2v b)
{
  h2v r;
  asm("v_pk_max_f16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// NB: 32-key slices (32 (NB - 1) < N <= 32 NB); SQ: the scale multiplies q (1) or the scores (0).
// A work-group owns a range of 16-query blocks of one (image, head): all of them when
// batch x heads fills the 256 CUs, else a share.
template <int NB, int SQ>
__global__ void __launch_bounds__(64 * kAttnWaves, 3) attn_kernel(const AttnParams a, int ngrp)
{
  using F = Mf<16>;
  typedef F::acc_t acc_t;
  constexpr int KD = kAttnKD, HD = kAttnHD;
  static_assert(KD == 32 && HD == 64, "one 16x16x32 MFMA per 16 keys, four 16-channel output blocks");
  constexpr int NT = 64 * kAttnWaves;
  constexpr int NP = NB * 32;     // keys padded to whole slices
  constexpr int VP = NP + 16;     // v row pitch (halves)
  constexpr int VS = VP / 8;      // 16-byte slots per v row
  constexpr int VDMA = (HD * VS + 63) / 64;  // v copy instructions (64 slots each)
  __shared__ __attribute__((aligned(16))) _Float16 Kt[NP * KD];
  __shared__ __attribute__((aligned(16))) _Float16 Vs[VDMA * 512];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = a.n;
  const int nqb = (N + 15) / 16, qpg = (nqb + ngrp - 1) / ngrp;
  // the work-groups of one (image, head) are neighbours on one XCD: its k and v stay in L2
  const int r = xcd_tile(blockIdx.x, gridDim.x);
  const int bh = r / ngrp, grp = r - bh * ngrp;
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int qb0 = grp * qpg, qb1 = min(nqb, qb0 + qpg);
  const _Float16 * qp = reinterpret_cast<const _Float16 *>(a.q.ptr) + (long)b * a.q.img + (long)h * a.q.cs;
  const _Float16 * kp = reinterpret_cast<const _Float16 *>(a.k.ptr) + (long)b * a.k.img + (long)h * a.k.cs;
  const __half * vp = a.v.ptr + (long)b * a.v.img + (long)h * a.v.cs;
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(a.y.ptr + (long)b * a.y.img + (long)h * a.y.cs,
                                                                     (short)0, HD * N * 2, kBufDword3);

  // q^T fragment of a 16-query block (B operand of the scores): channels 8g..8g+7 of the
  // lane's query; the first one is loaded before the staging, each next one a block ahead
  const int rr = lane & 15, g = lane >> 4;
  // buffer accesses: a per-lane offset and a uniform one per channel (no 64-bit address
  // arithmetic per element); queries past N fall outside the range (reads zero, no store)
  const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16 *>(qp), (short)0,
                                                                     KD * N * 2, kBufDword3);
  auto load_q = [&](int qb) __attribute__((always_inline)) {
    const int qi = qb * 16 + rr;
    const unsigned off = qi < N ? (unsigned)(8 * g * N + qi) * 2u : kBufOOB;
    h8 v;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      v[k] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(qr, off, k * N * 2, 0));
    return v;
  };
  h8 qn = qb0 + wave < qb1 ? load_q(qb0 + wave) : h8{};

  // ---- stage k^T (through registers: transposed to key rows) and v (DMA, straight into
  // LDS; it lands while the scores are computed).  A thread loads channels 2c and 2c + 1 of
  // 8 consecutive keys of k (two 16-byte loads) and writes the 8 channel pairs as dwords;
  // keys past N are zero (N is a multiple of 8).
  constexpr int KPC = (KD / 2) * (NP / 8);  // k pieces
  constexpr int KI = (KPC + NT - 1) / NT;
  h8 kr[KI][2];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int e = tid + NT * i, c2 = e % (KD / 2), j = e / (KD / 2);
    const bool ok = e < KPC && 8 * j < N;
#pragma unroll
    for (int u = 0; u < 2; ++u) kr[i][u] = ok ? *reinterpret_cast<const h8 *>(kp + (long)(2 * c2 + u) * N + 8 * j) : h8{};
  }
  {
    // v: copy instruction i writes slots [64 i, 64 i + 64) of the [HD][VS] slot array; slot
    // (d, piece) holds keys 8 piece .. 8 piece + 7 of channel d (zeros past N and in the pad)
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<__half *>(vp), (short)0,
                                                                       HD * N * 2, kBufDword3);
    for (int i = wave; i < VDMA; i += kAttnWaves) {
      const int slot = 64 * i + lane, d = slot / VS, piece = slot - d * VS;
      const bool ok = d < HD && 8 * piece < N;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void *)(Vs + 512 * i), 16,
                                               ok ? (d * N + 8 * piece) * 2 : (int)kBufOOB, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int e = tid + NT * i, c2 = e % (KD / 2), j = e / (KD / 2);
    if (e < KPC) {
      // keys 8j..8j+7 share bit 3 (= bit 0 of j): one chunk position for the piece
      const int pos = ((c2 >> 2) ^ ((j & 1) << 1)) * 8 + 2 * (c2 & 3);
#pragma unroll
      for (int t = 0; t < 8; ++t) *reinterpret_cast<h2v *>(Kt + (8 * j + t) * KD + pos) = h2v{kr[i][0][t], kr[i][1][t]};
    }
  }
  __syncthreads();  // k^T in LDS

  // the scale: the plan multiplies q^T (SQ) or the scores by it (an ew_binary node: fp32
  // product, fp16 store).  The product of two fp16 values is exact in fp32, so one fp16
  // multiply rounds it as the node does.
  const _Float16 sc16 = (_Float16)a.scale;  // an fp16 value (the plan's init)
  const h2v ss2 = {sc16, sc16};
  const _Float16 ninf = (_Float16)(-__builtin_inff());
  constexpr float kLog2e = 1.4426950408889634f;
  // k^T row of this lane in the slice's MFMA h: key 32 j + 8 (rr / 4) + 4 h + rr % 4; its
  // chunk g sits at position g ^ (2 * bit 3 of the key) = g ^ (2 * bit 2 of rr)
  const int krow = (8 * (rr >> 2) + (rr & 3)) * KD + 8 * (g ^ (((rr >> 2) & 1) << 1));
  const int vrow = rr * VP + 8 * g;
  // every wave passes the barrier that publishes v exactly once, after its first block's
  // softmax (or at once, without a block)
  bool v_ready = false;
  auto wait_v = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    __syncthreads();
    v_ready = true;
  };

  for (int qb = qb0 + wave; qb < qb1; qb += kAttnWaves) {
    const int qi = qb * 16 + rr;  // this lane's query (column)
    // q^T fragment (B operand): channels 8g..8g+7 of query qi, loaded one block ahead
    h8 qf = qn;
    if (qb + kAttnWaves < qb1) qn = load_q(qb + kAttnWaves);
    if (SQ) {
#pragma unroll
      for (int k = 0; k < 8; ++k) qf[k] = qf[k] * sc16;
    }
    // ---- T = fp16(fp16(S) * scale) (or fp16(S) of the scaled q), keys 32 j + 8 g + 0..7;
    // running maxima as four independent partials (short dependency chains)
    h2v T[NB][4];
    h2v mx[4] = {{ninf, ninf}, {ninf, ninf}, {ninf, ninf}, {ninf, ninf}};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const h8 fa = *reinterpret_cast<const h8 *>(Kt + (32 * j + 4 * hh) * KD + krow);
        acc_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = F::mma(fa, qf, acc);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const h2v s2 = {(_Float16)acc[2 * u], (_Float16)acc[2 * u + 1]};
          T[j][2 * hh + u] = SQ ? s2 : s2 * ss2;
        }
      }
      // keys past N, in the last slice only (32 (NB - 1) < N <= 32 NB): N is a multiple of 8,
      // so a lane's 8 keys 32 j + 8 g + 0..7 are all inside or all outside
      if (j == NB - 1) {
        const bool pad = 32 * j + 8 * g >= N;
#pragma unroll
        for (int u = 0; u < 4; ++u) T[j][u] = __builtin_bit_cast(h2v, pad ? 0xfc00fc00u : __builtin_bit_cast(unsigned, T[j][u]));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) mx[u] = pk_max(mx[u], T[j][u]);
    }
    // ---- softmax over the keys: lane-local, then across the four lane groups of the query
    const h2v mx2 = pk_max(pk_max(mx[0], mx[1]), pk_max(mx[2], mx[3]));
    float m = fmaxf((float)mx2[0], (float)mx2[1]);
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    // exp(T - m) = exp2(T log2e - m log2e), one v_fma_mix_f32 on the fp16 score (T log2e is
    // exact inside the fma) and one v_exp_f32.  The fp32 rounding of m log2e is the same for
    // every key of the query, so it scales all of the query's exponentials and their sum by
    // one factor 2^-d (|d| <= ulp(m log2e) / 2), which the division by the sum cancels: the
    // probabilities do not depend on it, however large m is.  The exponentials stay in fp32
    // registers between the sum and the probabilities.
    const float mb = -m * kLog2e;
    float e[NB][8];
    float ps[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        e[j][v] = __builtin_amdgcn_exp2f(fmaf((float)T[j][v / 2][v % 2], kLog2e, mb));
        ps[v & 3] += e[j][v];
      }
    }
    float sum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const float inv = 1.0f / sum;
    if (!v_ready) wait_v();

    // ---- O = v P^T: A = 16 channels x 32 keys of v, B = the slice's 32 probabilities
    acc_t o[HD / 16];
#pragma unroll
    for (int db = 0; db < HD / 16; ++db) o[db] = acc_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      unsigned pb2[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) pb2[u] = mul_pack(e[j][2 * u], e[j][2 * u + 1], inv);
      const h8 pb = __builtin_bit_cast(h8, pb2);
#pragma unroll
      for (int db = 0; db < HD / 16; ++db) {
        const h8 fa = *reinterpret_cast<const h8 *>(Vs + db * 16 * VP + vrow + 32 * j);
        o[db] = F::mma(fa, pb, o[db]);
      }
    }
    // ---- store O[d][query] (fp16): channel 16 db + 4 g + v, 16 lanes on 16 consecutive queries
    const unsigned yoff = qi < N ? (unsigned)(4 * g * N + qi) * 2u : kBufOOB;
#pragma unroll
    for (int db = 0; db < HD / 16; ++db)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (_Float16)o[db][v]), yr, yoff,
                                              (16 * db + v) * N * 2, 0);
  }
  if (!v_ready) wait_v();  // waves without a block still take part in the barrier
}

int attn_key_blocks(int n)
{
  const int nb = (n + 31) / 32;
  return nb >= 1 && nb <= 13 ? nb : 0;
}

// Work-groups per (image, head): one when batch x heads fills the 256 CUs, else enough
// query ranges to (each re-stages k and v, from L2 after the first)
int attn_groups(const AttnParams & a)
{
  const int nqb = (a.n + 15) / 16;
  const long bh = (long)a.batch * a.heads;
  const int want = (int)std::min<long>((256 + bh - 1) / bh, nqb);
  return std::max(1, want);
}

template <int NB>
static void launch_attn_nb(const AttnParams & a, int ng, hipStream_t s)
{
  const dim3 grid((unsigned)((long)a.batch * a.heads * ng)), blk(64 * kAttnWaves);
  if (a.scale_q) hipLaunchKernelGGL((attn_kernel<NB, 1>), grid, blk, 0, s, a, ng);
  else hipLaunchKernelGGL((attn_kernel<NB, 0>), grid, blk, 0, s, a, ng);
}

void launch_attention(const AttnParams & a, hipStream_t s)
{
  const int ng = attn_groups(a);
  switch (attn_key_blocks(a.n)) {
  case 1: launch_attn_nb<1>(a, ng, s); break;
  case 2: launch_attn_nb<2>(a, ng, s); break;
  case 3: launch_attn_nb<3>(a, ng, s); break;
  case 4: launch_attn_nb<4>(a, ng, s); break;
  case 5: launch_attn_nb<5>(a, ng, s); break;
  case 6: launch_attn_nb<6>(a, ng, s); break;
  case 7: launch_attn_nb<7>(a, ng, s); break;
  case 8: launch_attn_nb<8>(a, ng, s); break;
  case 9: launch_attn_nb<9>(a, ng, s); break;
  case 10: launch_attn_nb<10>(a, ng, s); break;
  case 11: launch_attn_nb<11>(a, ng, s); break;
  case 12: launch_attn_nb<12>(a, ng, s); break;
  case 13: launch_attn_nb<13>(a, ng, s); break;
  default: throw std::runtime_error("fused attention: more than 416 tokens");
  }
}

}  // namespace ivh
