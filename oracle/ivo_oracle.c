/*
 * ivo_oracle.c -- CPU oracle for infvino's plan-driven conv/GEMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it is loaded by tests/,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product library (infvino_amd/csrc), which must fail loudly rather than fall
 * back to anything here.
 *
 * Every function restates, in plain C over one image in NCHW fp16 storage, the
 * arithmetic of the reference kernel it names (paths are into the reference
 * repository).  Two numeric modes:
 *   IVO_F32 (0): exact fp32 accumulation, one fp16 rounding (RNE) at the store.
 *                This is what the numpy-fp32 oracle of scripts/kernel_check.py
 *                computes, and it is the semantics the HIP kernels implement.
 *   IVO_REF (1): the reference kernels' own rounding points: fp16 accumulation
 *                with fused multiply-add (gemm.cl:468-472, conv_ov.cl:167,
 *                conv_general.cl:101), bias added in fp16, activation in fp32 on
 *                an fp16 value then rounded, residual added in fp16
 *                (gemm.cl:644-650, conv_ov.cl:285-288).  The exact trajectory
 *                under Intel IGC mad contraction cannot be reproduced on a CPU,
 *                so this mode bounds, rather than replays, the reference.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   f16 conversions  - every one of the 2^16 half patterns (exact f16->f32),
 *                      numpy astype(float16) for RNE, and the reference's own
 *                      src/Half.cpp built into oracle/_ref for truncation.
 *   conv / gemm      - torch.nn.functional.conv2d on CPU (a library routine),
 *                      delta-kernel and constant-input closed forms, brute force.
 *   depthwise        - torch conv2d with groups=C.
 *   small ops        - numpy closed forms (softmax sums to 1, permute twice is
 *                      identity, maxpool of a ramp, nearest resize by repeat).
 *   IVO_REF mode     - bounded by the reference's published error magnitudes
 *                      (docs/benchmark.md:14-20) on the reference's own seeds.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define IVO_F32 0
#define IVO_REF 1

/* ---------------------------------------------------------------- fp16 bits */

/* Exact fp16 -> fp32, denormals included (include/infvino/Half.hpp:26-49). */
float ivo_h2f(uint16_t h)
{
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t f;
  if (exp == 0) {
    if (mant == 0) {
      f = sign;
    } else {
      /* value = mant * 2^-24: normalise into an fp32 exponent */
      int e = -14;
      while (!(mant & 0x400u)) { mant <<= 1; --e; }
      mant &= 0x3ffu;
      f = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    f = sign | 0x7f800000u | (mant << 13);
  } else {
    f = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float out;
  memcpy(&out, &f, 4);
  return out;
}

/* IEEE fp32 -> fp16, round to nearest even, with denormals, overflow to inf and
 * NaN preserved -- the conversion numpy's astype(np.float16) performs, used by
 * scripts/onnx2plan.py:64 for weights and by every fp16 store of a (half) cast. */
uint16_t ivo_f2h(float f)
{
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf or nan */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) { /* below the smallest normal half: denormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to zero */
    const uint32_t e = ax >> 23;                 /* 102..112 */
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;             /* 14..24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  /* normal range: rebias and round the 13 dropped mantissa bits */
  uint32_t r = ((ax >> 13) - (112u << 10));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

/* The reference's boundary conversion (include/infvino/Half.hpp:14-24):
 * truncate the mantissa, flush results with exponent <= 0 to signed zero,
 * saturate exponent >= 31 (NaN included) to signed infinity. */
uint16_t ivo_f2h_trunc(float f)
{
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((x >> 23) & 0xffu) - 127 + 15;
  const uint32_t mant = x & 0x7fffffu;
  if (exp <= 0) return (uint16_t)sign;
  if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | ((uint32_t)exp << 10) | (mant >> 13));
}

void ivo_f32_to_f16_trunc_bulk(const float *in, uint16_t *out, long n)
{
  for (long i = 0; i < n; ++i) out[i] = ivo_f2h_trunc(in[i]);
}
void ivo_f32_to_f16_rne_bulk(const float *in, uint16_t *out, long n)
{
  for (long i = 0; i < n; ++i) out[i] = ivo_f2h(in[i]);
}
void ivo_f16_to_f32_bulk(const uint16_t *in, float *out, long n)
{
  for (long i = 0; i < n; ++i) out[i] = ivo_h2f(in[i]);
}

static inline float rh(float v) { return ivo_h2f(ivo_f2h(v)); } /* round to half */

/* fp16 fused multiply-add: one rounding of the exact a*b+c.  a*b of two halves is
 * exact in fp32 (22 significant bits); the fp32 add may round once more before
 * the fp16 rounding, a double rounding that is below the reference's own
 * uncertainty about mad contraction. */
static inline float fma_h(float a, float b, float c) { return rh(a * b + c); }

/* ------------------------------------------------------------- activations */

/* Canonical codes (include/infvino/KernelFamily.hpp:70-73, scripts/onnx2plan.py:130-138):
 * 0 none, 1 SiLU, 2 ReLU, 3 HardSwish, 4 HardSigmoid, 5 Sigmoid.
 * Formulas as gemm.cl:137-154. */
float ivo_act(float f, int act)
{
  switch (act) {
  case 1: return f / (1.0f + expf(-f));
  case 2: return f > 0.0f ? f : 0.0f;
  case 3: return f * fminf(fmaxf(f + 3.0f, 0.0f), 6.0f) / 6.0f;
  case 4: return fminf(fmaxf(f + 3.0f, 0.0f), 6.0f) / 6.0f;
  case 5: return 1.0f / (1.0f + expf(-f));
  default: return f;
  }
}

/* ew_unary has its own table (kernels/ops.cl:50-63):
 * 0 Sigmoid, 1 SiLU, 2 ReLU, 3 HardSwish, 4 HardSigmoid. */
static int unary_to_canonical(int op)
{
  static const int map[5] = {5, 1, 2, 3, 4};
  return (op >= 0 && op < 5) ? map[op] : 0;
}

/* ------------------------------------------------------------------- conv */

/* Generic 2-D convolution over one image, NCHW.
 *   x   [Cin][H][W]          w [Cout][Cin/G][K][K]      bias [Cout] or NULL
 *   res [Cout][Ho][Wo] or NULL (added after the activation)
 *   y   [Cout][Ho][Wo]
 * IVO_F32: y = rne(act(sum + b) + r).
 * IVO_REF, by the kernel family that the reference dispatches for the node:
 *   family 0 (gemm_f16 / conv3x3_ov / conv3x3_cin3 / depthwise_f16): fp16
 *     accumulation over (ci, ky, kx) ascending, v = half(acc) + half(b) in fp16,
 *     half(act(v)), then + half(res) in fp16 (gemm.cl:468-472,644-650;
 *     conv_ov.cl:167,285-288; conv_general.cl:101,113).
 *   family 1 (conv1x1_gemv_f16, N == 1): fp32 accumulation, half(s) + half(b)
 *     in fp16, half(act), + half(res) (conv1x1.cl:170,186-196).
 *   family 2 (conv_general): fp32 accumulation with the bias preloaded,
 *     half(act(acc)) (conv_general.cl:27-47).  Activation codes are the canonical
 *     ones onnx2plan emits (onnx2plan.py:138); conv_general.cl:43-46 itself reads
 *     legacy codes (2 HardSwish, 3 ReLU). */
void ivo_conv2d(const uint16_t *x, int Cin, int H, int W,
                const uint16_t *w, int Cout, int K, int S, int P, int G,
                const uint16_t *bias, const uint16_t *res,
                uint16_t *y, int Ho, int Wo, int act, int mode, int family)
{
  const int cin_g = Cin / G, cout_g = Cout / G;
  const long HWo = (long)Ho * Wo;
  const int ref_half = (mode == IVO_REF && family == 0);
  float *xf = (float *)malloc(sizeof(float) * (size_t)Cin * H * W);
  for (long i = 0; i < (long)Cin * H * W; ++i) xf[i] = ivo_h2f(x[i]);
#pragma omp parallel
  {
    float *acc = (float *)malloc(sizeof(float) * (size_t)HWo);
#pragma omp for schedule(dynamic, 1)
    for (int co = 0; co < Cout; ++co) {
      const int g = co / cout_g;
      /* conv_general preloads the bias into its fp32 accumulator (conv_general.cl:27) */
      const float b = bias ? ivo_h2f(bias[co]) : 0.0f;
      const float acc0 = (mode == IVO_REF && family == 2) ? b : 0.0f;
      for (long i = 0; i < HWo; ++i) acc[i] = acc0;
      for (int cl = 0; cl < cin_g; ++cl) {
        const int ci = g * cin_g + cl;
        const float *xp = xf + (size_t)ci * H * W;
        for (int ky = 0; ky < K; ++ky)
          for (int kx = 0; kx < K; ++kx) {
            const float wv = ivo_h2f(w[(((size_t)co * cin_g + cl) * K + ky) * K + kx]);
            /* output columns whose input column ox*S-P+kx lies inside [0, W) */
            int lo = 0;
            while (lo < Wo && lo * S - P + kx < 0) ++lo;
            int hi = Wo;
            while (hi > lo && (hi - 1) * S - P + kx >= W) --hi;
            for (int oy = 0; oy < Ho; ++oy) {
              const int iy = oy * S - P + ky;
              if (iy < 0 || iy >= H) continue;
              float *ar = acc + (size_t)oy * Wo;
              const float *xr = xp + (size_t)iy * W - P + kx;
              if (ref_half) {
                for (int ox = lo; ox < hi; ++ox) ar[ox] = fma_h(xr[ox * S], wv, ar[ox]);
              } else if (S == 1) {
                for (int ox = lo; ox < hi; ++ox) ar[ox] += xr[ox] * wv;
              } else {
                for (int ox = lo; ox < hi; ++ox) ar[ox] += xr[ox * S] * wv;
              }
            }
          }
      }
      for (long i = 0; i < HWo; ++i) {
        const size_t oi = (size_t)co * HWo + i;
        float v;
        if (mode == IVO_REF && family != 2) {
          v = rh(rh(acc[i]) + b);
          v = rh(ivo_act(v, act));
          if (res) v = rh(v + ivo_h2f(res[oi]));
        } else if (mode == IVO_REF) {
          v = rh(ivo_act(acc[i], act));
          if (res) v = rh(v + ivo_h2f(res[oi]));
        } else {
          v = ivo_act(acc[i] + b, act);
          if (res) v += ivo_h2f(res[oi]);
        }
        y[oi] = ivo_f2h(v);
      }
    }
    free(acc);
  }
  free(xf);
}

/* --------------------------------------------------------- elementwise ops */

static inline float binop(float a, float b, int op)
{
  switch (op) {
  case 0: return a + b;
  case 1: return a - b;
  case 2: return a * b;
  default: return a / b;
  }
}

/* ew_binary, kernels/ops.cl:34-48 (b_scalar broadcasts b[0]); fp32 compute,
 * fp16 store. */
void ivo_ew_binary(const uint16_t *a, const uint16_t *b, uint16_t *y, long n, int op,
                   int b_scalar)
{
  for (long i = 0; i < n; ++i)
    y[i] = ivo_f2h(binop(ivo_h2f(a[i]), ivo_h2f(b_scalar ? b[0] : b[i]), op));
}

/* ew_binary_bcast, kernels/ops.cl:10-32: dims = [out(rank), a_strides(rank),
 * b_strides(rank)], strides in elements, 0 on broadcast dimensions. */
void ivo_ew_binary_bcast(const uint16_t *a, const uint16_t *b, uint16_t *y, long n, int op,
                         int rank, const int *dims)
{
  for (long i = 0; i < n; ++i) {
    long rem = i, ai = 0, bi = 0;
    for (int r = rank - 1; r >= 0; --r) {
      const long coord = rem % dims[r];
      rem /= dims[r];
      ai += coord * dims[rank + r];
      bi += coord * dims[2 * rank + r];
    }
    y[i] = ivo_f2h(binop(ivo_h2f(a[ai]), ivo_h2f(b[bi]), op));
  }
}

/* ew_unary, kernels/ops.cl:50-63. */
void ivo_ew_unary(const uint16_t *x, uint16_t *y, long n, int op)
{
  const int act = unary_to_canonical(op);
  for (long i = 0; i < n; ++i) y[i] = ivo_f2h(ivo_act(ivo_h2f(x[i]), act));
}

/* bias_add, kernels/ops.cl:268-274. */
void ivo_bias_add(const uint16_t *x, const uint16_t *b, uint16_t *y, long n, int HW)
{
  for (long i = 0; i < n; ++i) y[i] = ivo_f2h(ivo_h2f(x[i]) + ivo_h2f(b[i / HW]));
}

/* ---------------------------------------------------------- data movement */

/* copy_c, kernels/ops.cl:65-72. */
void ivo_copy_c(const uint16_t *x, uint16_t *y, int HW, int c0, int cnt, int dst_off)
{
  for (long i = 0; i < (long)cnt * HW; ++i) {
    const long c = i / HW, r = i % HW;
    y[dst_off + i] = x[(c0 + c) * HW + r];
  }
}

/* slice_axis, kernels/ops.cl:74-91. */
void ivo_slice_axis(const uint16_t *x, uint16_t *y, int outer, int axdim, int inner,
                    int start, int len)
{
  const long total = (long)outer * len * inner;
  for (long i = 0; i < total; ++i) {
    const long o = i / ((long)len * inner), rem = i % ((long)len * inner);
    y[i] = x[(o * axdim + start) * inner + rem];
  }
}

/* concat4, kernels/ops.cl:93-119 (NCHW output). */
void ivo_concat4(const uint16_t *a, int ca, const uint16_t *b, int cb, const uint16_t *c,
                 int cc, const uint16_t *d, int cd, uint16_t *y, int outer, int inner)
{
  const int sum = ca + cb + cc + cd;
  for (int o = 0; o < outer; ++o)
    for (int ax = 0; ax < sum; ++ax)
      for (int r = 0; r < inner; ++r) {
        uint16_t v;
        if (ax < ca) v = a[((long)o * ca + ax) * inner + r];
        else if (ax < ca + cb) v = b[((long)o * cb + (ax - ca)) * inner + r];
        else if (ax < ca + cb + cc) v = c[((long)o * cc + (ax - ca - cb)) * inner + r];
        else v = d[((long)o * cd + (ax - ca - cb - cc)) * inner + r];
        y[((long)o * sum + ax) * inner + r] = v;
      }
}

/* maxpool, kernels/ops.cl:148-166: out-of-bounds taps ignored, fp32 max. */
void ivo_maxpool(const uint16_t *x, uint16_t *y, int C, int H, int W, int Ho, int Wo, int K,
                 int S, int P)
{
  for (int c = 0; c < C; ++c)
    for (int oh = 0; oh < Ho; ++oh)
      for (int ow = 0; ow < Wo; ++ow) {
        float m = -3.4e38f;
        for (int kh = 0; kh < K; ++kh)
          for (int kw = 0; kw < K; ++kw) {
            const int yy = oh * S - P + kh, xx = ow * S - P + kw;
            if (yy >= 0 && yy < H && xx >= 0 && xx < W) {
              const float v = ivo_h2f(x[((long)c * H + yy) * W + xx]);
              m = v > m ? v : m;
            }
          }
        y[((long)c * Ho + oh) * Wo + ow] = ivo_f2h(m);
      }
}

/* resize_nn, kernels/ops.cl:168-179: integer scale S. */
void ivo_resize_nn(const uint16_t *x, uint16_t *y, int C, int H, int W, int S)
{
  const int Ho = H * S, Wo = W * S;
  for (int c = 0; c < C; ++c)
    for (int oh = 0; oh < Ho; ++oh)
      for (int ow = 0; ow < Wo; ++ow)
        y[((long)c * Ho + oh) * Wo + ow] = x[((long)c * H + oh / S) * W + ow / S];
}

/* softmax_axis, kernels/ops.cl:181-197: max-subtracted, fp32. */
void ivo_softmax_axis(const uint16_t *x, uint16_t *y, int outer, int axdim, int inner)
{
  for (int o = 0; o < outer; ++o)
    for (int r = 0; r < inner; ++r) {
      float m = -3.4e38f, s = 0.0f;
      for (int a = 0; a < axdim; ++a) {
        const float v = ivo_h2f(x[((long)o * axdim + a) * inner + r]);
        m = v > m ? v : m;
      }
      for (int a = 0; a < axdim; ++a)
        s += expf(ivo_h2f(x[((long)o * axdim + a) * inner + r]) - m);
      for (int a = 0; a < axdim; ++a) {
        const long i = ((long)o * axdim + a) * inner + r;
        y[i] = ivo_f2h(expf(ivo_h2f(x[i]) - m) / s);
      }
    }
}

/* permute_0213, kernels/ops.cl:199-222: mode 0 [D1,D2,I]->[D2,D1,I],
 * mode 1 [D1,D2,I]->[D1,I,D2]. */
void ivo_permute_0213(const uint16_t *x, uint16_t *y, int D1, int D2, int I, int mode)
{
  for (int d1 = 0; d1 < D1; ++d1)
    for (int d2 = 0; d2 < D2; ++d2)
      for (int r = 0; r < I; ++r) {
        const long i = ((long)d1 * D2 + d2) * I + r;
        if (mode == 0) y[((long)d2 * D1 + d1) * I + r] = x[i];
        else y[((long)d1 * I + r) * D2 + d2] = x[i];
      }
}

/* gap, kernels/ops.cl:224-243: fp32 mean. */
void ivo_gap(const uint16_t *x, uint16_t *y, int C, int HW)
{
  for (int c = 0; c < C; ++c) {
    float s = 0.0f;
    for (int i = 0; i < HW; ++i) s += ivo_h2f(x[(long)c * HW + i]);
    y[c] = ivo_f2h(s / (float)HW);
  }
}

/* bmm, kernels/ops.cl:276-294: [B0*B1][M][K] x [B0*B1][K][N], fp32 acc. */
void ivo_bmm(const uint16_t *A, const uint16_t *B, uint16_t *Y, int BB, int M, int K, int N)
{
  for (int b = 0; b < BB; ++b)
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k)
          acc += ivo_h2f(A[((long)b * M + m) * K + k]) * ivo_h2f(B[((long)b * K + k) * N + n]);
        Y[((long)b * M + m) * N + n] = ivo_f2h(acc);
      }
}
