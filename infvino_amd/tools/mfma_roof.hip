// MFMA roof probe: the fp16 matrix-core rate this GPU sustains on the loop shape of the
// conv kernels, for zero operands and for random operands.
//
// Each work-group (4 waves, 2 x 2 layout) runs `steps` K steps; a step reads its A and B
// fragments from LDS (4 x 2 blocks of 32 x 32 per wave, two 16-deep slices) and issues 16
// v_mfma_f32_32x32x16_f16, then a barrier -- the shape of the LDS-patch and pipelined conv
// kernels' inner loops without any global traffic.  Two work-groups per CU (68 KB of LDS
// each), 512 work-groups.  The LDS operands are either all zero or uniform in [-0.5, 0.5):
// the matrix cores draw more power on random data and the clock drops, so the random-data
// rate is the practical MFMA roof for real activations and weights.
//
// Build: make -C infvino_amd/csrc tools (part of the default build)
// Run:   infvino_amd/tools/mfma_roof [steps]
// Prints one JSON line: {"zeros_tflops": ..., "random_tflops": ..., "peak_tflops": 2500, ...}
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kLdsHalves = 68 * 512;  // 68 KB: two work-groups per CU
constexpr int kWgs = 512;

template <bool RND>
__global__ void __launch_bounds__(256, 2) mfma_loop(float * out, int steps)
{
  __shared__ __attribute__((aligned(16))) _Float16 lds[kLdsHalves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kLdsHalves / 8; i += 256) {
    h8 v = h8{};
    if (RND) {
      unsigned x = (unsigned)i * 2654435761u + blockIdx.x * 97u + 1u;
      for (int k = 0; k < 8; ++k) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        v[k] = (_Float16)((float)(x & 0xffff) * (1.0f / 65536.0f) - 0.5f);
      }
    }
    *reinterpret_cast<h8 *>(lds + i * 8) = v;
  }
  __syncthreads();
  f16v acc[2][4];
  for (int a = 0; a < 2; ++a)
    for (int b = 0; b < 4; ++b)
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  const int abase = wave * 4096 + lane * 8, bbase = 16384 + lane * 8;
  // every index below is masked into [0, kLdsHalves - 8] and 8-aligned (the mask's low three
  // bits are zero and it is below the array size)
  constexpr int kMask = kLdsHalves - 8;
  for (int s = 0; s < steps; ++s) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      h8 fa[2], fb[4];
#pragma unroll
      for (int t = 0; t < 2; ++t) fa[t] = *reinterpret_cast<const h8 *>(lds + ((abase + t * 512 + j * 1024 + s * 64) & kMask));
#pragma unroll
      for (int t = 0; t < 4; ++t) fb[t] = *reinterpret_cast<const h8 *>(lds + ((bbase + t * 512 + j * 2048 + s * 128) & kMask));
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[a], fb[b], acc[a][b], 0, 0, 0);
    }
    __syncthreads();
  }
  float t = 0.0f;
  for (int a = 0; a < 2; ++a)
    for (int b = 0; b < 4; ++b)
      for (int v = 0; v < 16; ++v) t += acc[a][b][v];
  out[blockIdx.x * 256 + tid] = t;
}

#define CHECK(x)                                                                      \
  do {                                                                                \
    const hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                           \
      std::fprintf(stderr, "mfma_roof: %s: %s\n", #x, hipGetErrorString(e_));         \
      std::exit(1);                                                                   \
    }                                                                                 \
  } while (0)

template <bool RND>
double rate_tflops(float * out, int steps)
{
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int i = 0; i < 3; ++i) hipLaunchKernelGGL(mfma_loop<RND>, dim3(kWgs), dim3(256), 0, 0, out, steps);
  CHECK(hipGetLastError());
  const int reps = 10;
  CHECK(hipEventRecord(e0, 0));
  for (int i = 0; i < reps; ++i) hipLaunchKernelGGL(mfma_loop<RND>, dim3(kWgs), dim3(256), 0, 0, out, steps);
  CHECK(hipEventRecord(e1, 0));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  const double flops = (double)kWgs * 4 * steps * 16 * 32768.0 * reps;  // 16 MFMAs of 32x32x16 per wave-step
  return flops / (ms * 1e-3) / 1e12;
}

}  // namespace

int main(int argc, char ** argv)
{
  const int steps = argc > 1 ? std::atoi(argv[1]) : 2000;
  if (steps < 1 || steps > 1000000) {
    std::fprintf(stderr, "mfma_roof: steps out of range\n");
    return 2;
  }
  float * out = nullptr;
  CHECK(hipMalloc(&out, (size_t)kWgs * 256 * sizeof(float)));
  const double z = rate_tflops<false>(out, steps);
  const double r = rate_tflops<true>(out, steps);
  CHECK(hipFree(out));
  std::printf("{\"zeros_tflops\": %.1f, \"random_tflops\": %.1f, \"peak_tflops\": 2500.0, "
              "\"zeros_frac\": %.4f, \"random_frac\": %.4f, \"loop\": \"4 waves x 4x2 32x32x16 f16 MFMA blocks, "
              "LDS fragments, one barrier per 16 MFMAs, 2 work-groups per CU, %d steps\"}\n",
              z, r, z / 2500.0, r / 2500.0, steps);
  return 0;
}
