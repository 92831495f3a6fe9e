// C++ drop-in check of the boundary: HipBackend / HipPlanModel used the way the
// reference's InferenceEngine / kernel_run use ClBackend / PlanModel.
//   test_backend <plan> <out.bin> <malformed_plan>
// Writes the f32 outputs of infer() on a fixed input (batch 2) to out.bin for the Python
// side to compare with the oracle; exits non-zero on any failed expectation.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "infvino_hip/HipBackend.hpp"

struct ModelInfoLike  // the members HipBackend reads from infvino::ModelInfo
{
  std::string plan;
  std::string device = "GPU.0";
};

#define EXPECT(c)                                                        \
  do {                                                                   \
    if (!(c)) {                                                          \
      std::fprintf(stderr, "EXPECT failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                                          \
    }                                                                    \
  } while (0)

int main(int argc, char ** argv)
{
  if (argc < 4) return 2;
  bool threw = false;
  ModelInfoLike info;
  info.plan = argv[1];
  // batch 2 without split-K: an image's result is then independent of the batch size, so
  // the single-image inference below must equal image 0 of the batch bit for bit
  infvino_hip::HipBackend be(info, false, 2, IVH_FLAG_NO_SPLITK);
  const auto & in = be.inputDims();
  size_t n = 1;
  for (auto d : in) n *= static_cast<size_t>(d);
  std::vector<float> x(2 * n);
  for (size_t i = 0; i < x.size(); ++i) x[i] = static_cast<float>((i * 2654435761u) % 1000u) / 1000.0f;
  auto out = be.infer(x.data(), x.size());
  EXPECT(out.size() == be.outputShapes().size());
  EXPECT(out[0].shape[0] == 2 * be.outputShapes()[0][0]);
  FILE * f = std::fopen(argv[2], "wb");
  EXPECT(f);
  std::fwrite(out[0].data.data(), 4, out[0].data.size(), f);
  std::fclose(f);
  for (float v : out[0].data) EXPECT(std::isfinite(v));
  EXPECT(be.lastInferMs() > 0.0);
  // device(): the members infvino::DeviceInfo has, read the way infvino_bench.cpp:89-97 does
  const auto & dev = be.device();
  std::printf("devices    :");
  for (const auto & d : dev.available) std::printf(" %s", d.c_str());
  std::printf("\nrequested  : %s -> resolved: %s%s (%s), %u CUs, %u MHz, %s\n", dev.requested.c_str(),
              dev.resolved.c_str(), dev.fell_back_to_cpu ? "  [CPU FALLBACK]" : "", dev.full_name.c_str(), dev.eu,
              dev.clock_mhz, dev.opencl_version.c_str());
  EXPECT(dev.eu > 0 && !dev.available.empty() && !dev.fell_back_to_cpu);
  EXPECT(dev.requested == "GPU.0" && dev.resolved == "GPU.0" && dev.opencl_version.rfind("HIP ", 0) == 0);
  // single image through infer equals image 0 of the batch
  auto one = be.infer(x.data(), n);
  EXPECT(one[0].shape == be.outputShapes()[0]);
  EXPECT(one[0].data.size() * 2 == out[0].data.size());
  EXPECT(std::memcmp(one[0].data.data(), out[0].data.data(), one[0].data.size() * 4) == 0);
  // and image 1 of the batch, sliced back out, equals image 1 run alone
  auto img1 = infvino_hip::HipBackend::image(out, 1, 2);
  auto one1 = be.infer(x.data() + n, n);
  EXPECT(img1[0].shape == one1[0].shape);
  EXPECT(std::memcmp(img1[0].data.data(), one1[0].data.data(), one1[0].data.size() * 4) == 0);
  // profiling = true (ClBackend(info, true)): per-node device times accumulate over infers
  {
    infvino_hip::HipBackend prof(info, true, 1, IVH_FLAG_NO_SPLITK);
    prof.infer(x.data(), n);
    prof.infer(x.data(), n);
    auto rows = prof.model().profile();
    int launched = 0;
    double total = 0.0;
    for (const auto & r : rows) {
      EXPECT(r.calls == 0 || r.calls == 2);
      launched += r.calls > 0;
      total += r.ms;
    }
    EXPECT(launched > 10 && total > 0.0);
    EXPECT(!prof.model().opProfile().empty());
    auto p1 = prof.infer(x.data(), n);
    EXPECT(std::memcmp(p1[0].data.data(), one[0].data.data(), one[0].data.size() * 4) == 0);
    prof.model().clearProfile();
    for (const auto & r : prof.model().profile()) EXPECT(r.calls == 0 && r.ms == 0.0);
  }
  // a CPU device request cannot be served by a GPU-only backend
  threw = false;
  try {
    ModelInfoLike cpu = info;
    cpu.device = "CPU";
    infvino_hip::HipBackend bad(cpu);
  } catch (const std::runtime_error & e) {
    threw = std::string(e.what()).find("HIP GPUs only") != std::string::npos;
  }
  EXPECT(threw);
  threw = false;
  try {
    be.infer(x.data(), n + 1);
  } catch (const std::runtime_error & e) {
    threw = std::string(e.what()).find("input numel mismatch") != std::string::npos;
  }
  EXPECT(threw);
  // PlanModel surface: fp16 in/out, readTensor of an unknown name
  infvino_hip::HipPlanModel pm(argv[1], 0, 1);
  std::vector<uint16_t> h(pm.inputNumel(), 0x3800);  // 0.5
  pm.setInput(h.data());
  pm.run();
  std::vector<uint16_t> o(pm.outputNumel(0));
  pm.readOutput(0, o.data());
  EXPECT(!pm.readTensor("no_such_tensor", o.data()));
  auto rows = pm.profile(1, 1);
  EXPECT(!rows.empty());
  // malformed plan -> std::runtime_error with the reference's message
  threw = false;
  try {
    infvino_hip::HipPlanModel bad(argv[3], 0, 1);
  } catch (const std::runtime_error & e) {
    threw = std::string(e.what()).find("plan has no 'output' line") != std::string::npos;
  }
  EXPECT(threw);
  std::printf("test_backend OK\n");
  return 0;
}
