// HipBackend: drop-in for infvino::ClBackend (include/infvino/ClBackend.hpp:29-53,
// src/ClBackend.cpp:13-65 of the reference) on one MI355X.
//   * constructed from the same ModelInfo (any type with `plan` and `device` string
//     members; "AUTO", "GPU" and "GPU.<n>" pick HIP device 0 / 0 / n) and the same
//     `bool profiling` (ClBackend(const ModelInfo&, bool profiling = false)): with profiling
//     every infer runs node by node and adds each node's device time to model().profile(),
//     as the reference's profiling PlanModel does; or from a plan path;
//   * infer(const float* input, size_t numel) -> std::vector<Tensor>: f32 NCHW in, the
//     reference's truncating f32 -> f16 conversion (done on the device), fp16 compute,
//     f32 Tensors out; numel must equal prod(inputDims()) (throws "input numel mismatch"
//     otherwise), or a multiple B <= maxBatch of it, in which case the outputs carry B
//     images along dim 0 (image(outputs, b, B) slices image b back out for per-image
//     decoders);
//   * device() returns a DeviceInfo with the members of infvino::DeviceInfo
//     (include/infvino/Device.hpp:16-26), so InferenceEngine::device() and the tools that
//     print it bind unchanged; built with INFVINO_HIP_USE_INFVINO_TENSOR inside the
//     reference tree it is infvino::DeviceInfo itself;
//   * infer serialised by a mutex so Sessions can share one backend (ClBackend.cpp:33).
#ifndef INFVINO_HIP_BACKEND_HPP_
#define INFVINO_HIP_BACKEND_HPP_

#include <chrono>
#include <cstddef>
#include <stdexcept>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "infvino_hip/HipPlanModel.hpp"
#include "infvino_hip/Tensor.hpp"

#ifdef INFVINO_HIP_USE_INFVINO_TENSOR
#include "infvino/Device.hpp"
namespace infvino_hip { using DeviceInfo = infvino::DeviceInfo; }
#else
namespace infvino_hip
{
/** The members of infvino::DeviceInfo (include/infvino/Device.hpp:16-26). */
struct DeviceInfo
{
  std::vector<std::string> available;  ///< every HIP device, "GPU.<n> (<name>)"
  std::string requested;               ///< the ModelInfo device string ("AUTO", "GPU", "GPU.1", ...)
  std::string resolved;                ///< device actually used, e.g. "GPU.0"
  std::string full_name;               ///< HIP device name
  bool fell_back_to_cpu = false;       ///< always false: there is no CPU path
  std::string opencl_version;          ///< the runtime in use: "HIP <version>, driver <version>"
  unsigned eu = 0;                     ///< compute units
  unsigned clock_mhz = 0;
};
}  // namespace infvino_hip
#endif

namespace infvino_hip
{

using HipDeviceInfo = DeviceInfo;

class HipBackend
{
public:
  explicit HipBackend(const std::string & plan, int device = 0, int max_batch = 1, uint32_t flags = 0,
                      const std::string & requested = "AUTO", bool profiling = false)
  {
    if (plan.empty())
      throw std::runtime_error("HipBackend: ModelInfo.plan is empty. Generate it first with "
                               "scripts/onnx2plan.py --onnx <model.onnx> --out-dir models");
    model_ = std::make_unique<HipPlanModel>(plan, device, max_batch, flags, profiling);
    input_dims_ = model_->inputDims();
    for (size_t i = 0; i < model_->outputCount(); ++i) output_shapes_.push_back(model_->outputDims(i));
    describe(device, requested);
  }

  /** ClBackend(const ModelInfo&, bool profiling = false): info.plan, info.device. */
  template <class Info, class = decltype(std::declval<const Info &>().plan)>
  explicit HipBackend(const Info & info, bool profiling = false)
  : HipBackend(info.plan, deviceIndex(info.device), 1, 0, info.device, profiling)
  {
  }

  /** An int second argument is rejected at compile time: it would otherwise convert to
   * `profiling` (an older signature took a maximum batch there). */
  template <class Info, class = decltype(std::declval<const Info &>().plan)>
  HipBackend(const Info & info, int) = delete;

  /** The same with a maximum batch (images per infer) and ivh.h flags. */
  template <class Info, class = decltype(std::declval<const Info &>().plan)>
  HipBackend(const Info & info, bool profiling, int max_batch, uint32_t flags = 0)
  : HipBackend(info.plan, deviceIndex(info.device), max_batch, flags, info.device, profiling)
  {
  }

  const std::vector<int64_t> & inputDims() const { return input_dims_; }
  const std::vector<std::vector<int64_t>> & outputShapes() const { return output_shapes_; }
  const DeviceInfo & device() const { return device_; }
  double lastInferMs() const { return last_infer_ms_; }
  HipPlanModel & model() { return *model_; }

  std::vector<Tensor> infer(const float * input_f32, size_t numel)
  {
    std::lock_guard<std::mutex> lock(mutex_);
    const size_t per = model_->inputNumel();
    if (numel == 0 || numel % per != 0 || numel / per > static_cast<size_t>(model_->maxBatch()))
      throw std::runtime_error("HipBackend: input numel mismatch: got " + std::to_string(numel) +
                               ", expected " + std::to_string(per));
    const int batch = static_cast<int>(numel / per);
    const auto t0 = std::chrono::steady_clock::now();
    model_->setInputF32(input_f32, batch);
    model_->run(batch);
    last_infer_ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    std::vector<Tensor> outputs;
    outputs.reserve(model_->outputCount());
    for (size_t i = 0; i < model_->outputCount(); ++i) {
      Tensor t;
      t.shape = model_->outputDims(i);
      if (batch > 1 && !t.shape.empty()) t.shape[0] *= batch;
      t.data.resize(model_->outputNumel(i) * batch);
      model_->readOutputF32(i, t.data.data(), batch);
      outputs.push_back(std::move(t));
    }
    return outputs;
  }

  /** Image b of outputs that infer() returned for a batch: every tensor's dim 0 back to one
   *  image, so per-image consumers (the reference's PoseDecoder / nms, which read a
   *  [1, C, N] tensor) run unchanged on each image of a batched inference. */
  static std::vector<Tensor> image(const std::vector<Tensor> & batched, int b, int batch)
  {
    if (batch < 1 || b < 0 || b >= batch) throw std::runtime_error("HipBackend: image index out of range");
    std::vector<Tensor> out;
    out.reserve(batched.size());
    for (const Tensor & t : batched) {
      if (t.shape.empty() || t.shape[0] % batch != 0 || t.data.size() % static_cast<size_t>(batch) != 0)
        throw std::runtime_error("HipBackend: tensor does not hold the batch");
      const size_t per = t.data.size() / static_cast<size_t>(batch);
      Tensor u;
      u.shape = t.shape;
      u.shape[0] /= batch;
      u.data.assign(t.data.begin() + static_cast<std::ptrdiff_t>(per * b),
                    t.data.begin() + static_cast<std::ptrdiff_t>(per * (b + 1)));
      out.push_back(std::move(u));
    }
    return out;
  }

private:
  /** "AUTO" / "GPU" -> 0, "GPU.<n>" -> n; a CPU request cannot be served (no CPU path). */
  static int deviceIndex(const std::string & dev)
  {
    if (dev.rfind("CPU", 0) == 0)
      throw std::runtime_error("HipBackend: device '" + dev + "' requested; this backend runs on HIP GPUs only");
    const auto p = dev.find('.');
    return p == std::string::npos ? 0 : std::atoi(dev.c_str() + p + 1);
  }

  void describe(int device, const std::string & requested)
  {
    int n = 0;
    check(ivh_device_count(&n));
    char name[256] = {0};
    int cu = 0, mhz = 0;
    for (int i = 0; i < n; ++i) {
      check(ivh_device_info(i, name, sizeof name, &cu, &mhz));
      device_.available.push_back("GPU." + std::to_string(i) + " (" + name + ")");
    }
    check(ivh_device_info(device, name, sizeof name, &cu, &mhz));
    device_.requested = requested;
    device_.resolved = "GPU." + std::to_string(device);
    device_.full_name = name;
    device_.fell_back_to_cpu = false;
    char ver[128] = {0};
    check(ivh_runtime_version(ver, sizeof ver));
    device_.opencl_version = ver;
    device_.eu = static_cast<unsigned>(cu);
    device_.clock_mhz = static_cast<unsigned>(mhz);
  }

  std::unique_ptr<HipPlanModel> model_;
  std::vector<int64_t> input_dims_;
  std::vector<std::vector<int64_t>> output_shapes_;
  DeviceInfo device_;
  double last_infer_ms_ = 0.0;
  std::mutex mutex_;
};

}  // namespace infvino_hip

#endif  // INFVINO_HIP_BACKEND_HPP_
