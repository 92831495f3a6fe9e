// HipPlanModel: the plan executor on one MI355X, with the public surface of
// infvino::PlanModel (include/infvino/PlanModel.hpp:57-234 of the reference).  Header-only
// wrapper over the C ABI in ivh.h; every failure throws std::runtime_error carrying the
// message the reference would throw (missing tensor, missing input/output line, unknown
// op, missing init file, ...).
//
// Differences from PlanModel, all additive:
//   * the constructor takes a device index, a maximum batch and ivh.h flags instead of an
//     OpenCL kernel directory / platform; `profiling` keeps its meaning: per-node device
//     times accumulate over run() calls (profile(), opProfile(), clearProfile());
//   * setInput / run / readOutput / readTensor take a batch count B (default 1): B images
//     stored back to back, each laid out exactly as the plan's batch-1 tensor.
// Single-threaded, like PlanModel (PlanModel.hpp:36); HipBackend adds the mutex.
#ifndef INFVINO_HIP_PLAN_MODEL_HPP_
#define INFVINO_HIP_PLAN_MODEL_HPP_

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "ivh.h"

namespace infvino_hip
{

inline void check(int rc)
{
  if (rc != IVH_OK) throw std::runtime_error(ivh_last_error());
}

class HipPlanModel
{
public:
  explicit HipPlanModel(const std::string & plan_path, int device = 0, int max_batch = 1, uint32_t flags = 0,
                        bool profiling = false)
  : plan_path_(plan_path), profiling_(profiling)
  {
    if (profiling) flags |= IVH_FLAG_PROFILE;
    check(ivh_create(plan_path.c_str(), device, max_batch, flags, &m_));
    input_dims_ = dims([&](int64_t * d, int * r) { return ivh_input_dims(m_, d, r); });
    int n = 0;
    check(ivh_output_count(m_, &n));
    for (int i = 0; i < n; ++i)
      output_dims_.push_back(dims([&](int64_t * d, int * r) { return ivh_output_dims(m_, i, d, r); }));
    max_batch_ = max_batch;
  }
  ~HipPlanModel() { ivh_destroy(m_); }
  HipPlanModel(const HipPlanModel &) = delete;
  HipPlanModel & operator=(const HipPlanModel &) = delete;

  const std::string & planPath() const { return plan_path_; }
  const std::vector<int64_t> & inputDims() const { return input_dims_; }
  size_t inputNumel() const { return numel(input_dims_); }
  size_t outputCount() const { return output_dims_.size(); }
  const std::vector<int64_t> & outputDims(size_t i) const { return output_dims_.at(i); }
  size_t outputNumel(size_t i) const { return numel(output_dims_.at(i)); }
  int maxBatch() const { return max_batch_; }

  /** Fills the graph input from `batch` fp16 images (inputNumel() each). */
  void setInput(const void * fp16_host, int batch = 1)
  {
    check(ivh_set_input_f16(m_, static_cast<const uint16_t *>(fp16_host), batch));
  }
  /** f32 input, converted on the device with the reference's truncating f32 -> f16. */
  void setInputF32(const float * host, int batch = 1) { check(ivh_set_input_f32(m_, host, batch)); }
  void run(int batch = 1) { check(ivh_run(m_, batch)); }
  void readOutput(size_t i, void * fp16_host, int batch = 1)
  {
    check(ivh_read_output_f16(m_, static_cast<int>(i), static_cast<uint16_t *>(fp16_host), batch));
  }
  void readOutputF32(size_t i, float * host, int batch = 1)
  {
    check(ivh_read_output_f32(m_, static_cast<int>(i), host, batch));
  }
  /** Any declared tensor as NCHW fp16; false when no tensor has that name. */
  bool readTensor(const std::string & name, void * fp16_host, int batch = 1) const
  {
    if (tensorNumel(name) == 0) return false;
    check(ivh_read_tensor_f16(m_, name.c_str(), static_cast<uint16_t *>(fp16_host), batch));
    return true;
  }
  size_t tensorNumel(const std::string & name) const
  {
    size_t n = 0;
    check(ivh_tensor_numel(m_, name.c_str(), &n));
    return n;
  }
  double lastRunMs() const
  {
    double ms = 0;
    check(ivh_last_run_ms(m_, &ms));
    return ms;
  }

  bool profiling() const { return profiling_; }

  struct NodeRow
  {
    int index = 0;
    std::string op, kernel, tag;
    std::string launch;  // kernel label and launch detail (ivh_node_tag)
    double ms = 0.0, flops = 0.0, bytes = 0.0;
    int calls = 0;
  };
  /** PlanModel::profile().nodes: per-node device time summed over the run() calls since
   *  construction or clearProfile() (profiling models only; zeros otherwise), with the
   *  number of runs that launched the node. */
  std::vector<NodeRow> profile() const
  {
    int n = 0;
    check(ivh_node_count(m_, &n));
    std::vector<double> ms(n);
    std::vector<int> calls(n);
    check(ivh_node_times(m_, ms.data(), calls.data(), n));
    std::vector<NodeRow> rows = describeNodes(n);
    for (int i = 0; i < n; ++i) {
      rows[i].ms = ms[i];
      rows[i].calls = calls[i];
    }
    return rows;
  }
  /** PlanModel::opProfile(): plan op -> {summed ms, summed launches} over profiled runs. */
  std::map<std::string, std::pair<double, int>> opProfile() const
  {
    std::map<std::string, std::pair<double, int>> out;
    for (const NodeRow & r : profile()) {
      if (r.calls == 0) continue;
      auto & e = out[r.op];
      e.first += r.ms;
      e.second += r.calls;
    }
    return out;
  }
  void clearProfile() { check(ivh_clear_profile(m_)); }

  /** Measured on demand: each node `iters` times back to back between two HIP events on the
   *  model stream (any model), mean ms per run. */
  std::vector<NodeRow> profile(int batch, int iters = 5)
  {
    int n = 0;
    check(ivh_node_count(m_, &n));
    std::vector<double> ms(n);
    check(ivh_profile_nodes(m_, batch, iters, ms.data(), n));
    std::vector<NodeRow> rows = describeNodes(n);
    for (int i = 0; i < n; ++i) {
      rows[i].ms = ms[i];
      rows[i].calls = iters;
    }
    return rows;
  }

private:
  std::vector<NodeRow> describeNodes(int n) const
  {
    std::vector<NodeRow> rows(n);
    for (int i = 0; i < n; ++i) {
      char op[64], kern[64], desc[256];
      check(ivh_node_info(m_, i, op, sizeof op, kern, sizeof kern, desc, sizeof desc, &rows[i].flops, &rows[i].bytes));
      rows[i].index = i;
      rows[i].op = op;
      rows[i].kernel = kern;
      rows[i].tag = desc;
      char lt[256];
      check(ivh_node_tag(m_, i, lt, sizeof lt));
      rows[i].launch = lt;
    }
    return rows;
  }

  template <class F>
  static std::vector<int64_t> dims(F f)
  {
    int64_t d[8];
    int r = 8;
    check(f(d, &r));
    return std::vector<int64_t>(d, d + r);
  }
  static size_t numel(const std::vector<int64_t> & d)
  {
    size_t n = 1;
    for (auto v : d) n *= static_cast<size_t>(v < 0 ? 0 : v);
    return n;
  }

  ivh_model * m_ = nullptr;
  std::string plan_path_;
  std::vector<int64_t> input_dims_;
  std::vector<std::vector<int64_t>> output_dims_;
  int max_batch_ = 1;
  bool profiling_ = false;
};

}  // namespace infvino_hip

#endif  // INFVINO_HIP_PLAN_MODEL_HPP_
