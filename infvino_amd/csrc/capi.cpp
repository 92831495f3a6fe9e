// C ABI (include/ivh.h) over ivh::Model.  Every entry point converts exceptions into a
// status code plus a thread-local message, as the reference's callers expect a
// std::runtime_error message (src/ClBackend.cpp:16-18,36-39; src/PlanModel.cpp:437,498,536-539).
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>

#include "../../include/ivh.h"
#include "executor.hpp"

struct ivh_model {
  ivh::Model * m = nullptr;
};

namespace {
thread_local std::string g_err;

template <class F>
int guard(F && f)
{
  try {
    f();
    return IVH_OK;
  } catch (const std::invalid_argument & e) {
    g_err = e.what();
    return IVH_ERR_INVALID;
  } catch (const std::runtime_error & e) {
    g_err = e.what();
    return std::strncmp(e.what(), "HIP error", 9) == 0 ? IVH_ERR_DEVICE : IVH_ERR_INVALID;
  } catch (const std::exception & e) {
    g_err = e.what();
    return IVH_ERR_INTERNAL;
  } catch (...) {
    g_err = "unknown error";
    return IVH_ERR_INTERNAL;
  }
}

ivh::Model & M(const ivh_model * m)
{
  if (!m || !m->m) throw std::invalid_argument("null model handle");
  return *m->m;
}

void dims_out(const std::vector<int64_t> & d, int64_t * dims, int * rank)
{
  if (!rank) throw std::invalid_argument("null rank");
  if (dims) {
    if (*rank < (int)d.size()) throw std::invalid_argument("dims capacity too small");
    for (size_t i = 0; i < d.size(); ++i) dims[i] = d[i];
  }
  *rank = (int)d.size();
}
}  // namespace

extern "C" {

const char * ivh_last_error(void) { return g_err.c_str(); }

int ivh_version(int * major, int * minor)
{
  return guard([&] {
    if (major) *major = 0;
    if (minor) *minor = 1;
  });
}

int ivh_device_count(int * n)
{
  return guard([&] {
    int c = 0;
    const hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) c = 0;
    *n = c;
  });
}

int ivh_device_info(int device, char * name, size_t name_len, int * compute_units, int * clock_mhz)
{
  return guard([&] {
    auto chk = [](hipError_t e) {
      if (e != hipSuccess) throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e));
    };
    int cu = 0, clk = 0;
    chk(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, device));
    chk(hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, device));
    if (compute_units) *compute_units = cu;
    if (clock_mhz) *clock_mhz = clk / 1000;
    if (name && name_len) {
      char buf[256] = {0};
      chk(hipDeviceGetName(buf, sizeof buf, device));
      if (!buf[0]) {
        hipDeviceProp_t prop;
        chk(hipGetDeviceProperties(&prop, device));
        std::strncpy(buf, prop.gcnArchName, sizeof buf - 1);
      }
      std::strncpy(name, buf, name_len - 1);
      name[name_len - 1] = 0;
    }
  });
}

int ivh_create(const char * plan_path, int device, int max_batch, uint32_t flags, ivh_model ** out)
{
  return guard([&] {
    if (!plan_path || !out) throw std::invalid_argument("null argument");
    *out = nullptr;
    auto * h = new ivh_model;
    try {
      h->m = new ivh::Model(plan_path, device, max_batch, flags);
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

int ivh_destroy(ivh_model * m)
{
  return guard([&] {
    if (!m) return;
    delete m->m;
    delete m;
  });
}

int ivh_input_dims(const ivh_model * m, int64_t * dims, int * rank)
{
  return guard([&] { dims_out(M(m).inputDims(), dims, rank); });
}
int ivh_input_numel(const ivh_model * m, size_t * numel)
{
  return guard([&] { *numel = M(m).inputNumel(); });
}
int ivh_output_count(const ivh_model * m, int * n)
{
  return guard([&] { *n = M(m).outputCount(); });
}
int ivh_output_dims(const ivh_model * m, int i, int64_t * dims, int * rank)
{
  return guard([&] {
    if (i < 0 || i >= M(m).outputCount()) throw std::invalid_argument("output index out of range");
    dims_out(M(m).outputDims(i), dims, rank);
  });
}
int ivh_output_numel(const ivh_model * m, int i, size_t * numel)
{
  return guard([&] {
    if (i < 0 || i >= M(m).outputCount()) throw std::invalid_argument("output index out of range");
    *numel = M(m).outputNumel(i);
  });
}
int ivh_max_batch(const ivh_model * m, int * max_batch)
{
  return guard([&] { *max_batch = M(m).maxBatch(); });
}
int ivh_set_input_f16(ivh_model * m, const uint16_t * host, int batch)
{
  return guard([&] {
    if (!host) throw std::invalid_argument("null input");
    M(m).setInputF16(host, batch);
  });
}
int ivh_set_input_f32(ivh_model * m, const float * host, int batch)
{
  return guard([&] {
    if (!host) throw std::invalid_argument("null input");
    M(m).setInputF32Trunc(host, batch);
  });
}
int ivh_run(ivh_model * m, int batch)
{
  return guard([&] { M(m).run(batch); });
}
int ivh_sync(ivh_model * m)
{
  return guard([&] { M(m).sync(); });
}
int ivh_read_output_f16(ivh_model * m, int i, uint16_t * host, int batch)
{
  return guard([&] {
    if (!host) throw std::invalid_argument("null output buffer");
    M(m).readOutputF16(i, host, batch);
  });
}
int ivh_read_output_f32(ivh_model * m, int i, float * host, int batch)
{
  return guard([&] {
    if (!host) throw std::invalid_argument("null output buffer");
    M(m).readOutputF32(i, host, batch);
  });
}
int ivh_read_tensor_f16(ivh_model * m, const char * name, uint16_t * host, int batch)
{
  return guard([&] {
    if (!name || !host) throw std::invalid_argument("null argument");
    if (!M(m).readTensorF16(name, host, batch)) throw std::invalid_argument(std::string("no such tensor: ") + name);
  });
}
int ivh_tensor_numel(const ivh_model * m, const char * name, size_t * numel)
{
  return guard([&] {
    if (!name) throw std::invalid_argument("null name");
    *numel = M(m).tensorNumel(name);
  });
}
int ivh_last_run_ms(const ivh_model * m, double * ms)
{
  return guard([&] { *ms = M(m).lastRunMs(); });
}
int ivh_node_count(ivh_model * m, int * n)
{
  return guard([&] { *n = M(m).nodeCount(); });
}
int ivh_profile_nodes(ivh_model * m, int batch, int iters, double * ms, int cap)
{
  return guard([&] {
    auto v = M(m).profileNodes(batch, iters);
    if (!ms || cap < (int)v.size()) throw std::invalid_argument("profile buffer too small");
    for (size_t i = 0; i < v.size(); ++i) ms[i] = v[i];
  });
}
int ivh_node_info(ivh_model * m, int i, char * op, size_t op_len, char * kernel, size_t kernel_len, char * desc,
                  size_t desc_len, double * flops, double * bytes)
{
  return guard([&] {
    const ivh::NodeStat & s = M(m).nodeStat(i);
    auto cp = [](char * dst, size_t n, const std::string & src) {
      if (!dst || n == 0) return;
      std::strncpy(dst, src.c_str(), n - 1);
      dst[n - 1] = 0;
    };
    cp(op, op_len, s.op);
    cp(kernel, kernel_len, M(m).nodeKernel(i));
    cp(desc, desc_len, s.desc);
    if (flops) *flops = s.flops;
    if (bytes) *bytes = s.bytes;
  });
}
int ivh_memory_info(const ivh_model * m, int batch, size_t * arena_bytes, size_t * weight_bytes)
{
  return guard([&] {
    if (arena_bytes) *arena_bytes = M(m).arenaBytes(batch);
    if (weight_bytes) *weight_bytes = M(m).weightBytes();
  });
}

}  // extern "C"
