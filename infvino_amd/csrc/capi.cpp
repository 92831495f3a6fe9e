// C ABI (include/ivh.h) over ivh::Model.  Every entry point converts exceptions into a
// status code plus a thread-local message, as the reference's callers expect a
// std::runtime_error message (src/ClBackend.cpp:16-18,36-39; src/PlanModel.cpp:437,498,536-539).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/ivh.h"
#include "conv_pack.hpp"
#include "executor.hpp"
#include "kernels.hpp"

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
// ---- single-op helpers
ivh::ConvSpec conv_spec(const ivh_conv_desc * d, bool gemv)
{
  if (!d) throw std::invalid_argument("null conv descriptor");
  if (d->cin < 1 || d->cout < 1 || d->h < 1 || d->w < 1 || d->k < 1 || d->stride < 1 || d->pad < 0 ||
      d->groups < 1 || d->cin % d->groups || d->cout % d->groups || d->act < 0 || d->act > 5)
    throw std::invalid_argument("conv descriptor: bad geometry");
  ivh::ConvSpec s;
  s.Cin = d->cin; s.Cout = d->cout; s.H = d->h; s.W = d->w;
  s.K = d->k; s.S = d->stride; s.P = d->pad; s.G = d->groups;
  s.act = d->act;
  s.has_bias = d->has_bias != 0;
  s.x_nhwc = d->channels_last != 0;
  s.x_vec1 = gemv && d->cin % 8 == 0;
  if (s.Ho() < 1 || s.Wo() < 1) throw std::invalid_argument("conv descriptor: empty output");
  return s;
}

ivh::View tensor_view(const void * ptr, int C, int H, int W, bool nhwc)
{
  ivh::View v;
  v.ptr = static_cast<__half *>(const_cast<void *>(ptr));
  v.layout = nhwc ? ivh::kNHWC : ivh::kNCHW;
  const int cs8 = (C + 7) / 8 * 8;
  v.cs = nhwc ? cs8 : H * W;
  v.img = nhwc ? (long)H * W * cs8 : (long)C * H * W;
  return v;
}

void check_launch(const char * what)
{
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) throw std::runtime_error(std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
}

void check_batch(int batch)
{
  if (batch < 1 || batch > 65535) throw std::invalid_argument("batch must be in [1, 65535]");
}

void run_conv(const ivh_conv_desc * d, bool gemv, bool dw_only, const void * x, const void * packed, const void * res,
              void * y, int batch, void * stream)
{
  const ivh::ConvSpec s = conv_spec(d, gemv);
  const ivh::ConvPacking pk = ivh::conv_packing(s);
  if (dw_only && pk.family != ivh::kFamDw) throw std::invalid_argument("not a depthwise conv (groups == cin == cout, k 3/5)");
  if (gemv && (s.H != 1 || s.W != 1 || s.K != 1 || s.G != 1 || s.P != 0)) throw std::invalid_argument("gemv descriptor");
  check_batch(batch);
  if (!x || !packed || !y) throw std::invalid_argument("null operand");
  ivh::ConvParams p;
  p.batch = batch;
  p.Cin = s.Cin; p.H = s.H; p.W = s.W;
  p.Cout = s.Cout; p.Ho = s.Ho(); p.Wo = s.Wo();
  p.K = s.K; p.S = s.S; p.P = s.P; p.G = s.G;
  p.act = s.act;
  p.x = tensor_view(x, s.Cin, s.H, s.W, s.x_nhwc);
  p.y = tensor_view(y, s.Cout, p.Ho, p.Wo, s.x_nhwc);
  if (res) p.r = tensor_view(res, s.Cout, p.Ho, p.Wo, s.x_nhwc);
  if (gemv) {  // [batch][n] rows: one pixel per image, presented channels-last
    for (ivh::View * v : {&p.x, &p.y, &p.r}) {
      if (!v->ptr) continue;
      const int C = v == &p.x ? s.Cin : s.Cout;
      v->layout = ivh::kNHWC;
      v->cs = (C + 7) / 8 * 8;
      v->img = C;
    }
  }
  const int k = ivh::conv_resolve(s, pk, packed, batch, nullptr, p);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (k == ivh::kLaunchIgemm) ivh::launch_conv_igemm(p, st);
  else if (k == ivh::kLaunchDirect) ivh::launch_conv_direct(p, st);
  else ivh::launch_dwconv(p, st);
  check_launch("conv");
}

ivh::View flat_view(const void * ptr, long n)
{
  ivh::View v;
  v.ptr = static_cast<__half *>(const_cast<void *>(ptr));
  v.layout = ivh::kNCHW;
  v.cs = (int)n;
  v.img = n;
  return v;
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

int ivh_runtime_version(char * buf, size_t len)
{
  return guard([&] {
    if (!buf || len == 0) throw std::invalid_argument("null buffer");
    int rt = 0, drv = 0;
    if (hipRuntimeGetVersion(&rt) != hipSuccess || hipDriverGetVersion(&drv) != hipSuccess)
      throw std::runtime_error("HIP error: no HIP runtime / driver version");
    // HIP_VERSION encoding: major * 10^7 + minor * 10^5 + patch
    const std::string v = "HIP " + std::to_string(rt / 10000000) + "." + std::to_string(rt / 100000 % 100) + "." +
                          std::to_string(rt % 100000) + ", driver " + std::to_string(drv);
    std::snprintf(buf, len, "%s", v.c_str());
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
int ivh_set_input_f32_noalloc(ivh_model * m, const float * host, int batch)
{
  return guard([&] {
    if (!host) throw std::invalid_argument("null input");
    M(m).setInputF32TruncNoAlloc(host, batch);
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
int ivh_node_times(const ivh_model * m, double * ms, int * calls, int cap)
{
  return guard([&] {
    std::vector<double> t;
    std::vector<int> c;
    M(m).nodeTimes(t, c);
    if (cap < (int)t.size()) throw std::invalid_argument("node_times capacity too small");
    for (size_t i = 0; i < t.size(); ++i) {
      if (ms) ms[i] = t[i];
      if (calls) calls[i] = c[i];
    }
  });
}

int ivh_clear_profile(ivh_model * m)
{
  return guard([&] { M(m).clearProfile(); });
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
int ivh_node_tag(ivh_model * m, int i, char * tag, size_t tag_len)
{
  return guard([&] {
    M(m).nodeStat(i);  // range check
    const std::string t = M(m).nodeTag(i);
    if (!tag || tag_len == 0) return;
    std::strncpy(tag, t.c_str(), tag_len - 1);
    tag[tag_len - 1] = 0;
  });
}
int ivh_memory_info(const ivh_model * m, int batch, size_t * arena_bytes, size_t * weight_bytes)
{
  return guard([&] {
    if (arena_bytes) *arena_bytes = M(m).arenaBytes(batch);
    if (weight_bytes) *weight_bytes = M(m).weightBytes();
  });
}

int ivh_conv_out_dims(const ivh_conv_desc * d, int * ho, int * wo)
{
  return guard([&] {
    const ivh::ConvSpec s = conv_spec(d, false);
    if (ho) *ho = s.Ho();
    if (wo) *wo = s.Wo();
  });
}

int ivh_conv_packed_bytes(const ivh_conv_desc * d, size_t * bytes)
{
  return guard([&] {
    if (!bytes) throw std::invalid_argument("null bytes");
    *bytes = ivh::conv_packing(conv_spec(d, d && d->h == 1 && d->w == 1 && d->k == 1)).bytes;
  });
}

int ivh_pack_conv_weights(const ivh_conv_desc * d, const uint16_t * w_host, const uint16_t * bias_host,
                          void * packed_dev)
{
  return guard([&] {
    const ivh::ConvSpec s = conv_spec(d, d && d->h == 1 && d->w == 1 && d->k == 1);
    if (!w_host || !packed_dev) throw std::invalid_argument("null operand");
    if (s.has_bias && !bias_host) throw std::invalid_argument("has_bias set but bias is null");
    const ivh::ConvPacking pk = ivh::conv_packing(s);
    std::vector<uint8_t> blob;
    ivh::conv_pack(s, pk, w_host, s.has_bias ? bias_host : nullptr, blob);
    const hipError_t e = hipMemcpy(packed_dev, blob.data(), blob.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(e));
  });
}

int ivh_conv2d_f16(const ivh_conv_desc * d, const void * x, const void * packed, const void * res, void * y,
                   int batch, void * stream)
{
  return guard([&] { run_conv(d, false, false, x, packed, res, y, batch, stream); });
}

int ivh_dwconv_f16(const ivh_conv_desc * d, const void * x, const void * packed, const void * res, void * y,
                   int batch, void * stream)
{
  return guard([&] { run_conv(d, false, true, x, packed, res, y, batch, stream); });
}

int ivh_gemv_f16(const ivh_conv_desc * d, const void * x, const void * packed, void * y, int batch, void * stream)
{
  return guard([&] { run_conv(d, true, false, x, packed, nullptr, y, batch, stream); });
}

int ivh_eltwise_f16(int op, const void * a, const void * b, int b_scalar, void * y, size_t n, int batch,
                    void * stream)
{
  return guard([&] {
    check_batch(batch);
    if (!a || !y) throw std::invalid_argument("null operand");
    if (n < 1 || n > (size_t)INT32_MAX) throw std::invalid_argument("element count out of range");
    if (b ? (op < 0 || op > 3) : (op < 0 || op > 5)) throw std::invalid_argument("bad eltwise op");
    ivh::SmallParams q;
    q.batch = batch;
    q.C = 1; q.H = 1; q.W = (int)n;
    q.n = (long)n;
    q.op = op;
    q.a = flat_view(a, (long)n);
    q.y = flat_view(y, (long)n);
    int kind = ivh::kEwUnary;
    if (b) {
      q.b = flat_view(b, (long)n);
      if (b_scalar) { q.b.img = 0; q.b.cs = 0; }
      kind = ivh::kEwSame;
    }
    ivh::launch_small(kind, q, static_cast<hipStream_t>(stream));
    check_launch("eltwise");
  });
}

int ivh_pool_f16(int kind, const void * x, void * y, int c, int h, int w, int k, int s, int p, int batch,
                 void * stream)
{
  return guard([&] {
    check_batch(batch);
    if (!x || !y) throw std::invalid_argument("null operand");
    if (c < 1 || h < 1 || w < 1 || s < 1 || (kind != 0 && kind != 1)) throw std::invalid_argument("bad pool geometry");
    ivh::SmallParams q;
    q.batch = batch;
    q.C = c; q.H = h; q.W = w;
    if (kind == 0) {
      if (k < 1 || p < 0 || p >= k) throw std::invalid_argument("bad maxpool window");
      q.K = k; q.S = s; q.P = p;
      q.Ho = (h + 2 * p - k) / s + 1;
      q.Wo = (w + 2 * p - k) / s + 1;
      if (q.Ho < 1 || q.Wo < 1) throw std::invalid_argument("empty maxpool output");
    } else {
      q.i0 = s;
      q.Ho = h * s;
      q.Wo = w * s;
    }
    q.a = tensor_view(x, c, h, w, false);
    q.y = tensor_view(y, c, q.Ho, q.Wo, false);
    ivh::launch_small(kind == 0 ? ivh::kMaxPool : ivh::kResizeNN, q, static_cast<hipStream_t>(stream));
    check_launch("pool");
  });
}

int ivh_softmax_f16(const void * x, void * y, int outer, int axis, int inner, int batch, void * stream)
{
  return guard([&] {
    check_batch(batch);
    if (!x || !y) throw std::invalid_argument("null operand");
    if (outer < 1 || axis < 1 || inner < 1 || (long)outer * axis * inner > INT32_MAX)
      throw std::invalid_argument("bad softmax geometry");
    ivh::SmallParams q;
    q.batch = batch;
    q.i0 = outer; q.i1 = axis; q.i2 = inner;
    const long n = (long)outer * axis * inner;
    q.C = 1; q.H = 1; q.W = (int)n;
    q.n = n;
    q.a = flat_view(x, n);
    q.y = flat_view(y, n);
    ivh::launch_small(ivh::kSoftmax, q, static_cast<hipStream_t>(stream));
    check_launch("softmax");
  });
}

int ivh_bmm_f16(const void * a, const void * b, void * y, int bb, int m, int k, int n, int batch, void * stream)
{
  return guard([&] {
    check_batch(batch);
    if (!a || !b || !y) throw std::invalid_argument("null operand");
    if (bb < 1 || m < 1 || k < 1 || n < 1 || (long)bb * m * n > INT32_MAX || (long)bb * m * k > INT32_MAX ||
        (long)bb * k * n > INT32_MAX)
      throw std::invalid_argument("bad bmm geometry");
    ivh::SmallParams q;
    q.batch = batch;
    q.i0 = bb; q.i1 = m; q.i2 = k; q.i3 = n;
    q.a = flat_view(a, (long)bb * m * k);
    q.b = flat_view(b, (long)bb * k * n);
    q.y = flat_view(y, (long)bb * m * n);
    q.C = 1; q.H = 1; q.W = bb * m * n;
    q.n = (long)bb * m * n;
    ivh::launch_small(ivh::kBmm, q, static_cast<hipStream_t>(stream));
    check_launch("bmm");
  });
}

}  // extern "C"
