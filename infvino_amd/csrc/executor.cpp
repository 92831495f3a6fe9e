// HIP-native plan executor (MI355X / gfx950).
//
// Mirrors src/PlanModel.cpp of the reference: parse (447-573), graph fusions (575-882),
// activation memory plan (884-1210), per-node dispatch (run, 3127-4178), readOutput /
// readTensor (4180-4200).  Designed for one GPU with a batch of B images:
//   * every node describes one image; B is folded into the kernels' outer grid axis
//     (implicit-GEMM convs fold it into M), inits are shared by all images;
//   * conv-domain tensors are stored channels-last (NHWC, pixel stride rounded up to 8)
//     so MFMA operands are 16-byte loads; tensors that feed reshape/softmax/permute/bmm
//     or broadcasting stay NCHW, exactly the plan's layout;
//   * concat along channels and channel splits are zero-copy: the producers of a
//     concat's inputs write straight into the concat buffer at their channel offset
//     (the conv "concat write-offset" epilogue); splits are views;
//   * residual adds fold into the producing conv's epilogue (act first, then +res);
//   * activations live in one arena, placed by liveness (best fit), sized per image;
//   * the whole plan is replayed as one captured HIP graph per batch size.
#include "executor.hpp"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <numeric>
#include <set>
#include <sstream>
#include <stdexcept>

#include "../../include/ivh.h"
#include "kernels.hpp"

namespace ivh {

#define HIPCHECK(expr)                                                                   \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e_) + " at " \
                               + #expr);                                                 \
  } while (0)

namespace {

long prod(const std::vector<int64_t> & d)
{
  long n = 1;
  for (auto v : d) n *= (v < 0 ? 0 : v);
  return n;
}
long round_up(long v, long m) { return (v + m - 1) / m * m; }

std::vector<std::string> split_csv(const std::string & s)
{
  std::vector<std::string> out;
  if (s == "-") return out;
  std::stringstream ss(s);
  std::string t;
  while (std::getline(ss, t, ',')) out.push_back(t);
  return out;
}

float h2f(uint16_t h)
{
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, f;
  if (exp == 0) {
    if (mant == 0) f = sign;
    else {
      int e = -14;
      while (!(mant & 0x400u)) { mant <<= 1; --e; }
      f = sign | ((uint32_t)(e + 127) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else if (exp == 31) f = sign | 0x7f800000u | (mant << 13);
  else f = sign | ((exp + 112u) << 23) | (mant << 13);
  float o;
  std::memcpy(&o, &f, 4);
  return o;
}

int unary_to_act(int op)  // ew_unary table (kernels/ops.cl:50-63) -> canonical codes
{
  static const int m[5] = {kActSigmoid, kActSiLU, kActReLU, kActHSwish, kActHSigmoid};
  return (op >= 0 && op < 5) ? m[op] : kActNone;
}

void check_batch(int batch, int maxb)
{
  if (batch < 1 || batch > maxb)
    throw std::runtime_error("batch " + std::to_string(batch) + " out of range [1, " + std::to_string(maxb) + "]");
}

}  // namespace

int PlanNode::i(const char * key, int def) const
{
  auto it = attr.find(key);
  return it == attr.end() ? def : std::atoi(it->second.c_str());
}
std::string PlanNode::str(const char * key) const
{
  auto it = attr.find(key);
  return it == attr.end() ? std::string() : it->second;
}

struct Model::Tensor {
  std::string name;
  std::vector<int64_t> dims;
  enum Kind { kInput, kInit, kAct } kind = kAct;
  std::string file;
  int producer = -1;
  std::vector<int> users;
  int C = 1, H = 1, W = 1;  // per-image geometry (channel axis 1)
  long numel = 1;
  int root = -1;            // activation storage root
  int coff = 0;             // channel offset in the root
  long eoff = 0;            // element offset in the root when it is NCHW
};

struct Model::Root {
  int C = 1, H = 1, W = 1;
  long numel = 1;
  int parent = -1;
  int pcoff = 0;
  bool reshaped = false, is_input = false, is_output = false, flat = false;
  int layout = kNCHW;
  int cs = 0;
  int cs_align = 8;  // channels-last pixel pitch rounded up to this many channels
  long per_image = 0;
  int first = INT_MAX, last = -1;
  long off1 = 0;
};

// ================================================================ construction

Model::Model(const std::string & plan_path, int device, int max_batch, uint32_t flags)
: plan_path_(plan_path), device_(device), max_batch_(max_batch), flags_(flags)
{
  if (max_batch < 1) throw std::runtime_error("max_batch must be >= 1");
  dry_ = (flags_ & IVH_FLAG_DRY_RUN) != 0;
  if (!dry_) {
    int ndev = 0;
    HIPCHECK(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev)
      throw std::runtime_error("device index " + std::to_string(device) + " out of range (" +
                               std::to_string(ndev) + " devices)");
    HIPCHECK(hipSetDevice(device));
  }
  const auto pos = plan_path.find_last_of('/');
  plan_dir_ = pos == std::string::npos ? std::string(".") : plan_path.substr(0, pos);
  parse(plan_path);
  if (!(flags_ & IVH_FLAG_NO_FUSE)) {
    fuseDecode();
    fuseResidual();
    fuseActivation();
    fusePermuteMatmul();
    fuseAttention();
  }
  findPairs();
  findSiblings();
  plan();
  if (!dry_) HIPCHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  allocate();
  uploadWeights();
  buildStats();
}

Model::~Model()
{
  if (dry_) return;
  (void)hipSetDevice(device_);
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto & g : graphs_) (void)hipGraphExecDestroy(g.second);
  for (auto & e : prof_ev_) (void)hipEventDestroy(e);
  for (const auto & a : allocs_) (void)hipFree(reinterpret_cast<void *>(a.first));
  if (stream_) (void)hipStreamDestroy(stream_);
}

// ====================================================================== parse
// Grammar of include/infvino/PlanModel.hpp:5-12; same errors as src/PlanModel.cpp:447-573.
void Model::parse(const std::string & path)
{
  std::ifstream f(path);
  if (!f) throw std::runtime_error("PlanModel: cannot open plan: " + path);
  std::string line;
  auto add = [&](const std::string & name, std::vector<int64_t> d, Tensor::Kind k) -> Tensor & {
    auto t = std::make_unique<Tensor>();
    t->name = name;
    t->dims = std::move(d);
    t->kind = k;
    t->numel = prod(t->dims);
    Tensor & ref = *t;
    T_[name] = std::move(t);
    return ref;
  };
  while (std::getline(f, line)) {
    if (line.empty() || line[0] == '#') continue;
    std::istringstream ls(line);
    std::string kind;
    ls >> kind;
    if (kind == "input" || kind == "tensor") {
      std::string name;
      std::vector<int64_t> d;
      ls >> name;
      int64_t v;
      while (ls >> v) d.push_back(v);
      add(name, d, kind == "input" ? Tensor::kInput : Tensor::kAct);
      if (kind == "input" && input_name_.empty()) {
        input_name_ = name;
        input_dims_ = d;
      } else if (kind == "input") {
        T_[name]->kind = Tensor::kAct;  // only the first input is the graph input
      }
    } else if (kind == "init") {
      std::string name, file;
      std::vector<int64_t> d;
      ls >> name >> file;
      int64_t v;
      while (ls >> v) d.push_back(v);
      Tensor & t = add(name, d, Tensor::kInit);
      t.file = (file.empty() || file[0] == '/') ? file : (plan_dir_ + "/" + file);
    } else if (kind == "node") {
      PlanNode n;
      std::string ins, outs;
      ls >> n.op >> ins >> outs;
      n.ins = split_csv(ins);
      n.outs = split_csv(outs);
      std::string kv;
      while (ls >> kv) {
        const auto p = kv.find('=');
        if (p != std::string::npos) n.attr[kv.substr(0, p)] = kv.substr(p + 1);
      }
      if (n.outs.empty()) throw std::runtime_error("PlanModel: node without output: " + line);
      nodes_.push_back(std::move(n));
    } else if (kind == "output") {
      std::string name;
      ls >> name;
      if (!name.empty()) outputs_.push_back(name);
    }
  }
  if (input_name_.empty()) throw std::runtime_error("PlanModel: plan has no 'input' line");
  if (outputs_.empty()) throw std::runtime_error("PlanModel: plan has no 'output' line");
  for (const auto & o : outputs_)
    if (!T_.count(o)) throw std::runtime_error("PlanModel: output tensor not declared: " + o);
  for (const auto & n : nodes_) {
    for (const auto & i : n.ins)
      if (i != "-" && !T_.count(i)) throw std::runtime_error("PlanModel: missing tensor: " + i);
    for (const auto & o : n.outs)
      if (o != "-" && !T_.count(o)) throw std::runtime_error("PlanModel: missing tensor: " + o);
  }
  for (auto & kv : T_) {
    Tensor & t = *kv.second;
    const auto & d = t.dims;
    if (d.size() >= 2) {
      t.C = (int)d[1];
      long hw = t.C > 0 ? t.numel / t.C : 0;
      t.H = d.size() >= 4 ? (int)d[2] : 1;
      t.W = t.H > 0 ? (int)(hw / t.H) : 0;
    } else {
      t.C = (int)t.numel;
      t.H = t.W = 1;
    }
  }
}

// ====================================================================== fusions

// conv + same-shape Add -> conv epilogue residual (act first, then +res), the reference's
// fuseResidualAdd (src/PlanModel.cpp:667-740) extended to conv3x3.
void Model::fuseResidual()
{
  std::map<std::string, int> producer, uses;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & o : nodes_[i].outs) producer[o] = (int)i;
  for (const auto & n : nodes_)
    for (const auto & in : n.ins)
      if (in != "-") ++uses[in];
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  std::vector<char> remove(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i) {
    PlanNode & e = nodes_[i];
    if (e.op != "ew_binary" || e.i("op") != 0 || e.ins.size() < 2) continue;
    if (e.has("bdims") || e.i("b_scalar") != 0) continue;
    const Tensor & yo = *T_[e.outs[0]];
    for (int k = 0; k < 2; ++k) {
      const std::string & pname = e.ins[k];
      const std::string & rname = e.ins[1 - k];
      auto pit = producer.find(pname);
      if (pit == producer.end()) continue;
      PlanNode & c = nodes_[pit->second];
      if (c.op != "conv1x1" && c.op != "conv3x3") continue;
      if (uses[pname] != 1 || outs.count(pname) || c.outs[0] != pname) continue;
      const Tensor & pt = *T_[pname];
      const Tensor & rt = *T_[rname];
      if (rt.kind == Tensor::kInit || pt.numel != yo.numel || rt.numel != yo.numel) continue;
      if (pt.dims != yo.dims || rt.dims != yo.dims) continue;
      auto rit = producer.find(rname);
      if (rt.kind != Tensor::kInput && (rit == producer.end() || rit->second >= pit->second)) continue;
      if (c.ins.size() > 3 && c.ins[3] != "-") continue;
      if (c.ins.size() < 4) c.ins.resize(4, "-");
      c.ins[3] = rname;
      c.outs[0] = e.outs[0];
      const int cidx = pit->second;  // (pit dies with the erase)
      producer.erase(pname);
      producer[e.outs[0]] = cidx;
      remove[i] = 1;
      break;
    }
  }
  std::vector<PlanNode> kept;
  for (size_t i = 0; i < nodes_.size(); ++i)
    if (!remove[i]) kept.push_back(std::move(nodes_[i]));
  nodes_ = std::move(kept);
}

// Attention core -> one fused node.  After fusePermuteMatmul, ultralytics' Attention reads
// in one of two export forms:
//   S = bmm(q, k; ta)  [h][kd][N]^T x [h][kd][N] -> [h][N][N]
//   T = ew_binary mul (S, scalar init)
// or (ultralytics 8.4 exports, the reference's plans: the scale on q^T before the product)
//   q' = permute_0213 mode 1 (q)        [h][kd][N] -> [h][N][kd]
//   q" = ew_binary mul (q', scalar init)
//   T = bmm(q", k)
// then in both
//   P = softmax_axis (T) over the last axis
//   O = bmm(v, P; tb)  [h][hd][N] x [h][N][N]^T -> [h][hd][N]
// each intermediate with that single reader; the nodes become node "attention" (q, k, v ->
// O) with the scale's fp16 bits and where it applies (scale_q), run by attn_kernel
// (attention.hip), which keeps every node's fp16 rounding.  kd 32, hd 64, N a multiple of 8
// up to the kernel's limit; anything else stays node by node (as does everything with
// IVH_FLAG_NO_FUSE_ATTN).
void Model::fuseAttention()
{
  if (flags_ & (IVH_FLAG_NO_FUSE | IVH_FLAG_NO_FUSE_ATTN)) return;
  std::map<std::string, int> producer, uses;
  std::map<std::string, std::vector<int>> readers;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & o : nodes_[i].outs) producer[o] = (int)i;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & in : nodes_[i].ins)
      if (in != "-") {
        ++uses[in];
        readers[in].push_back((int)i);
      }
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  auto sole_reader = [&](const std::string & t) -> int {
    if (uses[t] != 1 || outs.count(t) || readers[t].size() != 1) return -1;
    return readers[t][0];
  };
  auto dims3 = [&](const std::string & t, int64_t & a, int64_t & b, int64_t & c) {
    const auto & d = T_.at(t)->dims;
    if (d.size() < 2) return false;
    b = d[d.size() - 2];
    c = d.back();
    a = T_.at(t)->numel / std::max<int64_t>(b * c, 1);
    return a * b * c == T_.at(t)->numel;
  };
  std::vector<char> remove(nodes_.size(), 0);
  std::map<int, PlanNode> replace;
  // a scalar multiply by a one-value init; the other operand's name in `x`
  auto scalar_mul = [&](const PlanNode & e, const std::string & x, std::string & sc) {
    if (e.op != "ew_binary" || e.i("op") != 2 || e.ins.size() < 2 || (e.ins[0] != x && e.ins[1] != x)) return false;
    sc = e.ins[0] == x ? e.ins[1] : e.ins[0];
    return T_.count(sc) && T_.at(sc)->kind == Tensor::kInit && T_.at(sc)->numel == 1;
  };
  for (size_t i = 0; i < nodes_.size(); ++i) {
    const PlanNode & m1 = nodes_[i];
    if (m1.op != "bmm" || m1.ins.size() < 2 || m1.i("tb") == 1 || remove[i]) continue;
    std::string sc, q;
    int is = -1, scale_q = 0;
    std::vector<int> extra;  // the scale (and permute) nodes folded in
    if (m1.i("ta") == 1) {   // S = q^T k, then T = S * scale
      const int ie = sole_reader(m1.outs[0]);
      if (ie < 0 || !scalar_mul(nodes_[ie], m1.outs[0], sc)) continue;
      is = sole_reader(nodes_[ie].outs[0]);
      q = m1.ins[0];
      extra = {ie};
    } else {                 // T = (q^T * scale) k
      auto pe = producer.find(m1.ins[0]);
      if (pe == producer.end() || sole_reader(m1.ins[0]) != (int)i) continue;
      const PlanNode & e = nodes_[pe->second];
      if (e.ins.size() < 2) continue;
      const std::string qt = T_.at(e.ins[0])->kind == Tensor::kInit ? e.ins[1] : e.ins[0];
      if (!scalar_mul(e, qt, sc)) continue;
      auto pp = producer.find(qt);
      if (pp == producer.end() || sole_reader(qt) != pe->second) continue;
      const PlanNode & pm = nodes_[pp->second];
      if (pm.op != "permute_0213" || pm.i("mode") != 1 || pm.ins.empty()) continue;
      const auto & qd = T_.at(pm.ins[0])->dims;
      const auto & td = T_.at(qt)->dims;
      if (qd.size() < 2 || td.size() != qd.size() || qd.back() != td[td.size() - 2] || td.back() != qd[qd.size() - 2])
        continue;
      q = pm.ins[0];
      is = sole_reader(m1.outs[0]);
      scale_q = 1;
      extra = {pe->second, pp->second};
    }
    if (is < 0) continue;
    const PlanNode & sm = nodes_[is];
    if (sm.op != "softmax_axis" || sm.i("inner", 1) != 1) continue;
    const int i2 = sole_reader(sm.outs[0]);
    if (i2 < 0) continue;
    const PlanNode & m2 = nodes_[i2];
    if (m2.op != "bmm" || m2.ins.size() < 2 || m2.i("tb") != 1 || m2.i("ta") == 1 || m2.ins[1] != sm.outs[0]) continue;
    int64_t hq, kd, n, hk, kd2, nk, hv, hd, nv, ho, hd2, no, hs, ns1, ns2;
    if (!dims3(q, hq, kd, n) || !dims3(m1.ins[1], hk, kd2, nk) || !dims3(m2.ins[0], hv, hd, nv) ||
        !dims3(m2.outs[0], ho, hd2, no) || !dims3(sm.outs[0], hs, ns1, ns2))
      continue;
    if (kd != kAttnKD || kd2 != kd || hd != kAttnHD || hd2 != hd || nk != n || nv != n || no != n || ns1 != n ||
        ns2 != n || hk != hq || hv != hq || ho != hq || hs != hq || sm.i("axdim") != n || n % 8 || n > kAttnMaxN ||
        attn_key_blocks((int)n) == 0)
      continue;
    // the scale: the init's one fp16 value
    uint16_t bits = 0;
    {
      std::ifstream f(T_.at(sc)->file, std::ios::binary);
      if (!f || !f.read(reinterpret_cast<char *>(&bits), 2)) continue;
    }
    PlanNode fz;
    fz.op = "attention";
    fz.ins = {q, m1.ins[1], m2.ins[0]};
    fz.outs = {m2.outs[0]};
    fz.attr["heads"] = std::to_string(hq);
    fz.attr["n"] = std::to_string(n);
    fz.attr["scale_bits"] = std::to_string(bits);
    fz.attr["scale_q"] = std::to_string(scale_q);
    remove[i] = remove[is] = 1;
    for (int x : extra) remove[x] = 1;
    replace[i2] = fz;
  }
  std::vector<PlanNode> kept;
  for (size_t i = 0; i < nodes_.size(); ++i) {
    if (remove[i]) continue;
    auto it = replace.find((int)i);
    kept.push_back(it != replace.end() ? std::move(it->second) : std::move(nodes_[i]));
  }
  nodes_ = std::move(kept);
}

// conv3x3 / conv_general without act + sole ew_unary consumer -> folded activation.
// (onnx2plan.py:135-147 can fold only HardSwish into conv3x3; ReLU/HardSigmoid/Sigmoid
// after a 3x3 stay separate in the plan.)  Numerically the reference rounds the conv
// output to fp16 before the activation; folding drops that intermediate rounding.
void Model::fuseActivation()
{
  std::map<std::string, int> producer, uses;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & o : nodes_[i].outs) producer[o] = (int)i;
  for (const auto & n : nodes_)
    for (const auto & in : n.ins)
      if (in != "-") ++uses[in];
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  std::vector<char> remove(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i) {
    PlanNode & u = nodes_[i];
    if (u.op != "ew_unary" || u.ins.empty()) continue;
    auto pit = producer.find(u.ins[0]);
    if (pit == producer.end()) continue;
    PlanNode & c = nodes_[pit->second];
    const bool conv = c.op == "conv3x3" || c.op == "conv_general" || c.op == "conv1x1";
    if (!conv || c.i("act") != 0 || uses[u.ins[0]] != 1 || outs.count(u.ins[0])) continue;
    if (c.ins.size() > 3 && c.ins[3] != "-") continue;  // residual would be added before act
    if (T_[u.ins[0]]->numel != T_[u.outs[0]]->numel) continue;
    c.attr["act"] = std::to_string(unary_to_act(u.i("op")));
    c.outs[0] = u.outs[0];
    producer[u.outs[0]] = pit->second;
    remove[i] = 1;
  }
  std::vector<PlanNode> kept;
  for (size_t i = 0; i < nodes_.size(); ++i)
    if (!remove[i]) kept.push_back(std::move(nodes_[i]));
  nodes_ = std::move(kept);
}

// permute_0213 swapping the last two dimensions (mode 1) whose only consumer is a bmm operand
// -> the bmm reads the permute's input as a transposed operand (attr ta / tb), and the
// permute launches nothing.  The C2PSA attention's q^T and attn^T (YOLO11n) are such pairs.
void Model::fusePermuteMatmul()
{
  if (flags_ & IVH_FLAG_NO_FUSE) return;
  std::map<std::string, int> producer, uses;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & o : nodes_[i].outs) producer[o] = (int)i;
  for (const auto & n : nodes_)
    for (const auto & in : n.ins)
      if (in != "-") ++uses[in];
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  std::vector<char> remove(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i) {
    PlanNode & m = nodes_[i];
    if (m.op != "bmm" || m.ins.size() < 2) continue;
    for (int j = 0; j < 2; ++j) {
      auto pit = producer.find(m.ins[j]);
      if (pit == producer.end() || remove[pit->second]) continue;
      const PlanNode & pn = nodes_[pit->second];
      if (pn.op != "permute_0213" || pn.i("mode") != 1 || uses[m.ins[j]] != 1 || outs.count(m.ins[j])) continue;
      const Tensor & src = *T_[pn.ins.at(0)];
      const Tensor & dst = *T_[m.ins[j]];
      // [.., D2, I] -> [.., I, D2]: the source's last two dims are the operand's, swapped
      if (src.dims.size() < 2 || dst.dims.size() != src.dims.size() || src.numel != dst.numel ||
          src.dims.back() != dst.dims[dst.dims.size() - 2] || dst.dims.back() != src.dims[src.dims.size() - 2])
        continue;
      m.ins[j] = pn.ins[0];
      m.attr[j == 0 ? "ta" : "tb"] = "1";
      remove[pit->second] = 1;
    }
  }
  std::vector<PlanNode> kept;
  for (size_t i = 0; i < nodes_.size(); ++i)
    if (!remove[i]) kept.push_back(std::move(nodes_[i]));
  nodes_ = std::move(kept);
}

// ============================================================= decode-tail fusion

// The export form of a Detect / Pose head's decode (ultralytics head.py Detect decode,
// Pose.kpts_decode) as a plan holds it, in either of two export forms:
//   ultralytics 8.4 (the reference's plans): box distributions per scale [4R, H, W] and class
//   scores per scale [nc, H, W], each reshaped and concatenated over the anchors on its own;
//   older exports: box + classes per scale [4R + nc, H, W] -> one concat over the anchors ->
//   copy_c box rows / class rows;
// then box rows -> reshape [4, R, A] -> permute_0213 -> softmax over the R bins -> conv1x1
//   with the bin weights (DFL) -> lt / rb (slice_axis, or copy_c in older exports) ->
//   anchors - lt, anchors + rb -> centre = sum / 2 (or * 0.5), size = x2y2 - x1y1 -> concat
//   -> * strides;  class rows -> sigmoid;
//   keypoints per scale [3 nk, H, W] -> concat over anchors -> slice xy -> * 2 + (anchors -
//   0.5) -> * strides; slice visibility -> sigmoid -> concat [nk, 3, A];
//   output = concat [box (4), classes (nc), keypoints (3 nk)] over A anchors (one three-way
//   concat, or two nested concats in older exports).
// About 35 nodes, each streaming the anchors through memory, become one "pose_decode" node
// whose kernel reads each head pixel once and writes the output once, rounding to fp16
// after every step where a node would have stored its result.  The match runs from each
// graph output backwards and checks every node's op, attributes, operand order and
// broadcast index map; a tail of any other shape is left node by node.
void Model::fuseDecode()
{
  if (flags_ & (IVH_FLAG_NO_FUSE | IVH_FLAG_NO_FUSE_DECODE)) return;
  std::map<std::string, int> producer;
  std::map<std::string, std::vector<int>> users;
  for (size_t i = 0; i < nodes_.size(); ++i) {
    for (const auto & o : nodes_[i].outs)
      if (o != "-") producer[o] = (int)i;
    for (const auto & in : nodes_[i].ins)
      if (in != "-") users[in].push_back((int)i);
  }
  const std::set<std::string> gouts(outputs_.begin(), outputs_.end());

  struct Match {
    std::set<int> region;
    std::vector<std::string> X, C, K;  // per-scale head tensors (C: separate class scores)
    std::vector<int> hw;               // pixels per scale
    std::string wd, anc, st, ancm, cbox, ckpt;
    int R = 0, nc = 0, nk = 0, box_div = 1;
  };
  for (const std::string & out : outputs_) {
    Match m;
    long A = 0;
    const auto id = [](long i) { return i; };
    const auto zero = [](long) { return 0L; };
    auto peek = [&](const std::string & t) -> const PlanNode * {
      auto it = producer.find(t);
      return it == producer.end() ? nullptr : &nodes_[it->second];
    };
    // producer of t if it is a single-output `op` node (added to the region)
    auto take = [&](const std::string & t, const char * op) -> const PlanNode * {
      auto it = producer.find(t);
      if (it == producer.end()) return nullptr;
      const PlanNode & n = nodes_[it->second];
      if (n.op != op || n.outs.size() != 1 || n.ins.empty()) return nullptr;
      m.region.insert(it->second);
      return &n;
    };
    auto unreshape = [&](std::string t) {
      for (;;) {
        auto it = producer.find(t);
        if (it == producer.end()) return t;
        const PlanNode & n = nodes_[it->second];
        if ((n.op != "reshape" && n.op != "flatten") || n.ins.empty()) return t;
        m.region.insert(it->second);
        t = n.ins[0];
      }
    };
    auto init_n = [&](const std::string & t, long n) {
      auto it = T_.find(t);
      return it != T_.end() && it->second->kind == Tensor::kInit && it->second->numel == n;
    };
    auto act_n = [&](const std::string & t, long n) {
      auto it = T_.find(t);
      return it != T_.end() && it->second->kind == Tensor::kAct && it->second->numel == n;
    };
    // an ew_binary `op` over n outputs whose operand indices are fa(i) and fb(i), by the
    // ops.cl rules (b_scalar reads b[0]; bdims = out dims, a strides, b strides)
    auto ew = [&](const PlanNode * e, int op, long n, const std::function<long(long)> & fa,
                  const std::function<long(long)> & fb) -> bool {
      if (!e || e->op != "ew_binary" || e->i("op") != op || e->ins.size() < 2 || !act_n(e->outs[0], n)) return false;
      const bool scalar = e->i("b_scalar") == 1;
      std::vector<long> d;
      if (e->has("bdims") && !scalar)
        for (const auto & v : split_csv(e->str("bdims"))) d.push_back(std::stol(v));
      if (d.size() % 3) return false;
      const int rank = (int)d.size() / 3;
      long tot = 1;
      for (int r = 0; r < rank; ++r) tot *= d[r];
      if (rank && tot != n) return false;
      const long na = T_.at(e->ins[0])->numel, nb = T_.at(e->ins[1])->numel;
      for (long i = 0; i < n; ++i) {
        long ai = i, bi = scalar ? 0 : i;
        if (rank) {
          long rem = i;
          ai = bi = 0;
          for (int r = rank - 1; r >= 0; --r) {
            const long c = rem % d[r];
            rem /= d[r];
            ai += c * d[rank + r];
            bi += c * d[2 * rank + r];
          }
        }
        if (ai != fa(i) || bi != fb(i) || ai >= na || bi >= nb) return false;
      }
      return true;
    };
    auto sigmoid_of = [&](const std::string & t) -> const PlanNode * {
      const PlanNode * u = take(t, "ew_unary");
      return (u && unary_to_act(u->i("op")) == kActSigmoid) ? u : nullptr;
    };
    auto concat2 = [&](const PlanNode * c, int outer, long inner, int ca, int cb) {
      return c && c->ins.size() >= 2 && c->i("outer", 1) == outer && c->i("inner", 1) == inner && c->i("ca") == ca &&
             c->i("cb") == cb && c->i("cc") == 0 && c->i("cd") == 0;
    };
    auto copy_rows = [&](const PlanNode * c, int c0, int cnt) {
      return c && c->i("HW", 1) == A && c->i("c0") == c0 && c->i("cnt") == cnt && c->i("dst_off") == 0;
    };
    // concat over anchors of per-scale [C, H_s, W_s] head tensors (through their reshapes)
    auto scales = [&](const std::string & t, int C, std::vector<std::string> & xs) -> bool {
      const PlanNode * c = take(t, "concat4");
      if (!c || c->i("outer", 1) != C || c->i("inner", 1) != 1 || c->ins.size() < 4) return false;
      const int cnt[4] = {c->i("ca"), c->i("cb"), c->i("cc"), c->i("cd")};
      std::vector<int> hw;
      long tot = 0;
      for (int j = 0; j < 4; ++j) {
        if (cnt[j] <= 0) {
          if (cnt[j] < 0 || (j + 1 < 4 && cnt[j + 1] > 0)) return false;
          continue;
        }
        const std::string s = unreshape(c->ins[j]);
        const Tensor & st = *T_.at(s);
        if (st.kind != Tensor::kAct || st.dims.size() != 4 || st.C != C || (long)st.H * st.W != cnt[j]) return false;
        xs.push_back(s);
        hw.push_back(cnt[j]);
        tot += cnt[j];
      }
      if (tot != A || xs.empty()) return false;
      if (m.hw.empty()) m.hw = hw;
      return m.hw == hw;
    };
    // lt (c0 = 0) / rb (c0 = 2) rows of the [4, A] DFL distances: a Slice over axis 1
    // (slice_axis) or, in older exports, a channel copy
    auto dist_rows = [&](const std::string & t, int c0) -> const PlanNode * {
      const PlanNode * n = peek(t);
      if (n && n->op == "slice_axis") {
        n = take(t, "slice_axis");
        const bool ok = n && n->i("outer", 1) == 1 && n->i("axdim") == 4 && n->i("inner", 1) == A &&
                        n->i("start") == c0 && n->i("len") == 2;
        return ok ? n : nullptr;
      }
      n = take(t, "copy_c");
      return copy_rows(n, c0, 2) ? n : nullptr;
    };
    // [dbox * strides (4), sigmoid(classes) (nc)]: the first two inputs of the output concat
    auto box = [&](const std::string & dbox_t, const std::string & cls_t) -> bool {
      const PlanNode * bx = take(dbox_t, "ew_binary");
      if (!bx || !init_n(bx->ins.at(1), A) || !ew(bx, 2, 4 * A, id, [A](long i) { return i % A; })) return false;
      m.st = bx->ins[1];
      const PlanNode * db = take(bx->ins[0], "concat4");
      if (!concat2(db, 1, A, 2, 2)) return false;
      const PlanNode * cxy = take(db->ins[0], "ew_binary");
      if (!cxy || cxy->ins.size() < 2 || !init_n(cxy->ins[1], 1)) return false;
      m.box_div = cxy->i("op") == 3;
      if (!ew(cxy, m.box_div ? 3 : 2, 2 * A, id, zero)) return false;
      m.cbox = cxy->ins[1];
      const PlanNode * sum = take(cxy->ins[0], "ew_binary");
      const PlanNode * wh = take(db->ins[1], "ew_binary");
      if (!ew(sum, 0, 2 * A, id, id) || !ew(wh, 1, 2 * A, id, id)) return false;
      const std::string x2y2 = wh->ins[0], x1y1 = wh->ins[1];
      if (!((sum->ins[0] == x1y1 && sum->ins[1] == x2y2) || (sum->ins[0] == x2y2 && sum->ins[1] == x1y1))) return false;
      const PlanNode * n1 = take(x1y1, "ew_binary");  // anchors - lt
      const PlanNode * n2 = take(x2y2, "ew_binary");  // anchors + rb (either order)
      if (!ew(n1, 1, 2 * A, id, id) || !ew(n2, 0, 2 * A, id, id) || !init_n(n1->ins[0], 2 * A)) return false;
      m.anc = n1->ins[0];
      const std::string rbt = n2->ins[0] == m.anc ? n2->ins[1] : (n2->ins[1] == m.anc ? n2->ins[0] : std::string());
      if (rbt.empty() || rbt == m.anc) return false;
      const PlanNode * lt = dist_rows(n1->ins[1], 0);
      const PlanNode * rb = dist_rows(rbt, 2);
      if (!lt || !rb || lt->ins[0] != rb->ins[0] || !act_n(lt->ins[0], 4 * A)) return false;
      const PlanNode * cv = take(unreshape(lt->ins[0]), "conv1x1");
      if (!cv || cv->ins.size() < 2 || cv->i("act") != 0) return false;
      if ((cv->ins.size() > 2 && cv->ins[2] != "-") || (cv->ins.size() > 3 && cv->ins[3] != "-")) return false;
      const Tensor & wt = *T_.at(cv->ins[0]);
      if (wt.kind != Tensor::kInit || wt.dims.empty() || wt.dims[0] != 1 || wt.numel < 1 || wt.numel > 64) return false;
      m.R = (int)wt.numel;
      m.wd = cv->ins[0];
      if (!act_n(cv->outs[0], 4 * A) || !act_n(cv->ins[1], 4 * A * m.R)) return false;
      const PlanNode * sm = take(cv->ins[1], "softmax_axis");
      if (!sm || sm->i("outer", 1) != 1 || sm->i("axdim") != m.R || sm->i("inner", 1) != 4 * A) return false;
      const PlanNode * pm = take(sm->ins[0], "permute_0213");
      if (!pm || pm->i("mode") != 0 || pm->i("D1", 1) != 4 || pm->i("D2", 1) != m.R || pm->i("I", 1) != A) return false;
      const PlanNode * sg = sigmoid_of(cls_t);
      if (!sg || !act_n(cls_t, (long)m.nc * A) || !act_n(sg->ins[0], (long)m.nc * A)) return false;
      const std::string bsrc = unreshape(pm->ins[0]);
      const PlanNode * bp = peek(bsrc);
      if (bp && bp->op == "concat4") {  // separate box and class concats over the anchors
        const PlanNode * cp = peek(sg->ins[0]);
        return cp && cp->op == "concat4" && scales(bsrc, 4 * m.R, m.X) && scales(sg->ins[0], m.nc, m.C);
      }
      const PlanNode * bsl = take(bsrc, "copy_c");  // one [4R + nc, A] concat, rows copied out
      if (!copy_rows(bsl, 0, 4 * m.R)) return false;
      const PlanNode * csl = take(sg->ins[0], "copy_c");
      if (!copy_rows(csl, 4 * m.R, m.nc) || csl->ins[0] != bsl->ins[0]) return false;
      return scales(bsl->ins[0], 4 * m.R + m.nc, m.X);
    };
    // [nk, 3, A] = concat [(xy * 2 + (anchors - 0.5)) * strides, sigmoid(visibility)]
    auto keypoints = [&](const std::string & t) -> bool {
      const PlanNode * kc = take(unreshape(t), "concat4");
      if (!kc) return false;
      m.nk = kc->i("outer", 1);
      if (m.nk < 1 || !concat2(kc, m.nk, A, 2, 1)) return false;
      const long nxy = 2L * m.nk * A;
      const PlanNode * k3 = take(kc->ins[0], "ew_binary");
      if (!k3 || k3->ins.size() < 2 || k3->ins[1] != m.st || !ew(k3, 2, nxy, id, [A](long i) { return i % A; }))
        return false;
      const PlanNode * k2 = take(k3->ins[0], "ew_binary");
      if (!k2 || k2->ins.size() < 2 || !init_n(k2->ins[1], 2 * A) || !ew(k2, 0, nxy, id, [A](long i) { return i % (2 * A); }))
        return false;
      m.ancm = k2->ins[1];
      const PlanNode * k1 = take(k2->ins[0], "ew_binary");
      if (!k1 || k1->ins.size() < 2 || !init_n(k1->ins[1], 1) || !ew(k1, 2, nxy, id, zero)) return false;
      m.ckpt = k1->ins[1];
      const PlanNode * sxy = take(k1->ins[0], "slice_axis");
      const PlanNode * vs = sigmoid_of(kc->ins[1]);
      const PlanNode * sv = vs ? take(vs->ins[0], "slice_axis") : nullptr;
      auto sl = [&](const PlanNode * s, int s0, int len) {
        return s && s->i("outer", 1) == m.nk && s->i("axdim") == 3 && s->i("inner", 1) == A && s->i("start") == s0 &&
               s->i("len") == len;
      };
      if (!sl(sxy, 0, 2) || !sl(sv, 2, 1) || sv->ins[0] != sxy->ins[0]) return false;
      if (!act_n(kc->ins[1], (long)m.nk * A) || !act_n(vs->ins[0], (long)m.nk * A) || !act_n(sxy->outs[0], nxy)) return false;
      return scales(unreshape(sxy->ins[0]), 3 * m.nk, m.K);
    };

    bool ok = false;
    try {
      const PlanNode * fin = take(out, "concat4");
      if (fin && fin->i("outer", 1) == 1 && fin->ins.size() >= 2) {
        A = fin->i("inner", 1);
        const PlanNode * first = peek(fin->ins[0]);
        if (A > 0 && first && first->op == "concat4" && first->i("ca") == 4 && first->i("cb") >= 1) {
          // pose, two nested concats: [[box, classes], keypoints]
          const PlanNode * bc = take(fin->ins[0], "concat4");
          m.nc = bc->i("cb");
          ok = concat2(bc, 1, A, 4, m.nc) && box(bc->ins[0], bc->ins[1]) && keypoints(fin->ins[1]) &&
               concat2(fin, 1, A, 4 + m.nc, 3 * m.nk) && act_n(fin->ins[1], 3L * m.nk * A);
        } else if (A > 0 && fin->ins.size() >= 3 && fin->i("cc") > 0) {
          // pose, one concat: [box, classes, keypoints]
          m.nc = fin->i("cb");
          ok = fin->i("ca") == 4 && m.nc >= 1 && fin->i("cd") == 0 && box(fin->ins[0], fin->ins[1]) &&
               keypoints(fin->ins[2]) && fin->i("cc") == 3 * m.nk && act_n(fin->ins[2], 3L * m.nk * A);
        } else if (A > 0) {  // detect: box + classes only
          m.nc = fin->i("cb");
          ok = concat2(fin, 1, A, 4, m.nc) && m.nc >= 1 && box(fin->ins[0], fin->ins[1]);
        }
      }
    } catch (const std::exception &) {
      ok = false;
    }
    if (!ok || m.X.size() > 4 || m.X.empty() || (m.nk && m.K.size() != m.X.size()) ||
        (!m.C.empty() && m.C.size() != m.X.size()))
      continue;
    // nothing outside the region may read what the region computes
    for (int ni : m.region)
      for (const auto & o : nodes_[ni].outs) {
        if (o == out || o == "-") continue;
        if (gouts.count(o)) ok = false;
        for (int u : users[o])
          if (!m.region.count(u)) ok = false;
      }
    if (!ok) continue;

    PlanNode f;
    f.op = "pose_decode";
    f.ins = m.X;
    f.ins.insert(f.ins.end(), m.C.begin(), m.C.end());
    if (m.nk) f.ins.insert(f.ins.end(), m.K.begin(), m.K.end());
    for (const std::string & s : {m.wd, m.anc, m.st, m.nk ? m.ancm : std::string("-"), m.cbox,
                                  m.nk ? m.ckpt : std::string("-")})
      f.ins.push_back(s);
    f.outs = {out};
    f.attr["S"] = std::to_string(m.X.size());
    f.attr["R"] = std::to_string(m.R);
    f.attr["nc"] = std::to_string(m.nc);
    f.attr["nk"] = std::to_string(m.nk);
    f.attr["A"] = std::to_string(A);
    f.attr["box_div"] = std::to_string(m.box_div);
    f.attr["split"] = m.C.empty() ? "0" : "1";
    for (size_t s = 0; s < m.hw.size(); ++s) f.attr["hw" + std::to_string(s)] = std::to_string(m.hw[s]);
    const int last = *m.region.rbegin();
    std::vector<PlanNode> kept;
    for (size_t i = 0; i < nodes_.size(); ++i) {
      if ((int)i == last) kept.push_back(f);
      else if (!m.region.count((int)i)) kept.push_back(std::move(nodes_[i]));
    }
    nodes_ = std::move(kept);
    producer.clear();
    users.clear();
    for (size_t i = 0; i < nodes_.size(); ++i) {
      for (const auto & o : nodes_[i].outs)
        if (o != "-") producer[o] = (int)i;
      for (const auto & in : nodes_[i].ins)
        if (in != "-") users[in].push_back((int)i);
    }
  }
}

// ====================================================================== planning

// ew_binary whose smaller operand is one value per output channel ([.., C, 1, 1]), the
// reference's ew_binary_ch pattern (src/PlanModel.cpp:2603-2623).  Returns 1 if that
// operand is `a`, 0 if it is `b`, -1 if the node is not such a broadcast.
int Model::chanBroadcast(const PlanNode & n) const
{
  if (n.op != "ew_binary" || !n.has("bdims") || n.i("b_scalar") == 1 || n.ins.size() < 2) return -1;
  const Tensor & at = *T_.at(n.ins[0]);
  const Tensor & bt = *T_.at(n.ins[1]);
  const Tensor & yt = *T_.at(n.outs[0]);
  const Tensor * s = nullptr;
  int a_is = 0;
  if (at.numel != yt.numel && bt.numel == yt.numel) { s = &at; a_is = 1; }
  else if (bt.numel != yt.numel && at.numel == yt.numel) s = &bt;
  if (!s || s->numel != yt.C || yt.dims.size() < 3) return -1;
  int nonunit = 0, pos = -1;
  for (size_t i = 0; i < s->dims.size(); ++i)
    if (s->dims[i] != 1) { ++nonunit; pos = (int)i; }
  const int chidx = (int)s->dims.size() - 3;
  if (nonunit == 1 && pos == chidx && s->dims.size() == yt.dims.size()) return a_is;
  if (nonunit == 0 && yt.C == 1) return a_is;
  return -1;
}

void Model::plan()
{
  for (auto & kv : T_) { kv.second->users.clear(); kv.second->producer = -1; }
  for (size_t i = 0; i < nodes_.size(); ++i) {
    for (const auto & in : nodes_[i].ins)
      if (in != "-") T_[in]->users.push_back((int)i);
    for (const auto & o : nodes_[i].outs)
      if (o != "-") T_[o]->producer = (int)i;
  }
  skip_.assign(nodes_.size(), 0);
  assignViews();
  chooseLayouts();
  fuseUpsample();
}

// Upsample-concat fusion (YOLO necks: nn.Upsample(2) -> Concat -> the C2f / C3k2 cv1 1x1):
// when a 1x1 conv is the only reader of a zero-copy concat whose leading channels are the
// output of a 2x nearest resize read by nothing else, the conv's implicit GEMM reads those
// channels from the resize's input at (oy / 2, ox / 2) and the resize is not run, so the
// upsampled tensor (4x its input) is neither written nor read back.  The other concat inputs
// stay in the concat root, which the conv reads as before.
void Model::fuseUpsample()
{
  up_src_.assign(nodes_.size(), -1);
  if (flags_ & (IVH_FLAG_NO_FUSE | IVH_FLAG_NO_REUSE | IVH_FLAG_NO_FUSE_UPSAMPLE | IVH_FLAG_DIRECT_ONLY)) return;
  for (size_t k = 0; k < nodes_.size(); ++k) {
    const PlanNode & n = nodes_[k];
    if (n.op != "conv1x1" || n.ins.size() < 2 || n.ins[1] == "-") continue;
    const Tensor & xt = *T_[n.ins[1]];
    if (xt.kind != Tensor::kAct || xt.root < 0 || xt.producer < 0 || xt.users.size() != 1) continue;
    const Root & Q = *roots_[xt.root];
    if (Q.layout != kNHWC || xt.coff != 0 || xt.C != Q.C || xt.dims.size() != 4 || Q.H % 2 || Q.W % 2) continue;
    const int c = xt.producer;
    const PlanNode & cn = nodes_[c];
    if (cn.op != "concat4" || !skip_[c] || cn.ins.empty() || cn.ins[0] == "-") continue;
    const Tensor & ut = *T_[cn.ins[0]];
    const int cu = cn.i("ca");
    if (ut.kind != Tensor::kAct || ut.root != xt.root || ut.coff != 0 || ut.C != cu || ut.producer < 0 ||
        ut.users.size() != 1 || ut.users[0] != c)
      continue;
    const int r = ut.producer;
    const PlanNode & rn = nodes_[r];
    if (rn.op != "resize_nn" || skip_[r] || std::max(1, rn.i("S", 2)) != 2 || rn.ins.empty()) continue;
    const Tensor & at = *T_[rn.ins[0]];
    if (at.kind != Tensor::kAct || at.root < 0 || roots_[at.root]->layout != kNHWC || at.C != cu ||
        rn.i("C") != cu || rn.i("H") * 2 != Q.H || rn.i("W") * 2 != Q.W || (long)at.H * at.W != (long)rn.i("H") * rn.i("W") ||
        at.coff % 8 || roots_[at.root]->cs % 8)
      continue;
    // the conv's geometry the implicit GEMM's upsample build needs (upcat_ok at launch)
    const Tensor & wt = *T_[n.ins[0]];
    const int cin = (int)wt.dims[1], cout = (int)wt.dims[0];
    if (cin != Q.C || cin % 8 || cu % igemm_bk(cout, cin) || cu >= cin) continue;
    // nothing else may read the concat root's upsampled channels
    bool alone = true;
    for (const auto & kv : T_) {
      const Tensor & t = *kv.second;
      if (&t != &xt && &t != &ut && t.kind == Tensor::kAct && t.root == xt.root && t.coff < cu) alone = false;
    }
    if (!alone) continue;
    up_src_[k] = r;
    skip_[r] = 1;
  }
}

// Views: every activation tensor gets a root; reshape/flatten alias, copy_c is a channel
// view, channel concat redirects its inputs' roots into the concat root.
void Model::assignViews()
{
  roots_.clear();
  auto new_root = [&](Tensor & t) {
    auto r = std::make_unique<Root>();
    r->C = t.C; r->H = t.H; r->W = t.W; r->numel = t.numel;
    r->flat = t.dims.size() != 4;
    t.root = (int)roots_.size();
    t.coff = 0;
    t.eoff = 0;
    roots_.push_back(std::move(r));
  };
  Tensor & in = *T_[input_name_];
  new_root(in);
  roots_[in.root]->is_input = true;
  // resolve the current final root and offsets of a tensor through redirects
  auto resolve = [&](const Tensor & t, int & coff, long & eoff) {
    int r = t.root;
    coff = t.coff;
    eoff = t.eoff;
    while (roots_[r]->parent >= 0) {
      const Root & rr = *roots_[r];
      const Root & pp = *roots_[rr.parent];
      coff += rr.pcoff;
      eoff += (long)rr.pcoff * pp.H * pp.W;
      r = rr.parent;
    }
    return r;
  };
  const bool no_views = (flags_ & IVH_FLAG_NO_FUSE) != 0;
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    PlanNode & n = nodes_[ni];
    Tensor & out = *T_[n.outs[0]];
    if (!sib_[ni].empty()) {  // merged siblings: their outputs are channel views of one root
      auto r = std::make_unique<Root>();
      r->H = out.H;
      r->W = out.W;
      r->C = 0;
      for (int j : sib_[ni]) r->C += T_[nodes_[j].outs[0]]->C;
      r->numel = (long)r->C * r->H * r->W;
      const int rid = (int)roots_.size();
      roots_.push_back(std::move(r));
      int off = 0;
      bool blocks64 = true;
      for (int j : sib_[ni]) {
        Tensor & t = *T_[nodes_[j].outs[0]];
        t.root = rid;
        t.coff = off;
        t.eoff = (long)off * t.H * t.W;
        off += t.C;
        if (j != sib_[ni].back() && t.C % 64) blocks64 = false;
      }
      // members of whole 64-channel blocks: a 128-byte-aligned pixel pitch, so each member's
      // reader fetches whole 128-byte lines of its own channels (a 184-channel pitch had the
      // 64-channel readers fetch 1.75 lines per pixel: 38 -> 48 us for 64->64 at 80x80)
      if (blocks64) roots_[rid]->cs_align = 64;
    }
    if (n.op == "reshape" || n.op == "flatten") {
      const Tensor & src = *T_[n.ins.at(0)];
      if (src.numel != out.numel) throw std::runtime_error("reshape numel mismatch: " + out.name);
      if (src.kind == Tensor::kInit) { new_root(out); continue; }  // materialised by a copy
      out.root = src.root;
      out.coff = src.coff;
      out.eoff = src.eoff;
      roots_[src.root]->reshaped = true;
      skip_[ni] = 1;
      continue;
    }
    if (n.op == "copy_c" && !no_views && n.i("dst_off") == 0) {
      const Tensor & src = *T_[n.ins.at(0)];
      const int HW = n.i("HW", 1), c0 = n.i("c0"), cnt = n.i("cnt");
      if (src.kind == Tensor::kAct && (long)src.H * src.W == HW && c0 + cnt <= src.C &&
          out.numel == (long)cnt * HW && out.H * out.W == HW) {
        out.root = src.root;
        out.coff = src.coff + c0;
        out.eoff = src.eoff + (long)c0 * HW;
        skip_[ni] = 1;
        continue;
      }
    }
    if (out.root < 0) new_root(out);
    for (size_t k = 1; k < n.outs.size(); ++k)
      if (T_[n.outs[k]]->root < 0) new_root(*T_[n.outs[k]]);
    if (n.op == "concat4" && !no_views && n.i("outer", 1) == 1) {
      const int cnt[4] = {n.i("ca"), n.i("cb"), n.i("cc"), n.i("cd")};
      int off[4], tot = 0;
      for (int j = 0; j < 4; ++j) { off[j] = tot; tot += cnt[j]; }
      const int inner = n.i("inner", 1);
      const Root & Q = *roots_[out.root];
      const bool plain = tot == out.C && (long)Q.H * Q.W == inner;
      for (int j = 0; plain && j < 4; ++j) {
        if (cnt[j] <= 0) continue;
        const Tensor & t = *T_[n.ins.at(j)];
        int tc;
        long te;
        if (t.kind != Tensor::kAct) continue;
        const int r = resolve(t, tc, te);
        Root & R = *roots_[r];
        const int qroot = out.root;
        if (r == qroot) continue;  // already redirected into this concat (same root, earlier input)
        const int base = off[j] - tc;
        bool ok = R.parent < 0 && !R.is_input && !R.is_output && r != qroot &&
                  (long)R.H * R.W == inner && base >= 0 && base + R.C <= tot && t.C == cnt[j];
        for (const auto & o : outputs_)
          if (T_[o]->root == r) ok = false;
        // every concat input overlapping R's channel range must be the matching view of R
        for (int k = 0; ok && k < 4; ++k) {
          if (cnt[k] <= 0) continue;
          const int lo = std::max(off[k], base), hi = std::min(off[k] + cnt[k], base + R.C);
          if (lo >= hi) continue;
          const Tensor & tk = *T_[n.ins.at(k)];
          int kc;
          long ke;
          if (tk.kind != Tensor::kAct || resolve(tk, kc, ke) != r || off[k] - kc != base ||
              off[k] < base || off[k] + cnt[k] > base + R.C)
            ok = false;
        }
        if (!ok) continue;
        R.parent = qroot;
        R.pcoff = base;
      }
      // inputs that now resolve into the concat root at their own offset need no copy
      bool done = true;
      for (int j = 0; j < 4; ++j) {
        if (cnt[j] <= 0) continue;
        const Tensor & t = *T_[n.ins.at(j)];
        int tc;
        long te;
        if (t.kind != Tensor::kAct || resolve(t, tc, te) != out.root || tc != off[j]) done = false;
      }
      if (done && plain) skip_[ni] = 1;
    }
  }
  // every remaining activation without a root (e.g. declared but produced by nothing)
  for (auto & kv : T_)
    if (kv.second->kind == Tensor::kAct && kv.second->root < 0) new_root(*kv.second);
  // collapse redirects: every tensor points at its final root
  for (auto & kv : T_) {
    Tensor & t = *kv.second;
    if (t.root < 0) continue;
    int c;
    long e;
    const int r = resolve(t, c, e);
    t.root = r;
    t.coff = c;
    t.eoff = e;
  }
  for (const auto & o : outputs_) roots_[T_[o]->root]->is_output = true;
  // reshape flags propagate to final roots
  for (size_t i = 0; i < roots_.size(); ++i) {
    if (!roots_[i]->reshaped) continue;
    int r = (int)i;
    while (roots_[r]->parent >= 0) r = roots_[r]->parent;
    roots_[r]->reshaped = true;
  }
}

// NHWC for conv-domain roots whose every reader and writer handles channels-last.
void Model::chooseLayouts()
{
  // which (node, slot) reads accept NHWC
  auto reader_ok = [&](const PlanNode & n, size_t slot, const Tensor & t) -> bool {
    const std::string & op = n.op;
    if (op == "conv3x3") return slot == 0 || slot == 3;
    if (op == "conv1x1") return slot == 1 || slot == 3;
    if (op == "conv_general") return slot == 0;
    if (op == "maxpool" || op == "resize_nn" || op == "gap" || op == "ew_unary") return true;
    if (op == "copy_c") return n.i("dst_off") == 0;
    if (op == "concat4") return n.i("outer", 1) == 1;
    if (op == "ew_binary") {
      const Tensor & y = *T_[n.outs[0]];
      if (!n.has("bdims") || n.i("b_scalar") == 1) return t.numel == y.numel;
      return chanBroadcast(n) >= 0 && t.numel == y.numel;  // big operand of a per-channel broadcast
    }
    return false;
  };
  auto writer_ok = [&](const PlanNode & n) -> bool {
    const std::string & op = n.op;
    if (op == "conv3x3" || op == "conv1x1" || op == "conv_general" || op == "maxpool" ||
        op == "resize_nn" || op == "ew_unary")
      return true;
    if (op == "copy_c") return n.i("dst_off") == 0;
    if (op == "concat4") return n.i("outer", 1) == 1;
    if (op == "ew_binary") return !n.has("bdims") || n.i("b_scalar") == 1 || chanBroadcast(n) >= 0;
    return false;
  };
  std::vector<char> ok(roots_.size(), 1);
  for (size_t i = 0; i < roots_.size(); ++i) {
    const Root & r = *roots_[i];
    if (r.parent >= 0 || r.reshaped || r.is_input || r.is_output || r.flat || (long)r.H * r.W <= 1)
      ok[i] = 0;
  }
  if (flags_ & IVH_FLAG_NCHW_ONLY) std::fill(ok.begin(), ok.end(), 0);
  for (auto & kv : T_) {
    const Tensor & t = *kv.second;
    if (t.kind != Tensor::kAct || t.root < 0) continue;
    if (!ok[t.root]) continue;
    if ((long)t.H * t.W != (long)roots_[t.root]->H * roots_[t.root]->W || t.dims.size() != 4) {
      ok[t.root] = 0;
      continue;
    }
    if (t.producer >= 0 && !writer_ok(nodes_[t.producer])) ok[t.root] = 0;
    for (int u : t.users) {
      const PlanNode & n = nodes_[u];
      for (size_t s = 0; s < n.ins.size(); ++s)
        if (n.ins[s] == t.name && !reader_ok(n, s, t)) ok[t.root] = 0;
    }
  }
  for (size_t i = 0; i < roots_.size(); ++i) {
    Root & r = *roots_[i];
    r.layout = ok[i] ? kNHWC : kNCHW;
    const long HW = (long)r.H * r.W;
    if (r.layout == kNHWC) {
      r.cs = (int)round_up(r.C, r.cs_align);
      r.per_image = round_up(HW * r.cs, 64);
    } else {
      r.cs = (int)HW;
      r.per_image = round_up(std::max<long>(r.numel, 8), 64);
    }
  }
}

// ============================================================ memory + weights

// Device allocation; in a dry run (no GPU) a unique fake address is handed out instead so the
// planner and the launch validator run on any host.  Every allocation is registered so each
// launch's address range can be checked before it is enqueued.
void * Model::devAlloc(size_t bytes, bool zero)
{
  bytes = (size_t)round_up((long)std::max<size_t>(bytes, 256), 256);
  void * d = nullptr;
  if (dry_) {
    d = reinterpret_cast<void *>(fake_next_);
    fake_next_ += round_up((long)bytes + 4096, 4096);
  } else {
    HIPCHECK(hipMalloc(&d, bytes));
    if (zero) HIPCHECK(hipMemset(d, 0, bytes));
  }
  allocs_.push_back({reinterpret_cast<uintptr_t>(d), bytes});
  return d;
}

void Model::devUpload(void * d, const void * src, size_t bytes)
{
  if (!dry_) HIPCHECK(hipMemcpy(d, src, bytes, hipMemcpyHostToDevice));
}

void Model::allocate()
{
  // liveness over final roots
  for (auto & r : roots_) { r->first = INT_MAX; r->last = -1; }
  const int N = (int)nodes_.size();
  for (int ni = 0; ni < N; ++ni) {
    for (const auto & in : nodes_[ni].ins) {
      if (in == "-") continue;
      const Tensor & t = *T_[in];
      if (t.root < 0 || t.kind == Tensor::kInit) continue;
      Root & r = *roots_[t.root];
      r.last = std::max(r.last, ni);
      r.first = std::min(r.first, ni);
    }
    for (const auto & o : nodes_[ni].outs) {
      const Tensor & t = *T_[o];
      if (t.root < 0) continue;
      Root & r = *roots_[t.root];
      r.first = std::min(r.first, ni);
      r.last = std::max(r.last, ni);
    }
  }
  for (const auto & o : outputs_) roots_[T_[o]->root]->last = N + 1;
  // SPPF's three chained pools may run as one launch at node ni (emitNode): it reads x and
  // writes y1, y2 and y3 together, so all four must be live over [ni, ni + 2] and none may
  // take another's bytes.  The chain is a structural property of the plan; whether the
  // launch fuses also depends on alignment, and the wider intervals are harmless if not.
  for (int ni = 0; ni + 2 < N; ++ni) {
    if (!sppfChain((size_t)ni)) continue;
    for (const std::string * t : {&nodes_[ni].ins[0], &nodes_[ni].outs[0], &nodes_[ni + 1].outs[0], &nodes_[ni + 2].outs[0]}) {
      const Tensor & tt = *T_[*t];
      if (tt.root < 0 || tt.kind == Tensor::kInit) continue;
      Root & r = *roots_[tt.root];
      r.first = std::min(r.first, ni);
      r.last = std::max(r.last, ni + 2);
    }
  }
  // A bottleneck pair runs as one launch at its first conv ni: it reads x (the first conv's
  // input, and the second's residual) and writes y (the second conv's output) together, so
  // x stays live to the second conv and y is live from ni.
  for (int ni = 0; ni < N; ++ni) {
    const int nj = pair_next_[ni];
    if (nj < 0) continue;
    const Tensor & xt = *T_[nodes_[ni].ins[0]];
    const Tensor & yt = *T_[nodes_[nj].outs[0]];
    if (xt.root >= 0 && xt.kind != Tensor::kInit) roots_[xt.root]->last = std::max(roots_[xt.root]->last, nj);
    if (yt.root >= 0) roots_[yt.root]->first = std::min(roots_[yt.root]->first, ni);
  }
  // a conv with a fused upsample reads the resize's input at its own node
  for (int ni = 0; ni < N; ++ni) {
    const int r = up_src_[ni];
    if (r < 0) continue;
    const Tensor & at = *T_[nodes_[r].ins[0]];
    roots_[at.root]->last = std::max(roots_[at.root]->last, ni);
  }
  // best-fit placement, largest first, on closed [first, last] intervals
  std::vector<int> order;
  for (size_t i = 0; i < roots_.size(); ++i) {
    const Root & r = *roots_[i];
    if (r.parent >= 0 || r.is_input || r.first == INT_MAX) continue;
    order.push_back((int)i);
  }
  const bool no_reuse = (flags_ & IVH_FLAG_NO_REUSE) != 0;
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    return roots_[a]->per_image != roots_[b]->per_image ? roots_[a]->per_image > roots_[b]->per_image : a < b;
  });
  std::vector<int> placed;
  long total = 0;
  for (int id : order) {
    Root & r = *roots_[id];
    std::vector<std::pair<long, long>> busy;
    for (int pid : placed) {
      const Root & p = *roots_[pid];
      if (no_reuse || !(p.last < r.first || r.last < p.first)) busy.push_back({p.off1, p.off1 + p.per_image});
    }
    std::sort(busy.begin(), busy.end());
    long best = -1, best_gap = LONG_MAX, cur = 0;
    for (auto & iv : busy) {
      if (iv.first - cur >= r.per_image && iv.first - cur < best_gap) { best = cur; best_gap = iv.first - cur; }
      cur = std::max(cur, iv.second);
    }
    if (best < 0) best = cur;
    r.off1 = best;
    total = std::max(total, best + r.per_image);
    placed.push_back(id);
  }
  arena_elems1_ = total;
  verifyArena();
  arena_ = devAlloc((size_t)std::max<long>(total, 64) * max_batch_ * 2, true);
  const Tensor & in = *T_[input_name_];
  const long in_img = roots_[in.root]->per_image;
  input_buf_ = devAlloc((size_t)in_img * max_batch_ * 2, true);
}

// The memory plan's invariant (the reference checks the same for its pool,
// src/PlanModel.cpp:1083-1101): two arena roots whose closed live intervals intersect
// occupy disjoint [off1, off1 + per_image) ranges, and every root lies inside the arena.
void Model::verifyArena() const
{
  std::vector<int> placed;
  for (size_t i = 0; i < roots_.size(); ++i) {
    const Root & r = *roots_[i];
    if (r.parent >= 0 || r.is_input || r.first == INT_MAX) continue;
    if (r.off1 < 0 || r.off1 + r.per_image > arena_elems1_)
      throw std::runtime_error("activation arena: root " + std::to_string(i) + " outside the arena");
    placed.push_back((int)i);
  }
  for (size_t a = 0; a < placed.size(); ++a)
    for (size_t b = a + 1; b < placed.size(); ++b) {
      const Root & p = *roots_[placed[a]];
      const Root & q = *roots_[placed[b]];
      const bool live = !(p.last < q.first || q.last < p.first);
      const bool share = p.off1 < q.off1 + q.per_image && q.off1 < p.off1 + p.per_image;
      if (live && share && p.per_image > 0 && q.per_image > 0)
        throw std::runtime_error("activation arena: roots " + std::to_string(placed[a]) + " and " +
                                 std::to_string(placed[b]) + " are live together and share memory");
    }
}

void Model::uploadWeights()
{
  // raw fp16 inits (used by small ops and as operand views)
  std::map<std::string, std::vector<uint16_t>> host;
  for (auto & kv : T_) {
    Tensor & t = *kv.second;
    if (t.kind != Tensor::kInit) continue;
    std::vector<uint16_t> buf((size_t)t.numel);
    std::ifstream f(t.file, std::ios::binary);
    if (!f) throw std::runtime_error("PlanModel: cannot open init " + t.file);
    f.read(reinterpret_cast<char *>(buf.data()), (std::streamsize)(buf.size() * 2));
    if ((size_t)f.gcount() != buf.size() * 2)
      throw std::runtime_error("PlanModel: init file too short: " + t.file);
    const size_t bytes = round_up((long)buf.size() * 2 + 16, 256);
    void * d = devAlloc(bytes, true);
    devUpload(d, buf.data(), buf.size() * 2);
    dev_allocs_.push_back(d);
    weight_bytes_ += bytes;
    init_dev_[t.name] = d;
    host[t.name] = std::move(buf);
  }
  packed_.assign(nodes_.size(), Packed{});
  auto upload = [&](const void * src, size_t bytes) -> void * {
    void * d = devAlloc(bytes, false);
    devUpload(d, src, bytes);
    dev_allocs_.push_back(d);
    weight_bytes_ += round_up((long)bytes, 256);
    return d;
  };
  // one conv's packing; merged: the members of its sibling group together
  auto pack_conv = [&](size_t ni, bool merged) -> Packed {
    const PlanNode & n = nodes_[ni];
    const bool is1 = n.op == "conv1x1", is3 = n.op == "conv3x3", isg = n.op == "conv_general";
    const std::string wname = is1 ? n.ins.at(0) : n.ins.at(1);
    const Tensor & wt = *T_[wname];
    if (wt.kind != Tensor::kInit) throw std::runtime_error("conv weight is not an init: " + wname);
    const std::vector<uint16_t> * Wp = &host[wname];
    ConvSpec cs;
    cs.Cout = (int)wt.dims.at(0);
    // merged siblings: the members' weights and biases concatenated over output channels
    // (grouped: each member's input channels zero-padded to 64; the last member's rows padded
    // with zero rows up to the launch's output channels)
    std::vector<uint16_t> Wm, Bm;
    const bool grp = merged && sib_grouped_[ni];
    const int mcin = grp ? 64 : (int)wt.dims.at(1);
    if (merged) {
      cs.Cout = 0;
      for (size_t k = 0; k < sib_[ni].size(); ++k) {
        const PlanNode & m = nodes_[sib_[ni][k]];
        const Tensor & mw = *T_[m.ins.at(1)];
        const std::vector<uint16_t> & hw = host.at(m.ins.at(1));
        const std::vector<uint16_t> & hb = host.at(m.ins.at(2));
        const int co = (int)mw.dims[0], ci = (int)mw.dims[1];
        if (mw.dims.size() != 4 || mw.numel != (long)co * ci * 9 || ci > mcin || (!grp && ci != mcin) ||
            (long)hb.size() < co)
          throw std::runtime_error("merged sibling conv weights: " + m.outs[0]);
        const int rows = k + 1 == sib_[ni].size() ? sib_cout_[ni] - cs.Cout : co;
        if (rows < co) throw std::runtime_error("merged sibling conv rows: " + m.outs[0]);
        for (int r = 0; r < rows; ++r) {
          for (int c = 0; c < mcin; ++c)
            for (int t = 0; t < 9; ++t) Wm.push_back(r < co && c < ci ? hw[((size_t)r * ci + c) * 9 + t] : 0);
          Bm.push_back(r < co ? hb[r] : 0);
        }
        cs.Cout += rows;
      }
      Wp = &Wm;
    }
    const std::vector<uint16_t> & W = *Wp;
    cs.K = is1 ? 1 : (is3 ? 3 : n.i("K", 3));
    cs.G = isg ? n.i("G", 1) : 1;
    const int cin_g = (int)(wt.numel / ((long)wt.dims.at(0) * cs.K * cs.K));
    const Tensor & x = *T_[is1 ? n.ins.at(1) : n.ins.at(0)];
    cs.Cin = is1 ? (int)wt.dims.at(1) : (grp ? mcin : cin_g * cs.G);
    if (is1) {
      const long N = x.numel / std::max(cs.Cin, 1);
      if (x.dims.size() == 4 && (long)x.H * x.W == N && x.C == cs.Cin) { cs.H = x.H; cs.W = x.W; }
      else { cs.H = (int)N; cs.W = 1; }
    } else {
      cs.H = x.H;
      cs.W = x.W;
      cs.S = is3 ? n.i("stride", 1) : n.i("S", 1);
      cs.P = is3 ? n.i("pad", 1) : n.i("P", 1);
    }
    cs.act = n.i("act");
    const std::string bname = n.ins.size() > 2 ? n.ins[2] : "-";
    cs.has_bias = bname != "-";
    const uint16_t * B = nullptr;
    if (cs.has_bias) {
      const auto & Bv = merged ? Bm : host.at(bname);
      if ((long)Bv.size() < cs.Cout) throw std::runtime_error("bias too short: " + bname);
      B = Bv.data();
    }
    // kernel family decided here, where layouts are known
    const Root & xr = *roots_[x.root < 0 ? 0 : x.root];
    cs.x_nhwc = x.kind == Tensor::kAct && xr.layout == kNHWC && (x.coff % 8) == 0;
    cs.x_vec1 = is1 && (long)cs.H * cs.W == 1 && x.kind != Tensor::kInit && (x.eoff % 8) == 0 && xr.layout == kNCHW;
    // a 1x1 conv on NCHW channel planes (e.g. the graph input): the implicit GEMM reads
    // 8-pixel pieces of each plane and transposes them in LDS
    cs.x_planes8 = is1 && !cs.x_vec1 && x.kind != Tensor::kInit && xr.layout == kNCHW && ((long)cs.H * cs.W) % 8 == 0 &&
                   (x.eoff % 8) == 0 && (xr.per_image % 8) == 0;
    cs.flags = flags_;
    Packed pk;
    pk.spec = cs;
    pk.pk = conv_packing(cs);
    std::vector<uint8_t> blob;
    conv_pack(cs, pk.pk, W.data(), B, blob);
    pk.dev = upload(blob.data(), blob.size());
    return pk;
  };
  packed_grp_.assign(nodes_.size(), Packed{});
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    const std::string & op = nodes_[ni].op;
    if (!(op == "conv1x1" || op == "conv3x3" || op == "conv_general") || skip_[ni]) continue;
    const int lead = sib_lead_[ni];
    if (lead >= 0 && lead != (int)ni && !sib_grouped_[lead]) continue;  // packed with its lead
    const bool grouped_lead = !sib_[ni].empty() && sib_grouped_[ni];
    packed_[ni] = pack_conv(ni, !sib_[ni].empty() && !grouped_lead);
    // a grouped lead also keeps its own packing (and its members theirs): at a batch whose
    // grouped launch does not get the ping-pong kernel they run one by one
    if (grouped_lead) packed_grp_[ni] = pack_conv(ni, true);
  }
  // split-K workspace: the largest need over every node and every batch size, so launch
  // lists and captured graphs of different batch sizes share one fixed buffer
  size_t need = 0;
  if (!(flags_ & IVH_FLAG_NO_SPLITK))
    for (size_t ni = 0; ni < nodes_.size(); ++ni)
      if (packed_[ni].dev) need = std::max(need, conv_splitk_floats(packed_[ni].spec, packed_[ni].pk, max_batch_));
  if (need) {
    ws_ = static_cast<float *>(devAlloc(need * 4, false));
    ws_floats_ = need;
  }
}

// ==================================================================== dispatch

View Model::view(const std::string & name, int batch) const
{
  const Tensor & t = *T_.at(name);
  View v;
  if (t.kind == Tensor::kInit) {
    v.ptr = static_cast<__half *>(init_dev_.at(name));
    v.img = 0;
    v.layout = kNCHW;
    v.cs = t.H * t.W;
    return v;
  }
  const Root & r = *roots_.at(t.root);
  __half * base;
  if (r.is_input) base = static_cast<__half *>(input_buf_);
  else base = static_cast<__half *>(arena_) + r.off1 * batch;
  v.img = r.per_image;
  v.layout = r.layout;
  if (r.layout == kNHWC) {
    v.ptr = base + t.coff;
    v.cs = r.cs;
  } else {
    v.ptr = base + t.eoff;
    v.cs = t.H * t.W;
  }
  return v;
}

// Nodes ni, ni + 1, ni + 2 are SPPF's chained max pools: 5x5, stride 1, pad 2, each reading
// the previous one's output (which may have other readers), same geometry.
bool Model::sppfChain(size_t ni) const
{
  if ((flags_ & IVH_FLAG_NO_FUSE) || ni + 2 >= nodes_.size()) return false;
  for (size_t k = ni; k < ni + 3; ++k) {
    const PlanNode & n = nodes_[k];
    if (n.op != "maxpool" || skip_[k] || n.i("K", 5) != 5 || n.i("S", 1) != 1 || n.i("P", 2) != 2 ||
        n.i("Hout") != n.i("H") || n.i("Wout") != n.i("W") || n.i("C") != nodes_[ni].i("C") ||
        n.i("H") != nodes_[ni].i("H") || n.i("W") != nodes_[ni].i("W") || n.ins.empty() || n.outs.size() != 1)
      return false;
    if (k > ni && n.ins[0] != nodes_[k - 1].outs[0]) return false;
  }
  return true;
}

// Bottleneck pairs: node A = conv3x3 (stride 1, pad 1, C -> C channels with C = 16 or 32, no
// residual) whose output has one reader, node B = conv3x3 (stride 1, pad 1, C -> C) on it, B's
// residual none or A's input, both activations among those the kernel has.  Structural only: whether the
// pair runs fused also depends on the views (pairLaunch); the liveness that allocate gives
// a pair is harmless when it does not.
void Model::findPairs()
{
  pair_next_.assign(nodes_.size(), -1);
  if (flags_ & (IVH_FLAG_NO_FUSE | IVH_FLAG_NO_FUSE_PAIR | IVH_FLAG_DIRECT_ONLY | IVH_FLAG_NO_HALO)) return;
  std::map<std::string, std::vector<int>> readers;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (const auto & in : nodes_[i].ins)
      if (in != "-") readers[in].push_back((int)i);
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  auto act_ok = [](int a) { return a == kActNone || a == kActSiLU || a == kActReLU || a == kActHSwish; };
  // (input, output) channels of a conv that can be a pair member (3x3 stride 1 pad 1, same
  // map size), else (0, 0)
  auto pair_io = [&](const PlanNode & n) {
    const std::pair<int, int> none{0, 0};
    if (n.op != "conv3x3" || n.ins.size() < 2 || n.outs.size() != 1 || n.i("stride", 1) != 1 || n.i("pad", 1) != 1)
      return none;
    const Tensor & w = *T_.at(n.ins[1]);
    const Tensor & x = *T_.at(n.ins[0]);
    const bool ok = w.dims.size() == 4 && w.dims[1] == x.C && w.dims[2] == 3 && w.dims[3] == 3 &&
                    n.i("Hout") == x.H && n.i("Wout") == x.W && act_ok(n.i("act"));
    return ok ? std::pair<int, int>{x.C, (int)w.dims[0]} : none;
  };
  std::vector<char> used(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i) {
    const PlanNode & a = nodes_[i];
    if (used[i]) continue;
    const auto io = pair_io(a);
    const int c = io.first, mid = io.second;
    if (!pair_channels_ok(c, mid) || (a.ins.size() > 3 && a.ins[3] != "-")) continue;
    const std::string & t = a.outs[0];
    const auto it = readers.find(t);
    if (it == readers.end() || it->second.size() != 1 || outs.count(t)) continue;
    const int j = it->second[0];
    const PlanNode & b = nodes_[j];
    if (j <= (int)i || used[j] || pair_io(b) != std::pair<int, int>{mid, c} || b.ins[0] != t) continue;
    if (b.ins.size() > 3 && b.ins[3] != "-" && b.ins[3] != a.ins[0]) continue;
    if (T_.at(b.ins[0])->H != T_.at(a.ins[0])->H || T_.at(b.ins[0])->W != T_.at(a.ins[0])->W) continue;
    pair_next_[i] = j;
    used[i] = used[j] = 1;
  }
}

// Sibling merge: 3x3 convs that read the same tensor with the same stride, pad and
// activation (a Pose head's box, class and keypoint branches each start with one) run as one
// conv over the concatenated output channels, so x is read once and the MFMA tiles are
// fuller.  Each member's output becomes a channel view of one root (assignViews), whose
// readers must therefore all be convs; members with Cout % 8 != 0 are allowed only last, so
// every view starts on a 16-byte boundary.
void Model::findSiblings()
{
  sib_.assign(nodes_.size(), {});
  sib_lead_.assign(nodes_.size(), -1);
  sib_grouped_.assign(nodes_.size(), 0);
  sib_x_.assign(nodes_.size(), std::string());
  sib_cout_.assign(nodes_.size(), 0);
  if (flags_ & (IVH_FLAG_NO_FUSE | IVH_FLAG_NO_FUSE_SIBLINGS | IVH_FLAG_NCHW_ONLY | IVH_FLAG_DIRECT_ONLY)) return;
  std::map<std::string, std::vector<int>> readers;
  for (size_t i = 0; i < nodes_.size(); ++i)
    for (size_t k = 0; k < nodes_[i].ins.size(); ++k)
      if (nodes_[i].ins[k] != "-") readers[nodes_[i].ins[k]].push_back((int)i);
  std::set<std::string> outs(outputs_.begin(), outputs_.end());
  std::vector<char> paired(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i)
    if (pair_next_[i] >= 0) paired[i] = paired[pair_next_[i]] = 1;
  auto member_ok = [&](size_t j) {
    const PlanNode & n = nodes_[j];
    if (n.op != "conv3x3" || paired[j] || n.ins.size() < 3 || n.outs.size() != 1 || (n.ins.size() > 3 && n.ins[3] != "-"))
      return false;
    const Tensor & x = *T_.at(n.ins[0]);
    const Tensor & w = *T_.at(n.ins[1]);
    const Tensor & y = *T_.at(n.outs[0]);
    if (x.kind != Tensor::kAct || w.kind != Tensor::kInit || w.dims.size() != 4 || w.dims[1] != x.C ||
        y.kind != Tensor::kAct || y.dims.size() != 4 || y.C != w.dims[0] || outs.count(y.name) || n.ins[2] == "-")
      return false;
    // every reader of the output is a conv reading it as its input
    const auto it = readers.find(y.name);
    if (it == readers.end()) return false;
    for (int u : it->second) {
      const PlanNode & un = nodes_[u];
      const bool conv_in = ((un.op == "conv3x3" || un.op == "conv_general") && un.ins[0] == y.name &&
                            std::count(un.ins.begin(), un.ins.end(), y.name) == 1) ||
                           (un.op == "conv1x1" && un.ins.size() > 1 && un.ins[1] == y.name &&
                            std::count(un.ins.begin(), un.ins.end(), y.name) == 1);
      if (!conv_in) return false;
    }
    return true;
  };
  std::vector<char> taken(nodes_.size(), 0);
  for (size_t i = 0; i < nodes_.size(); ++i) {
    if (taken[i] || !member_ok(i)) continue;
    const PlanNode & a = nodes_[i];
    std::vector<int> g{(int)i};
    for (int j : readers[a.ins[0]]) {
      if (j <= (int)i || taken[j] || !member_ok(j)) continue;
      const PlanNode & b = nodes_[j];
      if (b.ins[0] != a.ins[0] || b.i("stride", 1) != a.i("stride", 1) || b.i("pad", 1) != a.i("pad", 1) ||
          b.i("act") != a.i("act") || b.i("Hout") != a.i("Hout") || b.i("Wout") != a.i("Wout"))
        continue;
      g.push_back(j);
    }
    if (g.size() < 2) continue;
    // channel order: 8-aligned members first (node order), then at most one ragged one
    std::vector<int> even, odd;
    for (int j : g) (T_.at(nodes_[j].outs[0])->C % 8 ? odd : even).push_back(j);
    if (odd.size() > 1) odd.resize(1);
    if (even.empty() || even.size() + odd.size() < 2) continue;
    even.insert(even.end(), odd.begin(), odd.end());
    for (int j : even) {
      taken[j] = 1;
      sib_lead_[j] = (int)i;
    }
    sib_[i] = even;
    int sum = 0;
    bool blocks = true;
    for (size_t k = 0; k < even.size(); ++k) {
      const int c = T_.at(nodes_[even[k]].outs[0])->C;
      sum += c;
      if (k + 1 < even.size() ? c % 64 != 0 : c > 64) blocks = false;
    }
    const int act = a.i("act");
    const bool act0 = act == kActNone || act == kActSiLU || act == kActReLU || act == kActHSwish;  // act(0) = 0
    sib_cout_[i] = blocks && act0 ? 64 * (int)even.size() : sum;
  }
  // Grouped siblings: the merged members' own next convs (3x3 stride 1, 64 -> 64, each the
  // one reader of its member's output) read consecutive 64-channel views of the merged root;
  // as a grouped conv on the ping-pong kernel (channel block y reads input channels 64 y ..)
  // they are one launch.  The members' outputs must be whole 64-channel blocks from channel 0.
  if (flags_ & (IVH_FLAG_NO_RESIDENT | IVH_FLAG_NO_PINGPONG | IVH_FLAG_PIPE_ANY)) return;
  const size_t n_first = nodes_.size();
  for (size_t i = 0; i < n_first; ++i) {
    if (sib_[i].empty() || sib_grouped_[i]) continue;
    // the last member's output may be narrower than 64 channels when the merge writes its
    // padding channels (zeros): its next conv then runs as a 64-channel group of zero-padded
    // weights
    const bool padded = sib_cout_[i] == 64 * (int)sib_[i].size();
    std::vector<int> tw;
    int off = 0, cout = 0;
    for (size_t k = 0; k < sib_[i].size(); ++k) {
      const Tensor & t = *T_.at(nodes_[sib_[i][k]].outs[0]);
      const bool last = k + 1 == sib_[i].size();
      const auto it = readers.find(t.name);
      if (!(t.C == 64 || (last && padded && t.C < 64)) || off != 64 * (int)tw.size() || it == readers.end() ||
          it->second.size() != 1)
        break;
      const int r = it->second[0];
      const PlanNode & rn = nodes_[r];
      const auto & wd = T_.at(rn.ins[1])->dims;
      if (taken[r] || !member_ok(r) || rn.ins[0] != t.name || rn.i("stride", 1) != 1 || rn.i("pad", 1) != 1 ||
          wd.size() != 4 || wd[1] != t.C || wd[2] != 3 || wd[3] != 3 || wd[0] > 64 || (!last && wd[0] != 64) ||
          rn.i("Hout") != t.H || rn.i("Wout") != t.W || (!tw.empty() && rn.i("act") != nodes_[tw[0]].i("act")))
        break;
      tw.push_back(r);
      off += 64;
      cout += (int)wd[0];
    }
    if (tw.size() < 2) continue;
    const int lead = *std::min_element(tw.begin(), tw.end());
    for (int r : tw) {
      taken[r] = 1;
      sib_lead_[r] = lead;
    }
    sib_[lead] = tw;
    sib_grouped_[lead] = 1;
    sib_x_[lead] = nodes_[sib_[i][0]].outs[0];
    sib_cout_[lead] = cout;
  }
}

bool Model::pairLaunch(size_t ni, int batch, Launch & L)
{
  const int nj = pair_next_[ni];
  if (nj < 0) return false;
  Launch A = convLaunch(ni, batch), B = convLaunch((size_t)nj, batch);
  if (A.kind != Launch::kIgemm || B.kind != Launch::kIgemm) return false;
  // both convs' LDS-patch packing of one channel chunk: [C rows][taps][C channels], 9 taps
  // with C = 32, 10 (a zero tenth) with C = 16.  A middle of M = C / 2 channels runs as C:
  // the first conv's rows past M and the second conv's channels past M are the packing's
  // zero padding, so the padded channels of t are act(0) = 0 and add nothing.
  const int C = A.cp.Cin, M = A.cp.Cout, hi = C == 16 ? 0 : 1, kpad = halo_taps(C) * C;  // halo segments 0: ck 16, 1: ck 32
  if (!pair_channels_ok(C, M) || B.cp.Cin != M || B.cp.Cout != C) return false;
  const std::pair<ConvParams *, size_t> convs[2] = {{&A.cp, ni}, {&B.cp, (size_t)nj}};
  for (const auto & pr : convs) {
    const Packed & pk = packed_[pr.second];
    if (pk.pk.halo[hi] == kNoSeg || pk.pk.kpad_halo[hi] != kpad || !pk.dev) return false;
    pr.first->w = reinterpret_cast<const __half *>(static_cast<const char *>(pk.dev) + pk.pk.halo[hi]);
    pr.first->kpad = kpad;
  }
  const ConvParams & a = A.cp;
  ConvParams & b = B.cp;
  auto nhwc16 = [&](const View & v) {
    return v.layout == kNHWC && v.cs % 8 == 0 && v.img % 8 == 0 && (reinterpret_cast<uintptr_t>(v.ptr) % 16) == 0;
  };
  if (!nhwc16(a.x) || !nhwc16(b.y) || a.H != b.H || a.W != b.W) return false;
  if (b.r.ptr && (b.r.ptr != a.x.ptr || b.r.img != a.x.img || b.r.cs != a.x.cs || b.r.layout != a.x.layout)) return false;
  const long xl = (long)(batch - 1) * a.x.img + ((long)a.H * a.W - 1) * a.x.cs + C;
  const long yl = (long)(batch - 1) * b.y.img + ((long)b.H * b.W - 1) * b.y.cs + C;
  if (xl * 2 >= (1L << 31) || yl * 2 >= (1L << 31) || (long)a.W * a.x.cs >= (1L << 23)) return false;
  int th, tw;
  if (!pair_plan(C, b.H, b.W, batch, &th, &tw)) return false;
  b.th = th;
  b.tw = tw;
  b.pipe = b.wide = b.res = b.halo = b.s2 = 0;
  b.ksplit = 1;
  b.ws = nullptr;
  L.kind = Launch::kPair;
  L.cp = b;
  L.cp2 = a;
  return true;
}

Launch Model::convLaunch(size_t ni, int batch, bool grouped)
{
  const PlanNode & n = nodes_[ni];
  const Tensor & yt = *T_[n.outs[0]];
  auto has = [&](size_t i) { return i < n.ins.size() && n.ins[i] != "-"; };
  auto fail = [&](const std::string & m) { throw std::runtime_error("node " + n.op + " -> " + yt.name + ": " + m); };
  const bool is1 = n.op == "conv1x1", is3 = n.op == "conv3x3", isg = n.op == "conv_general";
  {
    const Packed & pk = grouped ? packed_grp_.at(ni) : packed_[ni];
    const Tensor & wt = *T_[is1 ? n.ins[0] : n.ins[1]];
    const Tensor & xt = *T_[is1 ? n.ins[1] : n.ins[0]];
    Launch L;
    ConvParams & p = L.cp;
    p.batch = batch;
    p.Cout = (int)wt.dims[0];
    // merged siblings: all members' channels, written from channel 0 of their shared root
    const Tensor * ymerged = nullptr;
    if (!sib_[ni].empty() && (grouped || !sib_grouped_[ni])) {
      p.Cout = sib_cout_[ni];
      ymerged = T_[nodes_[sib_[ni][0]].outs[0]].get();
      const Root & mr = *roots_.at(ymerged->root);
      if (ymerged->coff != 0 || p.Cout < mr.C || p.Cout > (mr.layout == kNHWC ? mr.cs : mr.C)) fail("merged sibling root");
    }
    if (is1) {
      p.Cin = (int)wt.dims[1];
      const long N = xt.numel / std::max(p.Cin, 1);
      if (xt.numel != N * p.Cin) fail("x numel not a multiple of Cin");
      if (xt.dims.size() == 4 && (long)xt.H * xt.W == N && xt.C == p.Cin) { p.H = xt.H; p.W = xt.W; }
      else { p.H = (int)N; p.W = 1; }
      p.K = 1; p.S = 1; p.P = 0; p.G = 1;
      p.Ho = p.H; p.Wo = p.W;
    } else {
      p.Cin = grouped ? 64 : xt.C;
      p.H = xt.H; p.W = xt.W;
      p.K = is3 ? 3 : n.i("K", 3);
      p.S = is3 ? n.i("stride", 1) : n.i("S", 1);
      p.P = is3 ? n.i("pad", 1) : n.i("P", 1);
      p.G = isg ? n.i("G", 1) : 1;
      p.Ho = n.i("Hout"); p.Wo = n.i("Wout");
      if (p.Ho != (p.H + 2 * p.P - p.K) / p.S + 1 || p.Wo != (p.W + 2 * p.P - p.K) / p.S + 1)
        fail("Hout/Wout inconsistent with input geometry");
      if (!ymerged && wt.numel != (long)p.Cout * (p.Cin / p.G) * p.K * p.K) fail("weight shape mismatch");
    }
    if (p.G < 1 || p.Cin % p.G || p.Cout % p.G) fail("bad groups");
    const Tensor & yv = ymerged ? *ymerged : yt;
    if (ymerged ? yv.H != p.Ho || yv.W != p.Wo : yt.numel != (long)p.Cout * p.Ho * p.Wo)
      fail("output numel mismatch");
    p.act = n.i("act");
    p.x = view(grouped ? sib_x_[ni] : xt.name, batch);
    if (grouped) p.xg = 64;
    p.y = view(yv.name, batch);
    if (p.y.layout == kNHWC && yv.kind != Tensor::kInit) {
      const Root & yr = *roots_.at(yv.root);
      if (yv.coff + p.Cout == yr.C) p.ypad = yr.cs - yr.C;
    }
    if (has(3)) {
      const Tensor & rt = *T_[n.ins[3]];
      if (rt.numel != yt.numel) fail("residual numel mismatch");
      p.r = view(rt.name, batch);
    }
    if (up_src_[ni] >= 0) {
      const PlanNode & rn = nodes_[up_src_[ni]];
      p.xu = view(rn.ins[0], batch);
      p.cu = rn.i("C");
    }
    // single-pixel tensors: NCHW and NHWC coincide; present them channels-last
    auto pix1 = [](View & v, int C) { v.layout = kNHWC; v.cs = (int)round_up(C, 8); };
    if (p.H * p.W == 1) pix1(p.x, p.Cin);
    if (p.Ho * p.Wo == 1) { pix1(p.y, p.Cout); if (p.r.ptr) pix1(p.r, p.Cout); }
    if (!pk.dev || pk.spec.Cin != p.Cin || pk.spec.Cout != p.Cout || pk.spec.H != p.H || pk.spec.W != p.W ||
        pk.spec.K != p.K || pk.spec.G != p.G || pk.spec.Ho() != p.Ho || pk.spec.Wo() != p.Wo)
      fail("packed conv geometry");
    int k;
    try {
      k = conv_resolve(pk.spec, pk.pk, pk.dev, batch, (flags_ & IVH_FLAG_NO_SPLITK) ? nullptr : ws_, p);
    } catch (const std::exception & e) {
      fail(e.what());
    }
    L.kind = k == kLaunchIgemm ? Launch::kIgemm : (k == kLaunchDirect ? Launch::kDirect : Launch::kDw);
    return L;
  }

  fail("not a conv node");
  return Launch{};
}

void Model::emitNode(size_t ni, int batch, std::vector<Launch> & out, std::vector<char> & covered)
{
  const PlanNode & n = nodes_[ni];
  const Tensor & yt = *T_[n.outs[0]];
  auto fail = [&](const std::string & m) { throw std::runtime_error("node " + n.op + " -> " + yt.name + ": " + m); };
  if (n.op == "attention") {
    Launch L;
    L.kind = Launch::kAttn;
    AttnParams & a = L.ap;
    a.batch = batch;
    a.heads = n.i("heads");
    a.n = n.i("n");
    a.scale = h2f((uint16_t)n.i("scale_bits"));
    a.scale_q = n.i("scale_q");
    a.q = view(n.ins.at(0), batch);
    a.k = view(n.ins.at(1), batch);
    a.v = view(n.ins.at(2), batch);
    a.y = view(yt.name, batch);
    // per-head blocks of dense NCHW tensors: the view's channel stride is one head's block
    const long nn = a.n;
    for (View * v : {&a.q, &a.k, &a.v, &a.y}) {
      if (v->layout != kNCHW) fail("attention operands must be NCHW");
      const long blk = (v == &a.q || v == &a.k) ? kAttnKD * nn : kAttnHD * nn;
      const Tensor & t = *T_[v == &a.q ? n.ins[0] : v == &a.k ? n.ins[1] : v == &a.v ? n.ins[2] : yt.name];
      if (t.numel != blk * a.heads) fail("attention operand size");
      v->cs = (int)blk;  // head stride
      if ((reinterpret_cast<uintptr_t>(v->ptr) & 15) || (v->img & 7)) fail("attention operand alignment");
    }
    out.push_back(L);
    return;
  }
  if (n.op == "pose_decode") {
    Launch L;
    L.kind = Launch::kDecode;
    DecodeParams & d = L.dp;
    d.batch = batch;
    d.nscale = n.i("S");
    d.R = n.i("R");
    d.nc = n.i("nc");
    d.nk = n.i("nk");
    d.A = n.i("A");
    d.box_div = n.i("box_div");
    const int split = n.i("split");
    if (d.nscale < 1 || d.nscale > 4 || d.R < 1 || d.R > 64 || d.nc < 1 || d.nk < 0 || d.A < 1) fail("decode attributes");
    // per scale: box (4R) + classes (nc) in one tensor, or (split) box and classes apart
    const int no = 4 * d.R + (split ? 0 : d.nc), nkc = 3 * d.nk, ny = 4 + d.nc + nkc;
    const size_t base = (size_t)d.nscale * (1 + (split ? 1 : 0) + (d.nk ? 1 : 0));
    const size_t kfirst = (size_t)d.nscale * (split ? 2 : 1);
    if (n.ins.size() != base + 6) fail("decode inputs");
    // the heads stay NCHW (the decode is no channels-last reader): per-channel reads are
    // coalesced and the narrow head convs (1 or 51 channels) write NCHW rows faster
    long off = 0;
    d.nchw = 1;
    for (int s = 0; s < d.nscale; ++s) {
      const long hw = n.i(("hw" + std::to_string(s)).c_str());
      d.off[s] = (int)off;
      const Tensor & xt = *T_.at(n.ins[s]);
      if (xt.C != no || (long)xt.H * xt.W != hw || xt.numel != no * hw) fail("decode head geometry");
      d.x[s] = view(xt.name, batch);
      if (d.x[s].layout != kNCHW) d.nchw = 0;
      if (split) {
        const Tensor & ct = *T_.at(n.ins[d.nscale + s]);
        if (ct.C != d.nc || (long)ct.H * ct.W != hw || ct.numel != (long)d.nc * hw) fail("decode class geometry");
        d.c[s] = view(ct.name, batch);
        if (d.c[s].layout != kNCHW) d.nchw = 0;
      } else {  // the class channels follow the 4R box channels of the same tensor
        d.c[s] = d.x[s];
        d.c[s].ptr = d.x[s].ptr + (d.x[s].layout == kNCHW ? (long)4 * d.R * d.x[s].cs : (long)4 * d.R);
      }
      if (d.nk) {
        const Tensor & kt = *T_.at(n.ins[kfirst + s]);
        if (kt.C != nkc || (long)kt.H * kt.W != hw || kt.numel != nkc * hw) fail("decode keypoint geometry");
        d.k[s] = view(kt.name, batch);
        if (d.k[s].layout != kNCHW) d.nchw = 0;
      }
      off += hw;
    }
    if (off != d.A || yt.numel != (long)ny * d.A) fail("decode anchor count");
    auto konst = [&](size_t i, long numel) -> const __half * {
      const Tensor & t = *T_.at(n.ins.at(i));
      if (t.kind != Tensor::kInit || t.numel != numel) fail("decode constant " + t.name);
      return static_cast<const __half *>(init_dev_.at(t.name));
    };
    d.dflw = konst(base, d.R);
    d.anc = konst(base + 1, 2L * d.A);
    d.st = konst(base + 2, d.A);
    d.cbox = konst(base + 4, 1);
    if (d.nk) {
      d.ancm = konst(base + 3, 2L * d.A);
      d.ckpt = konst(base + 5, 1);
    }
    d.y = view(yt.name, batch);
    if (d.y.layout != kNCHW) fail("decode output must be NCHW");
    d.y.cs = d.A;
    out.push_back(L);
    return;
  }
  const bool is1 = n.op == "conv1x1", is3 = n.op == "conv3x3", isg = n.op == "conv_general";
  if (is1 || is3 || isg) {
    // grouped siblings: one launch when it gets the ping-pong kernel (the one family with a
    // grouped input), else every member launches by itself
    if (!sib_[ni].empty() && sib_grouped_[ni]) {
      Launch G = convLaunch(ni, batch, true);
      if (G.kind == Launch::kIgemm && G.cp.res == 4) {
        out.push_back(G);
        for (int j : sib_[ni])
          if (j != (int)ni) covered[j] = 1;
        return;
      }
    }
    if (pair_next_[ni] >= 0) {
      Launch P;
      if (pairLaunch(ni, batch, P)) {
        out.push_back(P);
        covered[pair_next_[ni]] = 1;
        return;
      }
    }
    out.push_back(convLaunch(ni, batch));
    return;
  }

  Launch L;
  L.kind = Launch::kSmall;
  SmallParams & q = L.sp;
  q.batch = batch;
  q.y = view(yt.name, batch);
  q.C = yt.C; q.H = yt.H; q.W = yt.W;
  const std::string & op = n.op;
  if (op == "reshape" || op == "flatten") {  // init source: materialise by a copy
    q.a = view(n.ins[0], batch);
    q.C = 1; q.H = 1; q.W = (int)yt.numel;
    q.a.layout = q.y.layout = kNCHW;
    q.a.cs = q.y.cs = (int)yt.numel;
    L.small = kCopy;
    out.push_back(L);
    return;
  }
  if (op == "ew_binary") {
    const Tensor & at = *T_[n.ins.at(0)];
    const Tensor & bt = *T_[n.ins.at(1)];
    q.op = n.i("op");
    q.a = view(at.name, batch);
    q.b = view(bt.name, batch);
    if (!n.has("bdims") || n.i("b_scalar") == 1) {
      if (n.i("b_scalar") == 1) {
        if (at.numel != yt.numel || bt.numel < 1) fail("scalar ew_binary shapes");
        q.b.img = 0;
        q.b.cs = 0;
      } else if (at.numel != yt.numel || bt.numel != yt.numel) {
        fail("ew_binary without bdims needs equal numel");
      }
      // dense NCHW operands of equal numel are walked in the output's (C, H*W) order
      if (q.a.layout == kNCHW) q.a.cs = yt.H * yt.W;
      if (q.b.layout == kNCHW && q.b.img | q.b.cs) q.b.cs = yt.H * yt.W;
      L.small = kEwSame;
      out.push_back(L);
      return;
    }
    // per-channel broadcast (ew_binary_ch) when one operand is [.., C, 1, 1]
    const int a_is_chan = chanBroadcast(n);
    if (a_is_chan >= 0) {
      q.i0 = a_is_chan;
      L.small = kEwChan;
      out.push_back(L);
      return;
    }
    // general broadcast: NCHW flat
    std::vector<int> v;
    {
      std::stringstream ss(n.str("bdims"));
      std::string tk;
      while (std::getline(ss, tk, ',')) v.push_back(std::atoi(tk.c_str()));
    }
    const int rank = (int)v.size() / 3;
    if (rank < 1 || rank > 6 || (int)v.size() != rank * 3) fail("bad bdims");
    long no = 1, amax = 0, bmax = 0;
    for (int r = 0; r < rank; ++r) {
      no *= v[r];
      amax += (long)(v[r] - 1) * v[rank + r];
      bmax += (long)(v[r] - 1) * v[2 * rank + r];
    }
    if (no != yt.numel || amax >= at.numel || bmax >= bt.numel) fail("bdims out of operand bounds");
    if (q.a.layout != kNCHW || q.b.layout != kNCHW || q.y.layout != kNCHW) fail("broadcast needs NCHW operands");
    q.rank = rank;
    for (int i = 0; i < rank * 3; ++i) q.dims[i] = v[i];
    q.n = yt.numel;
    L.small = kEwBcast;
    out.push_back(L);
    return;
  }
  if (op == "ew_unary") {
    const Tensor & at = *T_[n.ins.at(0)];
    if (at.numel != yt.numel) fail("ew_unary numel");
    q.a = view(at.name, batch);
    if (q.a.layout == kNCHW) q.a.cs = yt.H * yt.W;
    q.op = unary_to_act(n.i("op"));
    L.small = kEwUnary;
    out.push_back(L);
    return;
  }
  if (op == "bias_add") {
    const Tensor & at = *T_[n.ins.at(0)];
    const Tensor & bt = *T_[n.ins.at(1)];
    q.a = view(at.name, batch);
    q.b = view(bt.name, batch);
    q.i0 = std::max(1, n.i("HW", 1));
    q.n = yt.numel;
    if (at.numel != yt.numel || (yt.numel - 1) / q.i0 >= bt.numel) fail("bias_add shapes");
    if (q.a.layout != kNCHW || q.y.layout != kNCHW) fail("bias_add needs NCHW");
    L.small = kBiasAdd;
    out.push_back(L);
    return;
  }
  if (op == "copy_c") {  // not a view: copy `cnt` channels into y at dst_off
    const Tensor & xt = *T_[n.ins.at(0)];
    const int HW = n.i("HW", 1), c0 = n.i("c0"), cnt = n.i("cnt"), dst = n.i("dst_off");
    if ((long)(c0 + cnt) * HW > xt.numel || dst + (long)cnt * HW > yt.numel) fail("copy_c bounds");
    View xv = view(xt.name, batch), yv = view(yt.name, batch);
    if (xv.layout == kNHWC) {
      if ((long)xt.H * xt.W != HW || dst != 0) fail("copy_c on channels-last input");
      q.a = xv;
      q.a.ptr += c0;
    } else {
      q.a = xv;
      q.a.ptr += (long)c0 * HW;
      q.a.cs = HW;
    }
    if (yv.layout == kNHWC) {
      if (dst != 0) fail("copy_c dst_off on channels-last output");
      q.y = yv;
    } else {
      q.y = yv;
      q.y.ptr += dst;
      q.y.cs = HW;
    }
    q.C = cnt; q.H = 1; q.W = HW;
    L.small = kCopy;
    out.push_back(L);
    return;
  }
  if (op == "slice_axis") {
    const Tensor & xt = *T_[n.ins.at(0)];
    q.a = view(xt.name, batch);
    q.i0 = n.i("outer", 1); q.i1 = n.i("axdim"); q.i2 = n.i("inner", 1); q.i3 = n.i("start"); q.i4 = n.i("len");
    if ((long)q.i0 * q.i1 * q.i2 > xt.numel || q.i3 + q.i4 > q.i1 || (long)q.i0 * q.i4 * q.i2 != yt.numel)
      fail("slice_axis bounds");
    if (q.a.layout != kNCHW || q.y.layout != kNCHW) fail("slice_axis needs NCHW");
    L.small = kSliceAxis;
    out.push_back(L);
    return;
  }
  if (op == "concat4") {
    const int cnt[4] = {n.i("ca"), n.i("cb"), n.i("cc"), n.i("cd")};
    const int outer = n.i("outer", 1), inner = n.i("inner", 1);
    const int tot = cnt[0] + cnt[1] + cnt[2] + cnt[3];
    if ((long)outer * tot * inner != yt.numel) fail("concat4 geometry");
    int off = 0;
    for (int j = 0; j < 4; ++j) {
      if (cnt[j] <= 0) continue;
      const Tensor & st = *T_[n.ins.at(j)];
      if (st.numel != (long)outer * cnt[j] * inner) fail("concat4 input numel");
      Launch Lj = L;
      SmallParams & qj = Lj.sp;
      qj.a = view(st.name, batch);
      if (outer == 1) {
        // skip inputs already written in place by their producer
        if (st.kind == Tensor::kAct && st.root == yt.root && st.coff == yt.coff + off) { off += cnt[j]; continue; }
        qj.y = view(yt.name, batch);
        if (qj.y.layout == kNHWC) qj.y.ptr += off;
        else { qj.y.ptr += (long)off * inner; qj.y.cs = inner; }
        if (qj.a.layout == kNCHW) qj.a.cs = inner;
        qj.C = cnt[j]; qj.H = 1; qj.W = inner;
        if (qj.y.layout == kNHWC || qj.a.layout == kNHWC) {
          if ((long)yt.H * yt.W != inner || (long)st.H * st.W != inner) fail("concat4 channels-last geometry");
          qj.H = yt.H; qj.W = yt.W;
        }
        Lj.small = kCopy;
      } else {
        if (qj.a.layout != kNCHW || qj.y.layout != kNCHW) fail("concat4 outer>1 needs NCHW");
        qj.i0 = outer; qj.i1 = cnt[j]; qj.i2 = inner; qj.i3 = tot; qj.i4 = off;
        Lj.small = kConcatOuter;
      }
      out.push_back(Lj);
      off += cnt[j];
    }
    return;
  }
  if (op == "maxpool" || op == "resize_nn") {
    const Tensor & xt = *T_[n.ins.at(0)];
    q.a = view(xt.name, batch);
    q.C = n.i("C"); q.H = n.i("H"); q.W = n.i("W");
    if (op == "maxpool") {
      q.Ho = n.i("Hout"); q.Wo = n.i("Wout");
      q.K = n.i("K", 5); q.S = n.i("S", 1); q.P = n.i("P", 2);
      L.small = kMaxPool;
    } else {
      q.i0 = std::max(1, n.i("S", 2));
      q.Ho = q.H * q.i0; q.Wo = q.W * q.i0;
      L.small = kResizeNN;
    }
    if ((long)q.C * q.H * q.W != xt.numel || (long)q.C * q.Ho * q.Wo != yt.numel) fail("pool/resize geometry");
    if ((q.a.layout == kNHWC && (long)xt.H * xt.W != (long)q.H * q.W) ||
        (q.y.layout == kNHWC && (long)yt.H * yt.W != (long)q.Ho * q.Wo))
      fail("pool/resize channels-last geometry");
    if (q.a.layout == kNCHW) q.a.cs = q.H * q.W;
    if (q.y.layout == kNCHW) q.y.cs = q.Ho * q.Wo;
    // SPPF: the three chained pools as one launch when every view is 16-byte channels-last
    // and the plane's four LDS copies fit in 64 KB
    if (op == "maxpool" && sppfChain(ni)) {
      Launch F = L;
      SmallParams & f = F.sp;
      f.b = view(nodes_[ni + 1].outs[0], batch);
      f.c = view(nodes_[ni + 2].outs[0], batch);
      auto v8 = [&](const View & v, const std::string & t) {
        return v.layout == kNHWC && v.cs % 8 == 0 && v.img % 8 == 0 && T_.at(t)->coff % 8 == 0 &&
               (reinterpret_cast<uintptr_t>(v.ptr) & 15) == 0;
      };
      if (q.C % 8 == 0 && (long)q.H * q.W <= 1024 && v8(f.a, n.ins[0]) && v8(f.y, n.outs[0]) &&
          v8(f.b, nodes_[ni + 1].outs[0]) && v8(f.c, nodes_[ni + 2].outs[0])) {
        F.small = kMaxPoolSppf;
        out.push_back(F);
        covered[ni + 1] = covered[ni + 2] = 1;
        return;
      }
    }
    out.push_back(L);
    return;
  }
  if (op == "softmax_axis") {
    const Tensor & xt = *T_[n.ins.at(0)];
    q.a = view(xt.name, batch);
    q.i0 = n.i("outer", 1); q.i1 = n.i("axdim"); q.i2 = n.i("inner", 1);
    if ((long)q.i0 * q.i1 * q.i2 != xt.numel || xt.numel != yt.numel) fail("softmax geometry");
    if (q.a.layout != kNCHW || q.y.layout != kNCHW) fail("softmax needs NCHW");
    L.small = kSoftmax;
    out.push_back(L);
    return;
  }
  if (op == "permute_0213") {
    const Tensor & xt = *T_[n.ins.at(0)];
    q.a = view(xt.name, batch);
    q.i0 = n.i("D1", 1); q.i1 = n.i("D2", 1); q.i2 = n.i("I", 1); q.op = n.i("mode");
    if ((long)q.i0 * q.i1 * q.i2 != xt.numel || xt.numel != yt.numel) fail("permute geometry");
    if (q.a.layout != kNCHW || q.y.layout != kNCHW) fail("permute needs NCHW");
    L.small = kPermute;
    out.push_back(L);
    return;
  }
  if (op == "gap") {
    const Tensor & xt = *T_[n.ins.at(0)];
    q.a = view(xt.name, batch);
    q.C = n.i("C");
    const int HW = n.i("HW", 1);
    q.H = 1; q.W = HW;
    if ((long)q.C * HW != xt.numel || yt.numel != q.C) fail("gap geometry");
    if (q.a.layout == kNHWC) { q.H = xt.H; q.W = xt.W; }
    else q.a.cs = HW;
    L.small = kGap;
    out.push_back(L);
    return;
  }
  if (op == "gemm") {
    // C[M][N] = A[M][K] . B[K][N] with M = A.dims[0], K = A.dims[1] and N = numel(B) / K, so
    // B may have any rank (src/PlanModel.cpp:3935-3940); A and B are read row-major.
    const Tensor & at = *T_[n.ins.at(0)];
    const Tensor & bt = *T_[n.ins.at(1)];
    q.a = view(at.name, batch);
    q.b = view(bt.name, batch);
    if (at.dims.size() < 2) fail("gemm rank");
    const long M = at.dims[0], K = at.dims[1];
    if (M <= 0 || K <= 0) fail("gemm dims");
    const long Nn = bt.numel / K;
    if (Nn <= 0) fail("gemm: B smaller than K");
    if (M * Nn != yt.numel) fail("gemm output numel");
    if (M > INT32_MAX || Nn > INT32_MAX) fail("gemm dims");
    q.i0 = 1; q.i1 = (int)M; q.i2 = (int)K; q.i3 = (int)Nn;
    q.op = 0;
    if (q.a.layout != kNCHW || q.b.layout != kNCHW || q.y.layout != kNCHW) fail("matmul needs NCHW");
    L.small = kBmm;
    out.push_back(L);
    return;
  }
  if (op == "bmm") {
    const Tensor & at = *T_[n.ins.at(0)];
    const Tensor & bt = *T_[n.ins.at(1)];
    q.a = view(at.name, batch);
    q.b = view(bt.name, batch);
    const auto & ad = at.dims;
    const auto & bd = bt.dims;
    if (ad.size() < 2 || bd.size() < 2) fail("matmul rank");
    // operands folded from a last-two-dims permute are stored transposed (fusePermuteMatmul)
    const bool ta = n.i("ta") == 1, tb = n.i("tb") == 1;
    const int M = (int)(ta ? ad.back() : ad[ad.size() - 2]), K = (int)(ta ? ad[ad.size() - 2] : ad.back());
    const int Nn = (int)(tb ? bd[bd.size() - 2] : bd.back()), Kb = (int)(tb ? bd.back() : bd[bd.size() - 2]);
    if (Kb != K) fail("matmul inner dimensions differ");
    const long BB = at.numel / ((long)M * K);
    if ((long)K * Nn * BB != bt.numel) fail("matmul operand shapes");
    if (BB * M * Nn != yt.numel) fail("matmul output numel");
    q.i0 = (int)BB; q.i1 = M; q.i2 = K; q.i3 = Nn;
    q.op = (ta ? 1 : 0) | (tb ? 2 : 0);
    if (q.a.layout != kNCHW || q.b.layout != kNCHW || q.y.layout != kNCHW) fail("matmul needs NCHW");
    L.small = kBmm;
    out.push_back(L);
    return;
  }
  throw std::runtime_error("PlanModel: unknown op: " + op);
}

const Model::LaunchPlan & Model::launches(int batch)
{
  auto it = launch_cache_.find(batch);
  if (it != launch_cache_.end()) return it->second;
  LaunchPlan P;
  P.begin.assign(nodes_.size(), 0);
  P.end.assign(nodes_.size(), 0);
  P.covered.assign(nodes_.size(), 0);
  for (int r : up_src_)
    if (r >= 0) P.covered[r] = 1;  // the conv reading the resize's input does its work
  for (size_t ni = 0; ni < nodes_.size(); ++ni)  // in its lead's launch (grouped: emitNode decides)
    if (sib_lead_[ni] >= 0 && sib_lead_[ni] != (int)ni && !sib_grouped_[sib_lead_[ni]]) P.covered[ni] = 1;
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    P.begin[ni] = P.L.size();
    if (!skip_[ni] && !P.covered[ni]) emitNode(ni, batch, P.L, P.covered);
    P.end[ni] = P.L.size();
  }
  for (size_t ni = 0; ni < nodes_.size(); ++ni)
    for (size_t i = P.begin[ni]; i < P.end[ni]; ++i) {
      try {
        validate(P.L[i]);
      } catch (const std::exception & e) {
        throw std::runtime_error("node " + nodes_[ni].op + " -> " + nodes_[ni].outs[0] + ": " + e.what());
      }
    }
  return launch_cache_[batch] = std::move(P);
}

// Host-side bounds check of one launch: every element a kernel may touch (including the
// 16-byte vector over-reads of the channels-last paths) must lie inside one allocation.
void Model::validate(const Launch & l) const
{
  auto check = [&](const void * ptr, long first, long last, int elem, const char * what) {
    if (!ptr) throw std::runtime_error(std::string("null operand ") + what);
    if (last < first) return;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(ptr) + first * elem;
    const uintptr_t hi = reinterpret_cast<uintptr_t>(ptr) + (last + 1) * elem;
    for (const auto & a : allocs_)
      if (lo >= a.first && hi <= a.first + a.second) return;
    throw std::runtime_error(std::string("launch would access outside its buffers: ") + what);
  };
  // last element of a view covering B images x C channels x HW pixels
  auto vlast = [](const View & v, int B, long C, long HW) -> long {
    if (C <= 0 || HW <= 0 || B <= 0) return -1;
    return (long)(B - 1) * v.img + (v.layout == kNHWC ? (HW - 1) * v.cs + (C - 1) : (C - 1) * v.cs + (HW - 1));
  };
  if (l.kind == Launch::kAttn) {
    const AttnParams & a = l.ap;
    if (a.batch < 1 || a.batch > 65535 || a.heads < 1 || a.heads > 65535 || a.n < 8 || a.n % 8 || a.n > kAttnMaxN ||
        attn_key_blocks(a.n) == 0)
      throw std::runtime_error("attention geometry");
    if (a.q.cs != kAttnKD * a.n || a.k.cs != kAttnKD * a.n || a.v.cs != kAttnHD * a.n || a.y.cs != kAttnHD * a.n)
      throw std::runtime_error("attention head strides");
    const long qk = (long)a.heads * kAttnKD * a.n, vy = (long)a.heads * kAttnHD * a.n;
    check(a.q.ptr, 0, (long)(a.batch - 1) * a.q.img + qk - 1, 2, "attention q");
    check(a.k.ptr, 0, (long)(a.batch - 1) * a.k.img + qk - 1, 2, "attention k");
    check(a.v.ptr, 0, (long)(a.batch - 1) * a.v.img + vy - 1, 2, "attention v");
    check(a.y.ptr, 0, (long)(a.batch - 1) * a.y.img + vy - 1, 2, "attention y");
    return;
  }
  if (l.kind == Launch::kDecode) {
    const DecodeParams & d = l.dp;
    if (d.batch < 1 || d.batch > 65535 || d.nscale < 1 || d.nscale > 4) throw std::runtime_error("decode grid");
    const int nkc = 3 * d.nk, ny = 4 + d.nc + nkc;
    for (int s = 0; s < d.nscale; ++s) {
      const long hw = (s + 1 < d.nscale ? d.off[s + 1] : d.A) - d.off[s];
      if (hw < 1) throw std::runtime_error("decode scale offsets");
      check(d.x[s].ptr, 0, vlast(d.x[s], d.batch, 4 * d.R, hw), 2, "decode head");
      check(d.c[s].ptr, 0, vlast(d.c[s], d.batch, d.nc, hw), 2, "decode classes");
      if (d.nk) check(d.k[s].ptr, 0, vlast(d.k[s], d.batch, nkc, hw), 2, "decode keypoints");
    }
    check(d.dflw, 0, d.R - 1, 2, "decode bin weights");
    check(d.anc, 0, 2L * d.A - 1, 2, "decode anchors");
    check(d.st, 0, d.A - 1, 2, "decode strides");
    check(d.cbox, 0, 0, 2, "decode box constant");
    if (d.nk) {
      check(d.ancm, 0, 2L * d.A - 1, 2, "decode keypoint anchors");
      check(d.ckpt, 0, 0, 2, "decode keypoint constant");
    }
    if (d.y.layout != kNCHW || d.y.cs != d.A) throw std::runtime_error("decode output layout");
    check(d.y.ptr, 0, vlast(d.y, d.batch, ny, d.A), 2, "decode y");
    return;
  }
  if (l.kind == Launch::kPair) {
    const ConvParams & a = l.cp2;
    const ConvParams & p = l.cp;
    const long HW = (long)p.H * p.W;
    if (p.batch < 1 || p.batch > 65535 || a.batch != p.batch) throw std::runtime_error("batch out of grid range");
    const int C = a.Cin;
    if (!pair_channels_ok(C, a.Cout) || p.Cin != a.Cout || p.Cout != C || a.K != 3 || p.K != 3 || a.S != 1 ||
        p.S != 1 || a.P != 1 || p.P != 1 || a.H != p.H || a.W != p.W || p.Ho != p.H || p.Wo != p.W ||
        a.kpad != halo_taps(C) * C || p.kpad != halo_taps(C) * C)
      throw std::runtime_error("conv pair geometry");
    if (!pair_tile_ok(C, p.th, p.tw) || p.th + 4 > p.H + 1 || (long)p.batch * (p.H + 1) >= (1L << 22))
      throw std::runtime_error("conv pair tile");
    for (const View * v : {&a.x, &p.y})
      if (v->layout != kNHWC || v->cs % 8 || v->img % 8 || (reinterpret_cast<uintptr_t>(v->ptr) % 16))
        throw std::runtime_error("conv pair views");
    if (p.r.ptr && p.r.ptr != a.x.ptr) throw std::runtime_error("conv pair residual is not the pair's input");
    check(a.x.ptr, 0, vlast(a.x, p.batch, C, HW), 2, "conv pair x");
    check(p.y.ptr, 0, vlast(p.y, p.batch, C, HW), 2, "conv pair y");
    check(a.w, 0, (long)C * a.kpad - 1, 2, "conv pair first weights");
    check(p.w, 0, (long)C * p.kpad - 1, 2, "conv pair second weights");
    if (a.bias) check(a.bias, 0, C - 1, 4, "conv pair first bias");
    if (p.bias) check(p.bias, 0, C - 1, 4, "conv pair second bias");
    return;
  }
  if (l.kind != Launch::kSmall) {
    const ConvParams & p = l.cp;
    const long HW = (long)p.H * p.W, HWo = (long)p.Ho * p.Wo;
    if (p.batch < 1 || p.batch > 65535) throw std::runtime_error("batch out of grid range");
    if (p.cu && l.kind != Launch::kIgemm) throw std::runtime_error("upsample-concat input outside the implicit GEMM");
    // the resident-weight, pipelined and persistent stride-2 kernels write 4- or 8-channel
    // groups into the view's padding channels
    check(p.y.ptr, 0, vlast(p.y, p.batch, p.Cout + (p.res || p.pipe || p.wide || p.s2 > 2 || p.pw == 1 ? (res_store_width(p) - p.Cout % res_store_width(p)) % res_store_width(p) : 0), HWo), 2,
          "conv y");
    if (p.r.ptr) check(p.r.ptr, 0, vlast(p.r, p.batch, p.Cout, HWo), 2, "conv residual");
    // the MFMA epilogues read the zero-padded bias of round_up(Cout, 128) channels
    if (p.bias) check(p.bias, 0, (l.kind == Launch::kIgemm ? (p.Cout + 127) / 128 * 128 : p.Cout) - 1, 4, "conv bias");
    if (l.kind == Launch::kIgemm) {
      if (p.xt) {
        if (p.x.layout != kNCHW || p.K != 1 || p.S != 1 || p.P != 0 || p.halo || p.res || p.s2 || p.pipe || p.x.cs != HW ||
            HW % 8 || p.x.img % 8 || (p.pw && p.pw != 2))
          throw std::runtime_error("igemm planar input geometry");
        check(p.x.ptr, 0, vlast(p.x, p.batch, p.Cin, HW), 2, "igemm planar x");
      } else {
        if (p.x.layout != kNHWC) throw std::runtime_error("igemm needs channels-last input");
        check(p.x.ptr, 0, vlast(p.x, p.batch, p.cin8, HW), 2, "igemm x");
      }
      if (p.cu) {
        if (!upcat_ok(p)) throw std::runtime_error("igemm upsample-concat geometry");
        check(p.xu.ptr, 0, vlast(p.xu, p.batch, p.cu, HW / 4), 2, "igemm upsample source");
      }
      const long rows = (long)(p.Cout + igemm_bn(p.Cout) - 1) / igemm_bn(p.Cout) * igemm_bn(p.Cout);
      check(p.w, 0, rows * p.kpad - 1, 2, "igemm w");
      if (p.halo) {
        const int cfg = p.halo - 1, ck = p.ck;
        if (cfg < 0 || cfg >= kHaloCfgs || ck != halo_cfg_ck(cfg, p.Cin)) throw std::runtime_error("halo chunk size");
        if (p.K != 3 || p.S != 1 || p.P != 1 || p.ksplit != 1 || cfg >= kHaloCfgs || p.th < 1 || p.tw < 1 ||
            p.Ho != p.H || p.Wo != p.W || (p.th + 2) * (p.tw + 2) > halo_pmax(cfg) || p.th + 2 > kHaloMaxRows ||
            p.th * p.tw > (cfg < 4 ? 256 : cfg < 8 ? 128 : 64) || (p.Cout + halo_bn(cfg) - 1) / halo_bn(cfg) * halo_bn(cfg) > rows)
          throw std::runtime_error("halo geometry");
        if (p.kpad != (p.Cin + ck - 1) / ck * halo_taps(ck) * ck) throw std::runtime_error("halo weight packing");
        if ((long)p.batch * (p.H + 1) >= (1L << 22) || p.W >= (1 << 22)) throw std::runtime_error("halo geometry too large");
      }
      if (p.res) {
        const int cfg = p.res - 1, ck = p.ck;
        if (cfg < 0 || cfg > 3 || p.halo || p.s2 || ck != res_ck(p.Cin) || p.Cin > ck || p.K != 3 || p.S != 1 ||
            p.P != 1 || p.ksplit != 1 || p.th < 1 || p.tw < 1 || p.Ho != p.H || p.Wo != p.W ||
            p.th * p.tw > res_bm(cfg) || (p.th + 2) * (p.tw + 2) > res_pmax(cfg) || p.th + 2 > p.H + 1 ||
            p.th + 2 > kResMaxRows ||
            (cfg == 0 || cfg == 3) != (p.Cout > 32) || (cfg == 2) != (p.Cout <= 32 && ck == 64) ||
            (cfg == 3 && (ck != 64 || p.Cin % 8 || p.Cin != p.cin8)) || !res_views_ok(p))
          throw std::runtime_error("resident-weight conv geometry");
        if (p.kpad != halo_taps(ck) * ck) throw std::runtime_error("resident-weight packing");
        if ((long)p.batch * (p.H + 1) >= (1L << 22) || p.W >= (1 << 22)) throw std::runtime_error("resident-weight geometry too large");
        const long bn = res_bn(cfg), nrows = (p.Cout + bn - 1) / bn * bn;
        check(p.w, 0, nrows * p.kpad - 1, 2, "resident-weight w");
        if (p.xg) {  // grouped: block y reads input channels 64 y .. 64 y + 63
          if (cfg != 3 || p.xg != 64 || p.Cin != 64 || p.cin8 != 64) throw std::runtime_error("grouped conv geometry");
          check(p.x.ptr, 0, vlast(p.x, p.batch, (long)p.xg * (nrows / bn - 1) + p.cin8, HW), 2, "grouped conv x");
        }
        if (res_grid_x(p, cfg) < 1 || res_grid_x(p, cfg) > 65535) throw std::runtime_error("resident-weight grid");
      }
      if (p.pipe) {
        const int cfg = p.pipe - 1;
        if (cfg < 0 || cfg > 1 || p.halo || p.res || p.s2 || p.ck != 32 || p.K != 3 || p.S != 1 || p.P != 1 ||
            p.ksplit != 1 || p.th < 1 || p.tw < 1 || p.Ho != p.H || p.Wo != p.W || p.th * p.tw > 256 ||
            p.th + 2 > p.H + 1 || p.Cout > 256 || (cfg == 0) != (p.Cout > 64) || !pipe_views_ok(p) ||
            (long)(p.th + 2) * (5 * p.tw + 16) > (cfg == 0 ? 1728 : 2112))
          throw std::runtime_error("pipelined conv geometry");
        if (p.kpad != (p.Cin + 31) / 32 * 9 * 32) throw std::runtime_error("pipelined conv packing");
        if ((long)p.batch * (p.H + 1) >= (1L << 22) || p.W >= (1 << 14)) throw std::runtime_error("pipelined conv geometry too large");
        check(p.w, 0, (long)(p.Cout + 127) / 128 * 128 * p.kpad - 1, 2, "pipelined conv w");
      }
      if (p.wide) {
        const long nslot = ((long)p.batch * (p.H + 1) - 1) * p.W;
        const int bn = 128, pb = p.th;
        if (p.wide != 1 || p.halo || p.res || p.pipe || p.s2 || p.pw || p.ck != 16 || p.K != 3 || p.S != 1 ||
            p.P != 1 || p.ksplit != 1 || !wide_tm_ok(p.th) || p.tw < 1 || p.Ho != p.H || p.Wo != p.W ||
            p.Cin < 128 || p.Cin % 32 || p.Cout <= 64 || p.Cout > 256 || !pipe_views_ok(p) || p.act != kActSiLU ||
            nslot >= (1L << 22) - 64 || p.W >= (1 << 14) || p.tw > (nslot + 31) / 32 ||
            (long)p.tw * ((p.Cout + bn - 1) / bn) > 65535 ||
            (long)((p.W - 1 + 32 * pb - 1) / p.W + 3) * (3 * p.W + 16) > 2048)
          throw std::runtime_error("wide-layer conv geometry");
        if (p.kpad != 9 * p.Cin) throw std::runtime_error("wide-layer conv packing");
        check(p.w, 0, (long)(p.Cout + bn - 1) / bn * bn * p.kpad - 1, 2, "wide-layer conv w");
      }
      if (p.pw == 2) {
        if (p.ksplit != 1 || p.halo || p.res || p.pipe || p.wide || p.s2 || !pwt_plan(p) || pwt_lds_bytes(p) > 65536)
          throw std::runtime_error("planar pointwise streaming geometry");
        check(p.w, 0, (long)(p.Cout - 1) * p.kpad + p.cin8 - 1, 2, "planar pointwise w");
        if (!p.xt) check(p.x.ptr, 0, vlast(p.x, p.batch, p.cin8, HW), 2, "planar pointwise x");
      } else if (p.pw) {
        if (p.K != 1 || p.S != 1 || p.P != 0 || p.G != 1 || p.H != p.Ho || p.W != p.Wo || p.Cout > 128 || p.Cout < 1 ||
            p.cin8 > 512 || p.kpad < p.cin8 || p.ksplit != 1 || p.halo || p.res || p.pipe || p.s2 || p.xt ||
            !pw_views_ok(p) || pw_lds_bytes(p) > 65536 ||
            (p.act != kActNone && p.act != kActSiLU && p.act != kActReLU && p.act != kActHSwish))
          throw std::runtime_error("pointwise streaming geometry");
        check(p.w, 0, (long)(p.Cout - 1) * p.kpad + p.cin8 - 1, 2, "pointwise w");
      }
      if (p.s2 > 2) {
        const int cfg = p.s2 - 1, ck = s2pk_ck(cfg), cb = s2pk_cb(cfg);
        if (cfg > 6 || p.halo || p.res || p.pipe || p.K != 3 || p.S != 2 || p.P != 1 || p.ksplit != 1 ||
            p.cin8 != ck || p.Cin > ck || p.Cout > (cfg == 6 ? 128 : 32 * cb) || p.th != s2pk_th(cfg) ||
            p.tw != 16 || p.kpad < 9 * ck ||
            p.Ho != (p.H - 1) / 2 + 1 || p.Wo != (p.W - 1) / 2 + 1 || !s2pk_views_ok(p) ||
            (p.act != kActNone && p.act != kActSiLU && p.act != kActReLU && p.act != kActHSwish))
          throw std::runtime_error("persistent stride-2 geometry");
        check(p.w, 0, (long)(p.Cout + 32 * cb - 1) / (32 * cb) * 32 * cb * p.kpad - 1, 2, "persistent stride-2 w");
      } else if (p.s2) {
        const int cfg = p.s2 - 1;
        if (cfg < 0 || cfg > 1 || p.halo || p.K != 3 || p.S != 2 || p.P != 1 || p.ksplit != 1 ||
            p.cin8 != s2_cfg_ck(cfg) || p.Cout > s2_cfg_bn(cfg) || p.th < 1 || p.tw < 1 ||
            p.th * p.tw > s2_cfg_bm(cfg) || s2_patch(p.th, p.tw) > s2_cfg_pmax(cfg) ||
            p.Ho != (p.H - 1) / 2 + 1 || p.Wo != (p.W - 1) / 2 + 1 || p.kpad < 9 * p.cin8)
          throw std::runtime_error("stride-2 patch geometry");
      }
      if (p.ksplit > 1) {
        const long M = (long)p.batch * HWo;
        if ((size_t)p.ksplit * rows * M > ws_floats_) throw std::runtime_error("split-K workspace too small");
        check(p.ws, 0, (long)p.ksplit * rows * M - 1, 4, "igemm split-K workspace");
      }
      if (p.kpad % kIgemmBK && !p.res) throw std::runtime_error("kpad not a multiple of the K tile");
      if (!p.halo && !p.res && !p.pipe && !p.wide && (p.bk != 32 && p.bk != 64)) throw std::runtime_error("kpad not a multiple of the K tile");
      if (!p.halo && !p.res && !p.pipe && !p.wide && p.kpad % p.bk) throw std::runtime_error("kpad not a multiple of the K step");
    } else if (l.kind == Launch::kDirect && p.stem_mfma) {
      check(p.x.ptr, 0, vlast(p.x, p.batch, p.Cin, HW), 2, "stem x");
      check(p.w, 0, (long)(p.Cout + 15) / 16 * 16 * 32 - 1, 2, "stem w");
      if (p.Cin * 9 > 32 || p.Cout > 32) throw std::runtime_error("stem geometry");
      if (stem_rows_supported(p)) {
        check(p.w2, 0, 16 * 64 - 1, 2, "stem rows w");
        // each staged row reads W pixels of every channel plane; outputs cover Ho x Wo x Cout
        check(p.x.ptr, 0, vlast(p.x, p.batch, p.Cin, HW), 2, "stem rows x");
      }
    } else if (l.kind == Launch::kDirect) {
      check(p.x.ptr, 0, vlast(p.x, p.batch, p.Cin, HW), 2, "direct x");
      check(p.w, 0, (long)p.Cin * p.K * p.K * (p.Cout / p.G) + 16 - 1, 4, "direct w");
    } else {
      check(p.x.ptr, 0, vlast(p.x, p.batch, p.Cin, HW), 2, "dw x");
      check(p.w, 0, (long)p.K * p.K * p.Cin - 1, 4, "dw w");
      check(p.w2, 0, (long)p.K * p.K * p.Cin - 1, 2, "dw w16");
    }
    return;
  }
  const SmallParams & q = l.sp;
  const int B = q.batch;
  if (B < 1 || B > 65535) throw std::runtime_error("batch out of grid range");
  const long HW = (long)q.H * q.W;
  auto flat = [&](const View & v, long n, const char * what) { check(v.ptr, 0, (long)(B - 1) * v.img + n - 1, 2, what); };
  switch (l.small) {
  case kEwSame:
    check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "ew a");
    if (q.b.img == 0 && q.b.cs == 0) check(q.b.ptr, 0, 0, 2, "ew scalar b");
    else check(q.b.ptr, 0, vlast(q.b, B, q.C, HW), 2, "ew b");
    check(q.y.ptr, 0, vlast(q.y, B, q.C, HW), 2, "ew y");
    break;
  case kEwUnary:
  case kCopy:
    check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "a");
    check(q.y.ptr, 0, vlast(q.y, B, q.C, HW), 2, "y");
    break;
  case kEwChan:
    if (q.i0) { flat(q.a, q.C, "chan a"); check(q.b.ptr, 0, vlast(q.b, B, q.C, HW), 2, "chan b"); }
    else { check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "chan a"); flat(q.b, q.C, "chan b"); }
    check(q.y.ptr, 0, vlast(q.y, B, q.C, HW), 2, "chan y");
    break;
  case kEwBcast: {
    long amax = 0, bmax = 0;
    for (int r = 0; r < q.rank; ++r) {
      amax += (long)(q.dims[r] - 1) * q.dims[q.rank + r];
      bmax += (long)(q.dims[r] - 1) * q.dims[2 * q.rank + r];
    }
    flat(q.a, amax + 1, "bcast a");
    flat(q.b, bmax + 1, "bcast b");
    flat(q.y, q.n, "bcast y");
    break;
  }
  case kSliceAxis:
    flat(q.a, (long)q.i0 * q.i1 * q.i2, "slice x");
    flat(q.y, (long)q.i0 * q.i4 * q.i2, "slice y");
    break;
  case kConcatOuter:
    flat(q.a, (long)q.i0 * q.i1 * q.i2, "concat x");
    flat(q.y, (long)q.i0 * q.i3 * q.i2, "concat y");
    if (q.i4 + q.i1 > q.i3) throw std::runtime_error("concat offset beyond axis");
    break;
  case kMaxPool:
  case kResizeNN:
    check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "pool x");
    check(q.y.ptr, 0, vlast(q.y, B, q.C, (long)q.Ho * q.Wo), 2, "pool y");
    break;
  case kMaxPoolSppf:
    if (q.C % 8 || HW > 1024 || q.Ho != q.H || q.Wo != q.W) throw std::runtime_error("SPPF pool geometry");
    for (const View * v : {&q.a, &q.y, &q.b, &q.c})
      if (v->layout != kNHWC || v->cs % 8 || v->img % 8) throw std::runtime_error("SPPF pool views");
    check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "SPPF pool x");
    check(q.y.ptr, 0, vlast(q.y, B, q.C, HW), 2, "SPPF pool 5x5");
    check(q.b.ptr, 0, vlast(q.b, B, q.C, HW), 2, "SPPF pool 9x9");
    check(q.c.ptr, 0, vlast(q.c, B, q.C, HW), 2, "SPPF pool 13x13");
    break;
  case kSoftmax:
  case kPermute:
    flat(q.a, (long)q.i0 * q.i1 * q.i2, "x");
    flat(q.y, (long)q.i0 * q.i1 * q.i2, "y");
    break;
  case kGap:
    check(q.a.ptr, 0, vlast(q.a, B, q.C, HW), 2, "gap x");
    flat(q.y, q.C, "gap y");
    break;
  case kBmm:
    if ((long)q.batch * q.i0 > 65535) throw std::runtime_error("bmm batch x heads exceeds the grid");
    flat(q.a, (long)q.i0 * q.i1 * q.i2, "bmm a");
    flat(q.b, (long)q.i0 * q.i2 * q.i3, "bmm b");
    flat(q.y, (long)q.i0 * q.i1 * q.i3, "bmm y");
    break;
  case kBiasAdd:
    flat(q.a, q.n, "bias x");
    check(q.b.ptr, 0, (q.n - 1) / q.i0, 2, "bias b");
    flat(q.y, q.n, "bias y");
    break;
  default:
    throw std::runtime_error("unknown small op");
  }
}

void Model::dryRun(int batch)
{
  check_batch(batch, max_batch_);
  (void)launches(batch);
  last_batch_ = batch;
}

void Model::enqueue(const std::vector<Launch> & L, size_t b, size_t e)
{
  for (size_t i = b; i < e; ++i) {
    const Launch & l = L[i];
    switch (l.kind) {
    case Launch::kIgemm: launch_conv_igemm(l.cp, stream_); break;
    case Launch::kDirect: launch_conv_direct(l.cp, stream_); break;
    case Launch::kDw: launch_dwconv(l.cp, stream_); break;
    case Launch::kDecode: launch_pose_decode(l.dp, stream_); break;
    case Launch::kAttn: launch_attention(l.ap, stream_); break;
    case Launch::kPair: launch_conv_pair(l.cp2, l.cp, stream_); break;
    default: launch_small(l.small, l.sp, stream_); break;
    }
  }
  HIPCHECK(hipGetLastError());
}

// ==================================================================== running

size_t Model::inputNumel() const { return (size_t)prod(input_dims_); }
const std::vector<int64_t> & Model::outputDims(int i) const { return T_.at(outputs_.at(i))->dims; }
size_t Model::outputNumel(int i) const { return (size_t)T_.at(outputs_.at(i))->numel; }


void Model::setInputF16(const uint16_t * host, int batch)
{
  check_batch(batch, max_batch_);
  HIPCHECK(hipSetDevice(device_));
  const long n = (long)inputNumel();
  const long img = roots_[T_[input_name_]->root]->per_image;
  HIPCHECK(hipMemcpy2DAsync(input_buf_, img * 2, host, n * 2, n * 2, batch, hipMemcpyHostToDevice, stream_));
  HIPCHECK(hipStreamSynchronize(stream_));
}

void Model::setInputDeviceF16(const void * dev, int batch)
{
  check_batch(batch, max_batch_);
  HIPCHECK(hipSetDevice(device_));
  const long n = (long)inputNumel();
  const long img = roots_[T_[input_name_]->root]->per_image;
  HIPCHECK(hipMemcpy2DAsync(input_buf_, img * 2, dev, n * 2, n * 2, batch, hipMemcpyDeviceToDevice, stream_));
}

void Model::setInputF32Trunc(const float * host, int batch)
{
  check_batch(batch, max_batch_);
  HIPCHECK(hipSetDevice(device_));
  const long n = (long)inputNumel();
  const long img = roots_[T_[input_name_]->root]->per_image;
  if (!stage_f32_) stage_f32_ = devAlloc((size_t)n * max_batch_ * 4, false);
  HIPCHECK(hipMemcpyAsync(stage_f32_, host, (size_t)n * batch * 4, hipMemcpyHostToDevice, stream_));
  for (int b = 0; b < batch; ++b)
    launch_f32_to_f16_trunc(static_cast<const float *>(stage_f32_) + (long)b * n,
                            static_cast<__half *>(input_buf_) + (long)b * img, n, stream_);
  HIPCHECK(hipGetLastError());
  HIPCHECK(hipStreamSynchronize(stream_));
}

// The f32 input passes through the GPU's fixed 8 MiB scratch array in chunks: each chunk is
// copied in and converted before the next copy overwrites the array (one stream orders the
// copy after the previous chunk's kernel), so any batch fits and nothing is allocated.  Every
// model on the GPU shares the array, so the call holds the device's scratch lock from the
// first copy until its stream has drained (also when a HIP call fails midway): calls from
// models on one device, in any threads, run one after the other.
void Model::setInputF32TruncNoAlloc(const float * host, int batch)
{
  check_batch(batch, max_batch_);
  if (dry_) throw std::runtime_error("dry-run model has no device");
  HIPCHECK(hipSetDevice(device_));
  float * sc = boundary_scratch(device_);
  const long n = (long)inputNumel();
  const long img = roots_[T_[input_name_]->root]->per_image;
  std::lock_guard<std::mutex> lock(boundary_scratch_lock(device_));
  try {
    for (int b = 0; b < batch; ++b)
      for (long off = 0; off < n; off += kBoundaryScratchFloats) {
        const long len = std::min(n - off, kBoundaryScratchFloats);
        HIPCHECK(hipMemcpyAsync(sc, host + (long)b * n + off, (size_t)len * 4, hipMemcpyHostToDevice, stream_));
        launch_f32_to_f16_trunc(sc, static_cast<__half *>(input_buf_) + (long)b * img + off, len, stream_);
      }
    HIPCHECK(hipGetLastError());
    HIPCHECK(hipStreamSynchronize(stream_));
  } catch (...) {
    (void)hipStreamSynchronize(stream_);  // nothing of this call may still use the array
    throw;
  }
}

void Model::run(int batch)
{
  check_batch(batch, max_batch_);
  if (dry_) { dryRun(batch); return; }
  HIPCHECK(hipSetDevice(device_));
  const auto t0 = std::chrono::steady_clock::now();
  const LaunchPlan & P = launches(batch);
  last_batch_ = batch;
  const auto & L = P.L;
  if (flags_ & IVH_FLAG_PROFILE) {
    runProfiled(P);
  } else if (flags_ & IVH_FLAG_NO_GRAPH) {
    enqueue(L, 0, L.size());
  } else {
    auto it = graphs_.find(batch);
    if (it == graphs_.end()) {
      hipGraph_t g = nullptr;
      HIPCHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
      try {
        enqueue(L, 0, L.size());
      } catch (...) {
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HIPCHECK(hipStreamEndCapture(stream_, &g));
      hipGraphExec_t ge = nullptr;
      HIPCHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
      HIPCHECK(hipGraphDestroy(g));
      it = graphs_.emplace(batch, ge).first;
    }
    HIPCHECK(hipGraphLaunch(it->second, stream_));
  }
  if (!(flags_ & IVH_FLAG_ASYNC) || (flags_ & IVH_FLAG_PROFILE)) {
    HIPCHECK(hipStreamSynchronize(stream_));
    last_run_ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }
  if (flags_ & IVH_FLAG_PROFILE) {
    // the run is complete: add each node's time between its two events
    for (size_t ni = 0; ni < nodes_.size(); ++ni) {
      if (P.begin[ni] == P.end[ni]) continue;
      float t = 0;
      HIPCHECK(hipEventElapsedTime(&t, prof_ev_[ni], prof_ev_[ni + 1]));
      prof_ms_[ni] += t;
      prof_calls_[ni] += 1;
    }
  }
}

// One run node by node, a HIP event recorded before the first node and after every node
// (the reference's profiling runs time every kernel with its own event,
// src/PlanModel.cpp:3166-3205).
void Model::runProfiled(const LaunchPlan & P)
{
  if (prof_ev_.empty()) {
    prof_ev_.assign(nodes_.size() + 1, nullptr);
    for (auto & e : prof_ev_) HIPCHECK(hipEventCreate(&e));
    prof_ms_.assign(nodes_.size(), 0.0);
    prof_calls_.assign(nodes_.size(), 0);
  }
  HIPCHECK(hipEventRecord(prof_ev_[0], stream_));
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    enqueue(P.L, P.begin[ni], P.end[ni]);
    HIPCHECK(hipEventRecord(prof_ev_[ni + 1], stream_));
  }
}

void Model::nodeTimes(std::vector<double> & ms, std::vector<int> & calls) const
{
  ms = prof_ms_;
  calls = prof_calls_;
  ms.resize(nodes_.size(), 0.0);
  calls.resize(nodes_.size(), 0);
}

void Model::clearProfile()
{
  std::fill(prof_ms_.begin(), prof_ms_.end(), 0.0);
  std::fill(prof_calls_.begin(), prof_calls_.end(), 0);
}

void Model::sync()
{
  HIPCHECK(hipSetDevice(device_));
  HIPCHECK(hipStreamSynchronize(stream_));
}

void Model::readOutputF16(int i, uint16_t * host, int batch)
{
  check_batch(batch, max_batch_);
  if (i < 0 || i >= outputCount()) throw std::runtime_error("output index out of range");
  HIPCHECK(hipSetDevice(device_));
  const Tensor & t = *T_[outputs_[i]];
  const View v = view(t.name, batch);
  if (v.layout != kNCHW) throw std::runtime_error("output stored channels-last");
  HIPCHECK(hipMemcpy2DAsync(host, t.numel * 2, v.ptr, v.img * 2, t.numel * 2, batch, hipMemcpyDeviceToHost, stream_));
  HIPCHECK(hipStreamSynchronize(stream_));
}

void Model::readOutputF32(int i, float * host, int batch)
{
  const long n = (long)outputNumel(i);
  std::vector<uint16_t> h((size_t)n * batch);
  readOutputF16(i, h.data(), batch);
  for (size_t k = 0; k < h.size(); ++k) host[k] = h2f(h[k]);
}

size_t Model::tensorNumel(const std::string & name) const
{
  auto it = T_.find(name);
  return it == T_.end() ? 0 : (size_t)it->second->numel;
}

bool Model::readTensorF16(const std::string & name, uint16_t * host, int batch)
{
  auto it = T_.find(name);
  if (it == T_.end()) return false;
  check_batch(batch, max_batch_);
  if (it->second->producer >= 0 && nodes_[it->second->producer].op == "resize_nn" && skip_[it->second->producer])
    throw std::runtime_error("tensor " + name + " is not materialised: its upsample is fused into the 1x1 conv reading it "
                             "(IVH_FLAG_NO_FUSE_UPSAMPLE or IVH_FLAG_NO_REUSE keeps it)");
  HIPCHECK(hipSetDevice(device_));
  HIPCHECK(hipStreamSynchronize(stream_));
  const Tensor & t = *it->second;
  const View v = view(name, batch);
  const long img = std::max<long>(v.img, 0);
  // pull the whole root span of each image, then gather NCHW on the host
  const long span = t.kind == Tensor::kInit ? t.numel : roots_[t.root]->per_image;
  const __half * base = v.ptr;
  long lo = 0;
  if (t.kind != Tensor::kInit) {
    const Root & r = *roots_[t.root];
    lo = r.layout == kNHWC ? t.coff : t.eoff;
  }
  std::vector<uint16_t> buf((size_t)span);
  const long HW = (long)t.H * t.W;
  for (int b = 0; b < batch; ++b) {
    HIPCHECK(hipMemcpy(buf.data(), base - lo + (long)b * img, span * 2, hipMemcpyDeviceToHost));
    uint16_t * dst = host + (long)b * t.numel;
    if (v.layout == kNHWC) {
      for (int c = 0; c < t.C; ++c)
        for (long p = 0; p < HW; ++p) dst[c * HW + p] = buf[(size_t)(lo + p * v.cs + c)];
    } else {
      std::memcpy(dst, buf.data() + lo, (size_t)t.numel * 2);
    }
  }
  return true;
}

std::vector<double> Model::profileNodes(int batch, int iters)
{
  check_batch(batch, max_batch_);
  HIPCHECK(hipSetDevice(device_));
  const LaunchPlan & P = launches(batch);
  last_batch_ = batch;
  const auto & L = P.L;
  iters = std::max(iters, 1);
  std::vector<double> ms(nodes_.size(), 0.0);
  std::vector<hipEvent_t> ev(2 * nodes_.size());
  for (auto & e : ev) HIPCHECK(hipEventCreate(&e));
  // each node `iters` times back to back (launches queue up behind each other, so host
  // launch gaps do not count).  A node may then read arena memory that a later node has
  // reused (addresses never depend on data, so only values change); a final full pass
  // restores every tensor.
  enqueue(L, 0, L.size());
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    HIPCHECK(hipEventRecord(ev[2 * ni], stream_));
    for (int it = 0; it < iters; ++it) enqueue(L, P.begin[ni], P.end[ni]);
    HIPCHECK(hipEventRecord(ev[2 * ni + 1], stream_));
  }
  enqueue(L, 0, L.size());
  HIPCHECK(hipStreamSynchronize(stream_));
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    float t = 0;
    HIPCHECK(hipEventElapsedTime(&t, ev[2 * ni], ev[2 * ni + 1]));
    ms[ni] = P.begin[ni] == P.end[ni] ? 0.0 : t / iters;
  }
  for (auto & e : ev) (void)hipEventDestroy(e);
  return ms;
}

std::string Model::nodeTag(int i)
{
  std::string k = nodeKernel(i);
  const LaunchPlan & P = launches(labelBatch());
  if (P.begin.at(i) == P.end.at(i)) return k;
  const Launch & l = P.L[P.begin[i]];
  if (l.kind == Launch::kIgemm)
    return k + " " + igemm_launch_tag(l.cp) +
           (sib_.at(i).empty() || (sib_grouped_[i] && !l.cp.xg)
                ? ""
                : (sib_grouped_[i] ? " groups=" : " siblings=") + std::to_string(sib_[i].size()) + " cout=" + std::to_string(l.cp.Cout));
  if (l.kind == Launch::kDw) return k + " " + dw_launch_tag(l.cp);
  if (l.kind == Launch::kPair)
    return k + " th=" + std::to_string(l.cp.th) + " tw=" + std::to_string(l.cp.tw) + " tiles=" +
           std::to_string(pair_tiles(l.cp.H, l.cp.W, l.cp.batch, l.cp.th, l.cp.tw)) + (l.cp.r.ptr ? " +res" : "");
  return k;
}

std::string Model::nodeKernel(int i)
{
  const NodeStat & s = stats_.at(i);
  const LaunchPlan & P = launches(labelBatch());
  if (P.begin.at(i) == P.end.at(i)) return P.covered.at(i) ? "(fused)" : "(view)";
  const Launch & l = P.L[P.begin[i]];
  switch (l.kind) {
  case Launch::kIgemm:
    return l.cp.wide ? "conv_wide" : l.cp.pipe ? "conv_pipe" : l.cp.res ? "conv_res" : l.cp.halo ? "conv_halo" : (l.cp.pw == 2 ? "conv_pw_planar" : l.cp.pw ? "conv_pw" : l.cp.s2 ? (l.cp.s2 > 2 ? "conv_s2p" : "conv_s2") : (l.cp.ksplit > 1 ? "conv_igemm_sk" : "conv_igemm"));
  case Launch::kDirect: return l.cp.stem_mfma ? "conv_stem" : "conv_direct";
  case Launch::kDw: return "dwconv";
  case Launch::kDecode: return "pose_decode";
  case Launch::kAttn: return "attention";
  case Launch::kPair: return "conv_pair";
  case Launch::kSmall:
    if (l.small == kMaxPoolSppf) return "maxpool_sppf";
    return s.kernel;
  default: return s.kernel;
  }
}

// ================================================================= statistics
// Algorithmic FLOPs / compulsory fp16 bytes per image, for roofline reports.
void Model::buildStats()
{
  stats_.assign(nodes_.size(), NodeStat{});
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    const PlanNode & n = nodes_[ni];
    NodeStat & s = stats_[ni];
    s.op = n.op;
    const Tensor & y = *T_[n.outs[0]];
    double in_b = 0;
    for (size_t k = 0; k < n.ins.size(); ++k) {
      if (n.ins[k] == "-") continue;
      const Tensor & t = *T_[n.ins[k]];
      if (t.kind == Tensor::kInit) continue;
      in_b += 2.0 * t.numel;
    }
    s.bytes = skip_[ni] ? 0 : in_b + 2.0 * y.numel;
    char buf[256];
    if (n.op == "conv1x1" || n.op == "conv3x3" || n.op == "conv_general") {
      const bool is1 = n.op == "conv1x1";
      const Tensor & wt = *T_[is1 ? n.ins[0] : n.ins[1]];
      const Tensor & xt = *T_[is1 ? n.ins[1] : n.ins[0]];
      s.flops = 2.0 * wt.numel * (double)y.numel / std::max<int64_t>(wt.dims[0], 1);
      const int kind = packed_[ni].pk.family;
      s.kernel = kind == 0 ? "conv_igemm" : (kind == 1 ? "conv_direct" : "dwconv");
      std::snprintf(buf, sizeof(buf), "%s %dx%dx%d->%dx%dx%d k%d s%d g%d act%d%s", n.op.c_str(), xt.C, xt.H, xt.W,
                    y.C, y.H, y.W, is1 ? 1 : (n.op == "conv3x3" ? 3 : n.i("K", 3)),
                    is1 ? 1 : (n.op == "conv3x3" ? n.i("stride", 1) : n.i("S", 1)), n.i("G", 1), n.i("act"),
                    (n.ins.size() > 3 && n.ins[3] != "-") ? " +res" : "");
      s.desc = buf;
    } else {
      s.kernel = skip_[ni] ? "(view)" : n.op;
      if (n.op == "bmm") {
        const Tensor & at = *T_[n.ins[0]];
        const Tensor & bt = *T_[n.ins[1]];
        s.flops = 2.0 * at.numel * (double)bt.dims.back();
      }
      if (n.op == "gemm" && T_[n.ins[0]]->dims.size() >= 2) {  // M K N, N = numel(B) / K
        const Tensor & at = *T_[n.ins[0]];
        const double M = (double)at.dims[0], K = (double)at.dims[1];
        s.flops = K > 0 ? 2.0 * M * K * (double)(T_[n.ins[1]]->numel / at.dims[1]) : 0.0;
      }
      if (n.op == "attention") {
        const double N = n.i("n"), h = n.i("heads");
        s.flops = h * (2.0 * N * N * kAttnKD + 2.0 * kAttnHD * N * N);
      }
      if (n.op == "pose_decode")
        std::snprintf(buf, sizeof(buf), "pose_decode %d scales, %d anchors, R %d, %d classes, %d keypoints -> %s",
                      n.i("S"), n.i("A"), n.i("R"), n.i("nc"), n.i("nk"), y.name.c_str());
      else
        std::snprintf(buf, sizeof(buf), "%s -> %s [%ld]", n.op.c_str(), y.name.c_str(), (long)y.numel);
      s.desc = buf;
    }
  }
  // fused launches: what the one launch computes and must move
  for (size_t ni = 0; ni < nodes_.size(); ++ni) {
    NodeStat & s = stats_[ni];
    if (up_src_[ni] >= 0) {  // the upsampled channels come from the resize's input, 4x smaller
      const Tensor & at = *T_[nodes_[up_src_[ni]].ins[0]];
      s.bytes -= 2.0 * 3 * at.numel;
    }
    if (sib_[ni].empty()) continue;
    // merged siblings: x once (grouped: each member's own input), every member's output; the
    // lead carries the whole launch
    int cout = 0;
    for (int j : sib_[ni]) {
      if (j != (int)ni) {
        NodeStat & m = stats_[j];
        s.flops += m.flops;
        s.bytes += 2.0 * T_[nodes_[j].outs[0]]->numel + (sib_grouped_[ni] ? 2.0 * T_[nodes_[j].ins[0]]->numel : 0.0);
        m.flops = m.bytes = 0;
      }
      cout += T_[nodes_[j].outs[0]]->C;
    }
    const auto arrow = s.desc.find("->"), x = s.desc.find('x', arrow);
    if (arrow != std::string::npos && x != std::string::npos)
      s.desc = s.desc.substr(0, arrow + 2) + std::to_string(cout) + s.desc.substr(x) + " (" +
               std::to_string(sib_[ni].size()) + (sib_grouped_[ni] ? " groups)" : " siblings)");
    if (sib_grouped_[ni]) {  // a grouped conv: 64 input channels per group
      const auto sp = s.desc.find(' '), xi = s.desc.find('x', sp), g1 = s.desc.find(" g1 ");
      if (sp != std::string::npos && xi != std::string::npos && g1 != std::string::npos)
        s.desc = s.desc.substr(0, sp + 1) + std::to_string(64 * sib_[ni].size()) + s.desc.substr(xi, g1 + 2 - xi) +
                 std::to_string(sib_[ni].size()) + s.desc.substr(g1 + 3);
    }
  }
}

}  // namespace ivh
