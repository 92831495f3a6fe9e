// HIP-native plan executor: the MI355X counterpart of infvino::PlanModel
// (include/infvino/PlanModel.hpp:57-234, src/PlanModel.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "conv_pack.hpp"
#include "ivh_internal.hpp"

namespace ivh {

struct PlanNode {
  std::string op;
  std::vector<std::string> ins, outs;
  std::map<std::string, std::string> attr;
  int i(const char * key, int def = 0) const;
  bool has(const char * key) const { return attr.count(key) != 0; }
  std::string str(const char * key) const;
};

// One kernel launch with everything resolved for a given batch size.
struct Launch {
  enum Kind { kIgemm, kDirect, kDw, kSmall, kDecode, kAttn, kPair } kind = kSmall;
  int small = 0;
  ConvParams cp;
  ConvParams cp2;  // kPair: the first conv of the pair (cp is the second)
  SmallParams sp;
  DecodeParams dp;
  AttnParams ap;
};

struct NodeStat {
  std::string op, kernel, desc;
  double flops = 0, bytes = 0;  // algorithmic, per image
};

class Model {
 public:
  Model(const std::string & plan_path, int device, int max_batch, uint32_t flags);
  ~Model();
  Model(const Model &) = delete;
  Model & operator=(const Model &) = delete;

  const std::vector<int64_t> & inputDims() const { return input_dims_; }
  size_t inputNumel() const;
  int outputCount() const { return (int)outputs_.size(); }
  const std::vector<int64_t> & outputDims(int i) const;
  size_t outputNumel(int i) const;
  int maxBatch() const { return max_batch_; }
  int device() const { return device_; }
  hipStream_t stream() const { return stream_; }

  void setInputF16(const uint16_t * host, int batch);
  void setInputF32Trunc(const float * host, int batch);
  // the same conversion staged through the GPU's fixed scratch array: allocates nothing
  void setInputF32TruncNoAlloc(const float * host, int batch);
  void setInputDeviceF16(const void * dev, int batch);
  void run(int batch);
  void sync();
  void readOutputF16(int i, uint16_t * host, int batch);
  void readOutputF32(int i, float * host, int batch);
  bool readTensorF16(const std::string & name, uint16_t * host, int batch);
  size_t tensorNumel(const std::string & name) const;
  double lastRunMs() const { return last_run_ms_; }
  // Builds and bounds-checks the launches for `batch` without touching a device.
  void dryRun(int batch);
  bool isDry() const { return dry_; }

  // Per-node device time (ms, averaged over iters) measured with HIP events on the
  // model's stream around each node's launches.
  std::vector<double> profileNodes(int batch, int iters);
  // Time and run count accumulated per node over the runs of a model created with
  // IVH_FLAG_PROFILE (each run launches node by node with HIP events between nodes).
  void nodeTimes(std::vector<double> & ms, std::vector<int> & calls) const;
  void clearProfile();
  int nodeCount() const { return (int)nodes_.size(); }
  const NodeStat & nodeStat(int i) const { return stats_.at(i); }
  // kernel family node i launches (conv_halo / conv_igemm / conv_stem ...) at the batch of the
  // last run, dry run or profileNodes call (the largest batch before the first): kernel and
  // tile choices depend on the batch
  std::string nodeKernel(int i);
  // nodeKernel plus the launch detail (tile config, K step, split, build) at the same batch
  std::string nodeTag(int i);
  int labelBatch() const { return last_batch_ > 0 ? last_batch_ : max_batch_; }
  size_t arenaBytes(int batch) const { return (size_t)arena_elems1_ * batch * 2; }
  size_t weightBytes() const { return weight_bytes_; }

 private:
  struct Tensor;
  struct Root;
  struct LaunchPlan;
  void parse(const std::string & path);
  void fuseDecode();
  void fuseResidual();
  void fuseActivation();
  void fusePermuteMatmul();
  void fuseAttention();
  void plan();
  int chanBroadcast(const PlanNode & n) const;
  void assignViews();
  void chooseLayouts();
  // 1x1 convs reading concat(resize_nn x2 (a), b...): up_src_[ni] = the resize node whose work
  // conv ni does by reading a directly (that resize emits nothing), else -1
  void fuseUpsample();
  std::vector<int> up_src_;
  void allocate();
  void uploadWeights();
  void buildStats();
  const LaunchPlan & launches(int batch);
  void runProfiled(const LaunchPlan & P);
  // throws when two roots whose closed live intervals intersect share arena bytes
  void verifyArena() const;
  View view(const std::string & name, int batch) const;
  void enqueue(const std::vector<Launch> & L, size_t b, size_t e);
  // `covered`: nodes whose work a launch of node ni already does (they emit nothing)
  void emitNode(size_t ni, int batch, std::vector<Launch> & out, std::vector<char> & covered);
  bool sppfChain(size_t ni) const;
  // C2f / C3k2 bottleneck pairs (conv_pair.hip): pair_next_[ni] = node of the second conv
  // when node ni is the first conv of a pair, else -1 (decided at load, before allocate)
  void findPairs();
  std::vector<int> pair_next_;
  // sibling 3x3 convs (the heads' cv2 / cv3 / cv4 first convs read the same x): one launch
  // with the output channels of all of them, whose outputs are channel views of one root.
  // sib_[lead] = the members in channel order (the lead is the first in node order), empty
  // otherwise; sib_lead_[ni] = the lead of node ni's group, or -1
  void findSiblings();
  std::vector<std::vector<int>> sib_;
  std::vector<int> sib_lead_;
  // grouped siblings: 3x3 convs 64 -> 64 whose inputs are consecutive 64-channel views of one
  // merged root (the branches' second convs) run as one grouped launch; sib_x_[lead] = the
  // tensor of the first group's input
  std::vector<char> sib_grouped_;
  std::vector<std::string> sib_x_;
  // the launch's output channels: the members' sum, or for a merge whose members but the last
  // are whole 64-channel blocks 64 per member (the last member's padding channels written as
  // act(0) = 0 by zero weight rows, so a grouped launch may read them as its last group)
  std::vector<int> sib_cout_;
  // the launch of a conv node (conv1x1 / conv3x3 / conv_general) at a batch size
  // grouped: a grouped-siblings lead's one launch for all its members (packed_grp_)
  Launch convLaunch(size_t ni, int batch, bool grouped = false);
  // node ni and its pair partner as one kPair launch; false when a view does not suit it
  bool pairLaunch(size_t ni, int batch, Launch & L);
  void validate(const Launch & l) const;
  void * devAlloc(size_t bytes, bool zero);
  void devUpload(void * d, const void * src, size_t bytes);

  std::string plan_path_, plan_dir_;
  int device_ = 0, max_batch_ = 1;
  uint32_t flags_ = 0;
  hipStream_t stream_ = nullptr;

  std::vector<PlanNode> nodes_;
  std::vector<char> skip_;                  // node needs no launch (pure alias)
  std::map<std::string, std::unique_ptr<Tensor>> T_;
  std::vector<std::unique_ptr<Root>> roots_;
  std::string input_name_;
  std::vector<int64_t> input_dims_;
  std::vector<std::string> outputs_;

  // device memory
  void * arena_ = nullptr;                  // activations, max_batch images
  long arena_elems1_ = 0;                   // elements per image-unit
  void * input_buf_ = nullptr;              // graph input, max_batch images (fp16)
  void * stage_f32_ = nullptr;              // f32 staging for the truncating conversion
  std::vector<void *> dev_allocs_;          // weights etc.
  size_t weight_bytes_ = 0;
  std::map<std::string, void *> init_dev_;  // raw fp16 inits
  struct Packed {
    ConvSpec spec;
    ConvPacking pk;
    void * dev = nullptr;  // device copy of the packed operand blob
  };
  std::vector<Packed> packed_;              // per node
  std::vector<Packed> packed_grp_;          // grouped-siblings leads: the members' weights together
  float * ws_ = nullptr;                    // split-K partials
  size_t ws_floats_ = 0;

  // The resolved launches of one batch size and, per node, its [begin, end) range in them.
  // Kept together per batch: launch counts can differ between batch sizes (a fusion that
  // needs 16-byte aligned views may hold at one batch and not at another).
  struct LaunchPlan {
    std::vector<Launch> L;
    std::vector<size_t> begin, end;
    std::vector<char> covered;              // node's work done by an earlier node's launch
  };
  std::map<int, LaunchPlan> launch_cache_;
  // accumulated per-node device time of IVH_FLAG_PROFILE runs (PlanModel::profile())
  std::vector<double> prof_ms_;
  std::vector<int> prof_calls_;
  std::vector<hipEvent_t> prof_ev_;
  std::map<int, hipGraphExec_t> graphs_;
  std::vector<NodeStat> stats_;
  double last_run_ms_ = 0.0;
  int last_batch_ = 0;  // batch of the last run / dry run / profileNodes (0: none yet)
  bool dry_ = false;
  uintptr_t fake_next_ = (uintptr_t)1 << 44;
  std::vector<std::pair<uintptr_t, size_t>> allocs_;
};

}  // namespace ivh
