/*
 * ivh.h -- C ABI of the MI355X (gfx950) HIP backend for infvino plans.
 *
 * This is the drop-in boundary beneath infvino's ClBackend / PlanModel: plain C types,
 * plain pointers and sizes, no HIP/C++ types in the signatures.  Every function returns
 * an int status (IVH_OK = 0); on failure ivh_last_error() gives the message (thread-local),
 * the same text the reference throws as std::runtime_error.
 *
 * Reference interfaces each entry point replaces (file:line in the reference repository):
 *   ivh_create            PlanModel::PlanModel(plan_path, kernel_dir, platform, device, profiling)
 *                         include/infvino/PlanModel.hpp:57-59, src/PlanModel.cpp:116-209
 *   ivh_destroy           PlanModel::~PlanModel, include/infvino/PlanModel.hpp:60
 *   ivh_input_dims        PlanModel::inputDims / inputNumel, PlanModel.hpp:65-67
 *   ivh_output_count      PlanModel::outputCount, PlanModel.hpp:69
 *   ivh_output_dims       PlanModel::outputDims / outputNumel, PlanModel.hpp:71-72
 *   ivh_set_input_f16     PlanModel::setInput(const void* fp16), PlanModel.hpp:75; src/PlanModel.cpp:428-432
 *   ivh_set_input_f32     ClBackend::infer's f32_to_f16_bulk + setInput, src/ClBackend.cpp:42-44
 *                         (truncating conversion of include/infvino/Half.hpp:14-24)
 *   ivh_run               PlanModel::run, PlanModel.hpp:77; src/PlanModel.cpp:3127-4178
 *   ivh_read_output_f16   PlanModel::readOutput, PlanModel.hpp:79; src/PlanModel.cpp:4180-4184
 *   ivh_read_output_f32   ClBackend::infer's readOutput + f16_to_f32_bulk, src/ClBackend.cpp:53-61
 *   ivh_read_tensor_f16   PlanModel::readTensor, PlanModel.hpp:83; src/PlanModel.cpp:4186
 *   ivh_tensor_numel      PlanModel::tensorNumel, PlanModel.hpp:85
 *   ivh_last_run_ms       PlanModel::lastRunMs / ClBackend::lastInferMs, PlanModel.hpp:176, ClBackend.hpp:47
 *   ivh_profile_nodes     PlanModel::profile() per-node GPU time, PlanModel.hpp:201-224
 *   ivh_node_info         PlanModel::PlanProfile::NodeRow (op, tag, signature), PlanModel.hpp:203-211
 *   ivh_node_tag          PlanModel::PlanProfile::NodeRow::tag (shape and data path), PlanModel.hpp:208
 *   ivh_device_info       ClBackend::device() / describeDevice, ClBackend.hpp:46, include/infvino/Device.hpp
 *   ivh_runtime_version   DeviceInfo::opencl_version, include/infvino/Device.hpp:23
 *   ivh_node_times        PlanModel::profile() / opProfile() accumulated under profiling=true,
 *                         PlanModel.hpp:176-224; src/PlanModel.cpp:3183-3196
 *   ivh_clear_profile     PlanModel::clearProfile, PlanModel.hpp:226-233
 * The batch argument is new: the reference runs one image per call (src/PlanModel.cpp:3561-3564
 * read C,H,W from the last three dims).  Here a call processes `batch` images stored back to
 * back (image stride = the plan's per-image numel); batch == 1 is the reference behaviour.
 */
#ifndef IVH_H_
#define IVH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IVH_OK 0
#define IVH_ERR_INVALID 1   /* bad argument, malformed plan, missing file, shape mismatch */
#define IVH_ERR_DEVICE 2    /* HIP runtime error */
#define IVH_ERR_INTERNAL 3

/* ivh_create flags */
#define IVH_FLAG_NO_GRAPH 0x1u    /* launch node by node instead of replaying a HIP graph */
#define IVH_FLAG_NO_REUSE 0x2u    /* every tensor gets its own memory (readTensor sees all) */
#define IVH_FLAG_NO_FUSE 0x4u     /* no residual/activation fusion, no zero-copy views */
#define IVH_FLAG_NCHW_ONLY 0x8u   /* keep every activation in the plan's NCHW layout */
#define IVH_FLAG_DIRECT_ONLY 0x10u /* no MFMA implicit GEMM: direct convolution kernels */
#define IVH_FLAG_ASYNC 0x20u      /* ivh_run returns without waiting for the device */
#define IVH_FLAG_NO_SPLITK 0x80u  /* never split the K loop of an implicit-GEMM conv */
#define IVH_FLAG_NO_HALO 0x100u   /* 3x3 convs use the im2col path, never the LDS halo tile */
#define IVH_FLAG_NO_RESIDENT 0x200u /* 3x3 stride-1 convs never keep their weights resident in
                                       LDS (the halo tile or im2col path instead) */
#define IVH_FLAG_NO_FUSE_DECODE 0x400u /* keep a Detect / Pose head's decode tail (DFL,
                                          dist2bbox, keypoint decode) node by node instead of
                                          one fused kernel */
#define IVH_FLAG_DRY_RUN 0x40u    /* no device: plan, pack and bounds-check launches only
                                     (ivh_run validates, data calls fail) */
#define IVH_FLAG_NO_PIPE 0x2000u  /* 3x3 stride-1 convs never use the DMA-pipelined kernel */
#define IVH_FLAG_NO_FUSE_PAIR 0x8000u /* run a C2f / C3k2 bottleneck's two 3x3 convs (16 or
                                        32 channels) as two launches, not one */
#define IVH_FLAG_NO_S2_PERSIST 0x10000u /* 3x3 stride-2 convs never use the persistent
                                           resident-weight kernel */
#define IVH_FLAG_NO_WIDE 0x40000u /* 3x3 stride-1 convs never use the wide-layer kernel */
#define IVH_FLAG_NO_PINGPONG 0x80000u /* 3x3 stride-1 convs with Cin <= 64 never use the
                                         ping-pong resident-weight kernel */
#define IVH_FLAG_NO_FUSE_UPSAMPLE 0x100000u /* run a 2x resize_nn whose output only feeds a
                                               concat read by one 1x1 conv, instead of that
                                               conv reading the resize's input directly */
#define IVH_FLAG_NO_FUSE_SIBLINGS 0x200000u /* run sibling 3x3 convs that read the same
                                               tensor (a Pose head's branches) one by one
                                               instead of as one conv over all their output
                                               channels */
#define IVH_FLAG_NO_PW 0x20000u   /* 1x1 convs never use the streaming pointwise kernels */
#define IVH_FLAG_PIPE_ANY 0x4000u /* 3x3 stride-1 convs use the DMA-pipelined kernel wherever it
                                     applies (Cin >= 32, any grid size), not only where it is
                                     measured fastest */
#define IVH_FLAG_NO_FUSE_ATTN 0x1000u /* keep an attention core (q^T k, scale, softmax, v P^T)
                                         node by node instead of one fused kernel */
#define IVH_FLAG_PROFILE 0x800u   /* PlanModel's profiling=true: every run launches node by node
                                     with a HIP event between nodes, waits, and adds each node's
                                     time to the totals ivh_node_times reports (no graph) */

typedef struct ivh_model ivh_model;

const char * ivh_last_error(void);
int ivh_version(int * major, int * minor);
int ivh_device_count(int * n);
/* name / compute units / peak clock of a device (ClBackend::device(), src/Device.cpp) */
int ivh_device_info(int device, char * name, size_t name_len, int * compute_units, int * clock_mhz);
/* "HIP <runtime version>, driver <driver version>": the runtime string DeviceInfo carries in
   the reference's opencl_version slot (include/infvino/Device.hpp:16-26) */
int ivh_runtime_version(char * buf, size_t len);

int ivh_create(const char * plan_path, int device, int max_batch, uint32_t flags, ivh_model ** out);
int ivh_destroy(ivh_model * m);

/* dims: caller array of capacity *rank; on return *rank = actual rank */
int ivh_input_dims(const ivh_model * m, int64_t * dims, int * rank);
int ivh_input_numel(const ivh_model * m, size_t * numel);
int ivh_output_count(const ivh_model * m, int * n);
int ivh_output_dims(const ivh_model * m, int i, int64_t * dims, int * rank);
int ivh_output_numel(const ivh_model * m, int i, size_t * numel);
int ivh_max_batch(const ivh_model * m, int * max_batch);

/* host buffers hold `batch` images back to back (batch * per-image numel elements) */
int ivh_set_input_f16(ivh_model * m, const uint16_t * host, int batch);
int ivh_set_input_f32(ivh_model * m, const float * host, int batch);
/* ivh_set_input_f32 without any device allocation (no counterpart in the reference): for
   callers that cannot allocate -- code around HIP graph capture, serving loops that forbid
   hipMalloc.  ivh_set_input_f32 stages the f32 input in a device buffer it allocates on its
   first call; this one streams it through a fixed 8 MiB array that every GPU the library
   runs on holds until the process ends, 2^21 floats at a time, so no batch is too large for
   it (batch is checked against the model's maximum, as for ivh_set_input_f32).  Results are
   bit-identical to ivh_set_input_f32's.  Calls on one GPU (two models, or two threads) share
   the array; each call holds a per-device lock until its copies and conversions have
   finished, so such calls run one after the other. */
int ivh_set_input_f32_noalloc(ivh_model * m, const float * host, int batch);
int ivh_run(ivh_model * m, int batch);
int ivh_sync(ivh_model * m);
int ivh_read_output_f16(ivh_model * m, int i, uint16_t * host, int batch);
int ivh_read_output_f32(ivh_model * m, int i, float * host, int batch);
/* any declared tensor, as NCHW fp16; returns IVH_ERR_INVALID for an unknown name */
int ivh_read_tensor_f16(ivh_model * m, const char * name, uint16_t * host, int batch);
int ivh_tensor_numel(const ivh_model * m, const char * name, size_t * numel);
int ivh_last_run_ms(const ivh_model * m, double * ms);

/* profiling: per-node device time (ms): each node run `iters` times back to back between two
   HIP events on the model stream, mean per run; a full pass afterwards restores all tensors */
int ivh_node_count(ivh_model * m, int * n);
int ivh_profile_nodes(ivh_model * m, int batch, int iters, double * ms, int cap);
/* totals over the runs of an IVH_FLAG_PROFILE model since creation or ivh_clear_profile:
   per node the summed device time (ms) and the number of runs that launched it
   (PlanModel::profile().nodes / opProfile() accumulate the same way, PlanModel.hpp:176-234) */
int ivh_node_times(const ivh_model * m, double * ms, int * calls, int cap);
int ivh_clear_profile(ivh_model * m);  /* PlanModel::clearProfile, PlanModel.hpp:226-233 */
/* node i: op, kernel family and shape text; algorithmic FLOPs and fp16 bytes per image */
int ivh_node_info(ivh_model * m, int i, char * op, size_t op_len, char * kernel, size_t kernel_len,
                  char * desc, size_t desc_len, double * flops, double * bytes);
/* Runtime tag of node i: the kernel label of ivh_node_info followed by its launch detail
 * (tile config, channel chunk, K step, split, build), as PlanProfile::NodeRow::tag carries the
 * data path (include/infvino/PlanModel.hpp:208).  Kernel labels and tags describe the batch of
 * the model's last ivh_run / ivh_profile_nodes call (max_batch before the first), since kernel
 * and tile choices depend on the batch. */
int ivh_node_tag(ivh_model * m, int i, char * tag, size_t tag_len);
int ivh_memory_info(const ivh_model * m, int batch, size_t * arena_bytes, size_t * weight_bytes);

/* ---------------------------------------------------------------- single-op entry points
 * One operation on caller-owned device buffers (hipMalloc'd; `stream` is a hipStream_t, NULL
 * for the null stream), for op-level checks and benchmarks: the reference drives its kernels
 * one at a time from scripts/kernel_check.py:34-137 and tools/infvino_numtest.cpp:88-100
 * through PlanModel's per-op dispatch (src/PlanModel.cpp:3418-3990, small ops 2681-3088).
 * Every tensor holds `batch` images back to back (image stride = its per-image element
 * count, channels-last tensors: H*W*round8(C)); fp16 storage, fp32 accumulation.  The calls
 * enqueue and return; a bad argument is reported before anything is enqueued.
 */
typedef struct ivh_conv_desc {
  int cin, cout, h, w;      /* input / output channels, input height and width */
  int k, stride, pad, groups;
  int act;                  /* 0 none, 1 SiLU, 2 ReLU, 3 HardSwish, 4 HardSigmoid, 5 Sigmoid */
  int has_bias;             /* 1: the packing holds a bias */
  int channels_last;        /* 1: x, res and y are NHWC, pixel stride round8(C); 0: NCHW */
} ivh_conv_desc;

/* output height and width of d */
int ivh_conv_out_dims(const ivh_conv_desc * d, int * ho, int * wo);
/* bytes of d's packed operands (the device buffer ivh_pack_conv_weights fills) */
int ivh_conv_packed_bytes(const ivh_conv_desc * d, size_t * bytes);
/* packs plan-order fp16 weights w[cout][cin/groups][k][k] and fp16 bias[cout] (host memory;
   bias NULL when !has_bias) into packed_dev (replaces the reference's per-kernel weight
   repacks, src/PlanModel.cpp:232-334); synchronous */
int ivh_pack_conv_weights(const ivh_conv_desc * d, const uint16_t * w_host, const uint16_t * bias_host,
                          void * packed_dev);
/* y = act(conv(x, w) + b) (+ res; res may be NULL): conv1x1 -> gemm_f16 (kernels/gemm.cl:183-669),
   conv3x3 -> conv3x3_ov / _blk / _cin3 / _f16, grouped and depthwise -> conv_general
   (src/PlanModel.cpp:3447-3933) */
int ivh_conv2d_f16(const ivh_conv_desc * d, const void * x, const void * packed, const void * res, void * y,
                   int batch, void * stream);
/* the same for a depthwise conv only (groups == cin == cout, k 3 or 5): depthwise_f16 /
   depthwise_blk (kernels/conv_general.cl:85-187, depthwise_blk.cl:118-228) */
int ivh_dwconv_f16(const ivh_conv_desc * d, const void * x, const void * packed, const void * res, void * y,
                   int batch, void * stream);
/* FC: y[b][o] = act(sum_i W[o][i] x[b][i] + bias[o]), x [batch][n_in], y [batch][n_out]; packed
   with the desc {cin n_in, cout n_out, h 1, w 1, k 1, stride 1, pad 0, groups 1, act, has_bias,
   channels_last 0}: conv1x1_gemv_f16 (kernels/conv1x1.cl:157-198) */
int ivh_gemv_f16(const ivh_conv_desc * d, const void * x, const void * packed, void * y, int batch, void * stream);
/* elementwise over n elements per image (ew_binary / ew_unary, kernels/ops.cl:10-63): with b,
   y = a op b (op 0 add, 1 sub, 2 mul, 3 div; b_scalar: b is one element shared by all);
   with b == NULL, y = act_op(a) (op: the activation codes of ivh_conv_desc.act) */
int ivh_eltwise_f16(int op, const void * a, const void * b, int b_scalar, void * y, size_t n, int batch,
                    void * stream);
/* NCHW [batch][c][h][w]: kind 0 maxpool (k, s, p; taps outside the image ignored, ops.cl:148-166),
   kind 1 nearest upsample by s (k, p unused; ops.cl:168-179) */
int ivh_pool_f16(int kind, const void * x, void * y, int c, int h, int w, int k, int s, int p, int batch,
                 void * stream);
/* softmax over the middle axis of [outer][axis][inner] (ops.cl:181-197) */
int ivh_softmax_f16(const void * x, void * y, int outer, int axis, int inner, int batch, void * stream);
/* y[i] = a[i] . b[i]: a [bb][m][k], b [bb][k][n], y [bb][m][n] per image (ops.cl:276-294) */
int ivh_bmm_f16(const void * a, const void * b, void * y, int bb, int m, int k, int n, int batch,
                void * stream);

#ifdef __cplusplus
}
#endif

#endif /* IVH_H_ */
