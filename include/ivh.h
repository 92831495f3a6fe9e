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
 *   ivh_device_info       ClBackend::device() / describeDevice, ClBackend.hpp:46, include/infvino/Device.hpp
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
#define IVH_FLAG_DRY_RUN 0x40u    /* no device: plan, pack and bounds-check launches only
                                     (ivh_run validates, data calls fail) */

typedef struct ivh_model ivh_model;

const char * ivh_last_error(void);
int ivh_version(int * major, int * minor);
int ivh_device_count(int * n);
/* name / compute units / peak clock of a device (ClBackend::device(), src/Device.cpp) */
int ivh_device_info(int device, char * name, size_t name_len, int * compute_units, int * clock_mhz);

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
/* node i: op, kernel family and shape text; algorithmic FLOPs and fp16 bytes per image */
int ivh_node_info(ivh_model * m, int i, char * op, size_t op_len, char * kernel, size_t kernel_len,
                  char * desc, size_t desc_len, double * flops, double * bytes);
int ivh_memory_info(const ivh_model * m, int batch, size_t * arena_bytes, size_t * weight_bytes);

#ifdef __cplusplus
}
#endif

#endif /* IVH_H_ */
