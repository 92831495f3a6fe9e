// Host-side launchers of the gfx950 kernels.  Each takes fully resolved device views
// (batch-B pointers) and a stream; all shape checks happen in the executor before launch.
#pragma once

#include "ivh_internal.hpp"

#include <mutex>
#include <string>

namespace ivh {

// conv_mfma.hip
int igemm_bn(int cout);                    // N tile of the implicit GEMM for a Cout
int igemm_bk(int cout, int kk);            // K step of a layer with K*K*cin8 = kk (32 / 64)
bool upcat_ok(const ConvParams & p);      // the implicit GEMM's upsample-concat input applies
int igemm_kpad(int cout, int kk);          // packed K: kk rounded up to that step
constexpr int kIgemmBK = 32;               // packed K is always a multiple of this
constexpr int kIgemmRowPad = 128;          // packed weight rows padded to this multiple
void launch_conv_igemm(const ConvParams & p, hipStream_t s);
// launch detail of an implicit-GEMM-family conv (resident-weight / LDS-patch / stride-2 tile
// config, or the im2col tile, K step, split and build) for node tags
std::string igemm_launch_tag(const ConvParams & p);
int conv_batch_chunk(const ConvParams & p);                      // images per launch (< 2^31 B input)
ConvParams conv_batch_slice(const ConvParams & p, int b0, int nb);  // images [b0, b0 + nb)
int igemm_ksplit(long M, int cout, int kpad);  // 1 = no split

// conv_halo.hip: 3x3 stride-1 pad-1 convs with an LDS input patch
constexpr int kHaloCfgs = 9;         // tile configs of the LDS-patch kernel
int halo_cfg_ck(int cfg, int cin);  // input-channel chunk a tile config uses (16 / 32 / 64)
int halo_taps(int ck);               // taps per chunk in the packing (9, or 10 with a zero tap)
// tile config (cfg) and output tile th x tw for a layer at a batch size; false: not eligible
bool halo_plan(int cin, int cout, int H, int W, int batch, int * cfg, int * th, int * tw);
long halo_grid_x(const ConvParams & p);
int halo_bn(int cfg);
int halo_pmax(int cfg);
void launch_conv_halo(const ConvParams & p, hipStream_t s);

// conv_res.hip: 3x3 stride-1 pad-1 convs with 16 < Cin <= 64, weights resident in LDS
int res_ck(int cin);                 // channel chunk (= Cin rounded up to 32 / 64)
int res_bn(int cfg);
int res_bm(int cfg);
int res_pmax(int cfg);
long res_tiles(const ConvParams & p);
int res_grid_x(const ConvParams & p, int cfg);
// config and output tile th x tw for a layer at a batch size; false: not eligible
bool res_plan(int cin, int cout, int H, int W, int batch, int act, bool pingpong, int * cfg, int * th, int * tw);
// the output (and residual) views suit the kernel's 8-byte channels-last buffer stores
bool res_views_ok(const ConvParams & p);
int res_store_width(const ConvParams & p);  // channels per output store: 8, 4 or 1 (padding absorbs the rounding up)
constexpr int kResMinTiles = 1;  // fewer tiles: the halo / im2col kernels
constexpr int kResMaxRows = 34;  // patch rows (TH + 2) of the resident-weight kernel's tiles
constexpr int kHaloMaxRows = 34;  // patch rows (TH + 2) of the LDS-patch kernel's tiles
void launch_conv_res(const ConvParams & p, hipStream_t s);

// conv_wide.hip: 3x3 stride-1 pad-1 convs with Cin % 32 == 0, Cin >= 128, 64 < Cout <= 256,
// one persistent work-group per CU over an equal share of the output pixels
bool wide_plan(int cin, int cout, int H, int W, int batch, int act, int * tm, int * gx);
bool wide_tm_ok(int tm);
long wide_grid(const ConvParams & p);
void launch_conv_wide(const ConvParams & p, hipStream_t s);

// conv_pipe.hip: 3x3 stride-1 pad-1 convs with Cin % 8 == 0, Cin >= 32, fed through LDS by
// DMA (buffer loads into LDS), persistent over (tile, channel block) items
// config and output tile th x tw for a layer at a batch size; false: not eligible
bool pipe_plan(int cin, int cout, int H, int W, int batch, int act, int * cfg, int * th, int * tw);
int pipe_bn(int cfg);
long pipe_items(const ConvParams & p);
// the input, output and residual views suit the kernel (16-byte channels-last input pieces,
// 8-channel output stores, 4-channel residual loads)
bool pipe_views_ok(const ConvParams & p);
constexpr int kPipeMinItems = 256;  // fewer items: the other 3x3 kernels
void launch_conv_pipe(const ConvParams & p, hipStream_t s);

// conv_pair.hip: two chained 3x3 stride-1 convs of C = 16 or 32 channels (a bottleneck) in
// one launch
bool pair_plan(int C, int H, int W, int batch, int * th, int * tw);  // output tile; false: not eligible
// channels of a fused bottleneck pair: outer C (the block's input and output) and middle
// M (the first conv's output): C = 16 or 32 with M = C or M = C / 2
inline bool pair_channels_ok(int c, int m) { return (c == 16 || c == 32) && (m == c || 2 * m == c); }
bool pair_tile_ok(int C, int th, int tw);  // the tile fits the kernel's ring, patch and rows
long pair_tiles(int H, int W, int batch, int th, int tw);
// a: the first conv (x, weights / bias / act of conv 1), b: the second (y, residual,
// weights / bias / act of conv 2, th x tw); both weights in the 32-channel halo packing
void launch_conv_pair(const ConvParams & a, const ConvParams & b, hipStream_t s);

// conv_pw.hip: 1x1 stride-1 convs with Cout <= 128 on channels-last views (streaming)
bool pw_views_ok(const ConvParams & p);
bool pw_plan(const ConvParams & p);         // eligible (shape, activation, views, LDS)
long pw_blocks(const ConvParams & p);       // 32-pixel blocks of the batch
size_t pw_lds_bytes(const ConvParams & p);  // weights and bias in LDS
// planar-output variant (p.pw == 2): NCHW y, x NCHW planes (p.xt) or channels-last,
// Cin <= 64, Cout <= 128
bool pwt_views_ok(const ConvParams & p);
bool pwt_plan(const ConvParams & p);
size_t pwt_lds_bytes(const ConvParams & p);
constexpr long kPwMinBlocks = 1024;
void launch_conv_pw(const ConvParams & p, hipStream_t s);

// conv_s2.hip: 3x3 stride-2 pad-1 convs with 8 < Cin <= 16, Cout <= 64 (configs 0, 1: one
// tile per work-group), and the persistent resident-weight kernel (configs 2-5: 16 or 32
// input channels, Cout <= 32 or <= 64; config 6: 64 input channels, Cout <= 128)
int s2pk_ck(int cfg);                       // input-channel chunk of a persistent config
int s2pk_cb(int cfg);                       // 32-channel output blocks of a persistent config
int s2pk_th(int cfg);                       // output tile rows of a persistent config (16 columns)
bool s2pk_views_ok(const ConvParams & p);   // output NHWC 16-byte stores, no residual, 32-bit offsets
long s2pk_tiles(const ConvParams & p);      // output tiles (p.s2 set)
constexpr long kS2PkMinTiles = 512;
bool s2_plan(int cin, int cout, int Ho, int Wo, int * cfg, int * th, int * tw);
int s2_patch(int th, int tw);  // patch pixels of a th x tw output tile
int s2_cfg_bm(int cfg);
int s2_cfg_bn(int cfg);
int s2_cfg_ck(int cfg);
int s2_cfg_pmax(int cfg);
long s2_grid(const ConvParams & p);
void launch_conv_s2(const ConvParams & p, hipStream_t s);

// kernels_misc.hip
void launch_conv_direct(const ConvParams & p, hipStream_t s);   // any K/S/P/G, any layout
void launch_dwconv(const ConvParams & p, hipStream_t s);        // depthwise, any layout
std::string dw_launch_tag(const ConvParams & p);                 // kernel and tile of a depthwise launch
bool dwconv_vectorizable(const ConvParams & p);
bool stem_rows_supported(const ConvParams & p);  // the row-tiled stem kernel applies

enum SmallOp : int {
  kEwSame = 0,     // y = op(a, b), same geometry; b.img == 0 && b.cs == 0 -> scalar
  kEwBcast,        // NCHW flat broadcast, dims = bdims spec
  kEwChan,         // per-channel broadcast: i0 = 1 if a is the [C] operand
  kEwUnary,        // y = act(a), op = canonical activation code
  kCopy,           // y(c,p) = a(c,p) (any layouts): split / concat parts / layout change
  kSliceAxis,      // NCHW flat: i0 outer, i1 axdim, i2 inner, i3 start, i4 len
  kConcatOuter,    // NCHW flat 4-source concat along an inner axis (see executor)
  kMaxPool,
  kResizeNN,
  kSoftmax,        // NCHW flat: i0 outer, i1 axdim, i2 inner
  kPermute,        // NCHW flat: i0 D1, i1 D2, i2 I, op = mode
  kGap,            // a view [C,H,W] -> y flat [C]
  kBmm,            // NCHW flat: i0 BB, i1 M, i2 K, i3 N  (a: [BB][M][K], b: [BB][K][N]);
                   // op bit 0: a stored [BB][K][M], bit 1: b stored [BB][N][K]
  kBiasAdd,        // NCHW flat: i0 HW
  kMaxPoolSppf,    // NHWC, C % 8 == 0, H * W <= 1024: a -> y, b, c = 5x5, 9x9, 13x13 max
                   // pools (stride 1, clipped windows): three chained 5x5 pad-2 pools
};
void launch_small(int kind, const SmallParams & p, hipStream_t s);
void launch_pose_decode(const DecodeParams & p, hipStream_t s);  // fused head decode
void launch_attention(const AttnParams & a, hipStream_t s);      // fused attention core
int attn_key_blocks(int n);  // key blocks of 32 the fused attention kernel holds (0: n too large)
void launch_bmm_mfma(const SmallParams & q, hipStream_t s);  // bmm_mfma.hip

// boundary conversions (include/infvino/Half.hpp semantics for the truncating one)
void launch_f32_to_f16_trunc(const float * in, __half * out, long n, hipStream_t s);
// Device address of the current GPU's fixed staging array (kBoundaryScratchFloats floats,
// 8 MiB) for ivh_set_input_f32_noalloc; `device` must be the current device.
constexpr long kBoundaryScratchFloats = 1L << 21;
float * boundary_scratch(int device);
// one mutex per device, held by a caller while its copies and kernels use that device's array
std::mutex & boundary_scratch_lock(int device);
void launch_f16_to_f32(const __half * in, float * out, long n, hipStream_t s);

}  // namespace ivh
