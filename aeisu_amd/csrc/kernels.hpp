// Host-side launchers of the gfx950 kernels (defined in k_*.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace aeisu {

int project_num_tiles(int batch, int Hq, int Wq);
int grouped_num_tiles(int batch, int Hl, int Wl);
int refine_num_tiles(int batch, int Hq, int Wq);
int head_num_tiles(int batch, int H, int W);

hipError_t launch_project(int in_fp32, int precise, const void* src, const void* wfrag, const float* bias, void* skip,
                          const float* analysis24, int H, int W, int Hq, int Wq, int py, int px, int batch,
                          int grid, hipStream_t stream);
hipError_t launch_compress(int mode, const void* skip, const void* wfrag, const float* bias, const float* scale,
                           void* low, float inv_in, float inv_out, int Hl, int Wl, int batch, int grid,
                           hipStream_t stream);
hipError_t launch_grouped(int mode, const void* in, const void* wfrag, const float* bias, const float* scale,
                          void* out, float inv_out, int Hl, int Wl, int batch, int grid, hipStream_t stream);
hipError_t launch_expand(int mode, const void* low, const void* skip, const void* wfrag, const float* bias,
                         const float* scale, void* work, float inv_out, float s_out, int Hl, int Wl, int batch,
                         int grid, hipStream_t stream);
hipError_t launch_refine_tail(const void* work, const void* wfrag, const float* rbias, const float* tbias,
                              void* meta, int Hq, int Wq, int batch, int grid, hipStream_t stream);
// Head bank image (engine.cpp): kHeadBankFrags MFMA fragments of 64 lanes x 8 FP16, then the FP32 base of
// each lane group's rows per row tile (float4 [4][7]) for the quantized policies' head (qclamp).
constexpr int kHeadBankFrags = 14;
// qclamp: quantized policies' head (clamped coefficients rounded to FP16, one MFMA per row tile);
// 0: the FP16 policy's exact clamp split.
hipError_t launch_head(int in_fp32, int out_fp32, int qclamp, const void* src, const void* meta, const void* bankA,
                       void* out, int H, int W, int Hq, int Wq, int py, int px, int batch,
                       unsigned* nonfinite, int grid, hipStream_t stream);

// Fused body: compress, the four grouped layers and expand in one kernel (activations in LDS).
// Layer order in the arrays: 0 compress, 1..4 bottleneck 0..3, 5 expand.
// consts: the per-channel epilogue constants, kBodyConsts floats:
//   [0, 64) compress bias, [64, 128) compress scale, then per bottleneck l = 0..3
//   [128 + 128 l, +64) bias and [+64, +128) scale, then expand [640, 768) bias and
//   [768, 896) scale, both indexed T * 16 + m for output channel (16 * (T >> 2) + m) * 4 + (T & 3),
//   then the project bias [896, 928).  Scales are 0 for the FP16 policy.
// Input: the skip tensor (BodySrc::Skip, written by the project kernel), or (quantized
// policies) the frames themselves (FP16 / FP32), from which the kernel recomputes analysis features and project
// for the compress halo and again for the expand residual, so no skip tensor exists.  The
// frame-input variants take the compress weights in the project-accumulator K order: for the
// E4M3 policies every compress kernel uses that order, INT8 has a separate packing (compress_rgb).
constexpr int kBodyConsts = 928;
enum class BodySrc : int { Skip = 0, Frames16 = 1, Frames32 = 2 };
struct BodyFusedArgs {
  const _Float16* skip;    // BodySrc::Skip
  const void* frames;      // frame-input variants: planar [batch][3][H][W]
  _Float16* work;
  const void* frag[6];
  const void* pfrag;       // project weight fragments (frame-input variants)
  const float* consts;
  float inv_out[6];        // 1 / output activation scale of each layer (quantized policies)
  float inv_in;            // 1 / compress input scale
  float s_out;             // expand output scale (dequantization before the skip add)
  float analysis[24];      // analysis constants (frame-input variants)
  int Hl, Wl;
  int H, W, py, px;        // frame geometry (frame-input variants)
  int row0, rows;          // low-grid rows this launch covers: [row0, row0 + rows); rows = 0: all
  int col0, cols;          // low-grid columns likewise: [col0, col0 + cols); cols = 0: all
  // compress exchange (launch_body_fused_xc): each tile computes compress on its core only and takes
  // the 4-pixel ring of its compress region from its neighbours' cores
  unsigned char* xbuf;     // compress outputs of the tile cores' borders, [batch][Hl][Wl][64] bytes
  unsigned* xflags;        // per-tile launch counters (zeroed once; each launch adds one per tile)
  int xspins;              // polls of a neighbour's counter before the tile computes its ring itself
                           // (<= 0: always itself)
};
// tile = side of the body's output tile in low pixels (0: the policy's default, 24, or 16 for the FP16 policy)
int body_fused_num_tiles(int mode, int batch, int Hl, int Wl, int tile = 0);
// Frame-input body plan on a device with `cus` compute units: the leading `frames24` frames on 24x24
// tiles and the rest on 16x16 tiles, or (cols24 > 0) every frame's low columns [0, cols24) on 24x24
// tiles and the rest on 16x16 tiles
struct BodyPlan {
  int frames24, cols24;
};
BodyPlan body_fused_plan(int mode, int batch, int Hl, int Wl, int cus);
// Frame-input body with the compress exchange in launches of `frames` whole frames on tiles of side
// `tile` (tile 0: the launches do not fit or do not pay); tile24_only: compared with the single
// 24x24-tile launch instead of the body plan.
struct BodyXcPlan {
  int tile, frames;
};
BodyXcPlan body_fused_xc_plan(int mode, int batch, int Hl, int Wl, int cus, bool tile24_only);
// FP16 policy (skip input): low rows [0, R) on 16x16 tiles, the rest on 8x8 tiles; returns R
int body_fused_row_split(int mode, int batch, int Hl, int Wl, int cus);
hipError_t body_fused_prepare();
hipError_t launch_body_fused(int mode, BodySrc src, const BodyFusedArgs& args, int batch, int tile,
                             hipStream_t stream);
// Frame-input body with the compress exchange (quantized policies, whole frames, tile 24 or 16): one
// block per tile, every block resident at once (tiles <= CUs, one block per CU), neighbouring tiles
// synchronised through args.xflags.
hipError_t launch_body_fused_xc(int mode, BodySrc src, const BodyFusedArgs& args, int batch, int tile, int cus,
                                hipStream_t stream);
// two parts in one launch: batch1 frames (or a1's rows) on tile1 tiles, then batch2 frames (a2's
// rows) on tile2 tiles; tiles (24, 16) for the quantized policies, (16, 8) for the FP16 policy
hipError_t launch_body_fused_pair(int mode, BodySrc src, const BodyFusedArgs& a1, int batch1, int tile1,
                                  const BodyFusedArgs& a2, int batch2, int tile2, hipStream_t stream);

// Fused refine + tail + head (coefficients in LDS); one block per CU (1024 threads for FP16
// frames, 768 for FP32 frames).
int fused_num_tiles(int in_fp32, int batch, int H, int W, int Hq, int Wq, int py, int px);
hipError_t fused_prepare();
hipError_t launch_fused_tail_head(int in_fp32, int out_fp32, int qclamp, const void* work, const void* src,
                                  const void* rt_frag, const float* rbias, const float* tbias, const void* bankA,
                                  void* out, int H, int W, int Hq, int Wq, int py, int px, int batch,
                                  unsigned* nonfinite, int grid, hipStream_t stream);

// FP32 policy (k_fp32.hip): per-layer kernels on FP32 NHWC activations.  Weight image (floats),
// every layer [tap][ci][co] (co fastest) followed by its bias:
//   project  W[32 feature channel f*4+phase][32] b[32]; compress W[128 skip channel c*4+phase][64] b[64];
//   bottleneck l: W[9][32 group input][64] b[64] (output 32g+o reads group g's inputs);
//   expand W[64][128] b[128] (output c*4+phase); refine W[9][32][64] b[64]; tail W[64][64] b[64];
//   then adaptive_base [25][4], adaptive_basis [25][16][4], the 24 analysis constants.
constexpr int kF32Project = 0;
constexpr int kF32Compress = kF32Project + 32 * 32 + 32;
constexpr int kF32GroupedStride = 9 * 32 * 64 + 64;
constexpr int kF32Grouped = kF32Compress + 128 * 64 + 64;
constexpr int kF32Expand = kF32Grouped + 4 * kF32GroupedStride;
constexpr int kF32Refine = kF32Expand + 64 * 128 + 128;
constexpr int kF32Tail = kF32Refine + 9 * 32 * 64 + 64;
constexpr int kF32Base = kF32Tail + 64 * 64 + 64;
constexpr int kF32Basis = kF32Base + 25 * 4;
constexpr int kF32Analysis = kF32Basis + 25 * 16 * 4;
constexpr int kF32Floats = kF32Analysis + 24;
// project, compress, the four grouped layers, expand, refine + tail (events 1..5 after each stage
// when ev is not null); lows: the five layer outputs when every layer is kept, else null (ping-pong
// between low0 and low1)
hipError_t launch_f32_controller(int in_fp32, const void* src, const float* wimg, float* skip, float* low0, float* low1,
                                 float* const* lows, float* work, float* meta, int H, int W, int Hq, int Wq, int py, int px,
                                 int batch, hipStream_t stream, hipEvent_t* ev);
hipError_t launch_f32_head(int in_fp32, int out_fp32, const void* src, const float* meta, const float* wimg, void* out,
                           int H, int W, int Hq, int Wq, int py, int px, int batch, unsigned* nonfinite,
                           hipStream_t stream);

// Resident blocks per CU (occupancy), used to size the persistent grids.
int head_blocks_per_cu(int in_fp32, int out_fp32, int qclamp);
int project_blocks_per_cu(int in_fp32, int precise);
int refine_blocks_per_cu();
int body_blocks_per_cu(int kind, int mode);   // kind 0 compress, 1 grouped, 2 expand

// Static scratch of the allocation-free entry point (noalloc.hip): 72 MiB per device, enough for the
// work tensor (and the FP16 policy's skip tensor) of one 1920x1080 frame in every policy.
constexpr size_t kNoAllocScratchBytes = size_t(72) << 20;
// Once per device, with that device current: looks up the array's device address.
hipError_t noalloc_scratch_init(int device);
// The array's device address on `device` (nullptr before noalloc_scratch_init succeeded there).
void* noalloc_scratch(int device);

}  // namespace aeisu
