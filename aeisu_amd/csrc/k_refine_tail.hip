// Refine 3x3 (32 -> 64) + LeakyReLU + linear 1x1 tail (64 -> 64) at packed
// (half) resolution, producing the FP16 parity-major coefficient tensor.
//
// Reference: aeisu/model.py:489-490 (refine_540, metadata_head); native
// fused_native_fp16_refine_tail_conv_kernel,
// optimized/native/src/neural/srcpyr/SrcPyrNativeFp16Refine.cuh:334-557
// (FP16 operands, FP32 accumulation, FP32 refine bias, FP16-rounded tail bias).
//
// gfx950 mapping: a block owns a 32x4 pixel tile (one row of 32 px per wave,
// two 16-px MFMA column groups).  The zero-padded 34x6x32 FP16 input patch
// sits in LDS (80-byte pixel stride, conflict-free 16-byte reads).  Each
// wave keeps all refine (4 out tiles x 9 taps) and tail (4 x 2) weight
// fragments in registers; the refine accumulators are converted to FP16 and
// used directly as the tail's B operand (the tail's K order is permuted on
// the host to match the accumulator layout), so the 64-channel refine
// activation never leaves registers.
#include "common.hpp"

namespace aeisu {

constexpr int kRTW = 32, kRTH = 4;
constexpr int kRPW = kRTW + 2, kRPH = kRTH + 2;
constexpr int kRPix = 40;                     // halves per LDS pixel (32 + 8 pad)
constexpr int kRefineFrag = 4 * 9 * 64;       // h8 fragments
constexpr int kTailFrag = 4 * 2 * 64;

__global__ __launch_bounds__(256) void refine_tail_kernel(
    const _Float16* __restrict__ work, const h8* __restrict__ wfrag, const float* __restrict__ rbias,
    const float* __restrict__ tbias, _Float16* __restrict__ meta, int Hq, int Wq, int batch) {
  // LDS: weight staging (44 KB) then the activation patch (reuses the same space).
  __shared__ __attribute__((aligned(16))) unsigned char smem[(kRefineFrag + kTailFrag) * 16];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  {
    const u4* srcw = reinterpret_cast<const u4*>(wfrag);
    u4* dst = reinterpret_cast<u4*>(smem);
    for (int i = threadIdx.x; i < kRefineFrag + kTailFrag; i += 256) dst[i] = srcw[i];
  }
  lds_barrier();
  h8 Ar[4][9], At[4][2];
  {
    const h8* s = reinterpret_cast<const h8*>(smem);
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int k = 0; k < 9; ++k) Ar[T][k] = s[(T * 9 + k) * 64 + lane];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int k = 0; k < 2; ++k) At[T][k] = s[kRefineFrag + (T * 2 + k) * 64 + lane];
  }
  float rb[4][4], tb[4][4];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rb[T][r] = rbias[16 * T + 4 * g + r];
      tb[T][r] = tbias[16 * T + 4 * g + r];
    }
  _Float16(*patch)[kRPW][kRPix] = reinterpret_cast<_Float16(*)[kRPW][kRPix]>(smem);

  const int tiles_x = (Wq + kRTW - 1) / kRTW, tiles_y = (Hq + kRTH - 1) / kRTH;
  const int num_tiles = batch * tiles_x * tiles_y;
  const int iters = tile_iters(num_tiles);
  for (int it = 0; it < iters; ++it) {
    const int tidx = tile_of(it, num_tiles);
    if (tidx >= num_tiles) break;
    const int b = tidx / (tiles_x * tiles_y);
    const int rem = tidx - b * tiles_x * tiles_y;
    const int y0 = (rem / tiles_x) * kRTH, x0 = (rem % tiles_x) * kRTW;
    const _Float16* in = work + (size_t)b * Hq * Wq * 32;
    lds_barrier();
    for (int q = threadIdx.x; q < kRPH * kRPW * 4; q += 256) {
      const int pix = q >> 2, ch = (q & 3) * 8;
      const int ly = pix / kRPW, lx = pix - ly * kRPW;
      const int gy = y0 + ly - 1, gx = x0 + lx - 1;
      u4 v = {0u, 0u, 0u, 0u};
      if (gy >= 0 && gy < Hq && gx >= 0 && gx < Wq)
        v = *reinterpret_cast<const u4*>(in + ((size_t)gy * Wq + gx) * 32 + ch);
      *reinterpret_cast<u4*>(&patch[ly][lx][ch]) = v;
    }
    lds_barrier();
    const int yq = y0 + wave;
    if (yq >= Hq) continue;
#pragma unroll
    for (int j = 0; j < kRTW / 16; ++j) {
      f4 acc[4];
#pragma unroll
      for (int T = 0; T < 4; ++T) acc[T] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const h8 bop = *reinterpret_cast<const h8*>(&patch[wave + k / 3][16 * j + n + k % 3][8 * g]);
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = mfma_f16(Ar[T][k], bop, acc[T]);
      }
      h8 bt[2];
#pragma unroll
      for (int T = 0; T < 4; ++T)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          bt[T >> 1][(T & 1) * 4 + r] = (_Float16)leaky(acc[T][r] + rb[T][r], 0.1f);
      f4 o[4];
#pragma unroll
      for (int T = 0; T < 4; ++T) {
        o[T] = mfma_f16(At[T][0], bt[0], f4{0.f, 0.f, 0.f, 0.f});
        o[T] = mfma_f16(At[T][1], bt[1], o[T]);
      }
      const int xq = x0 + 16 * j + n;
      if (xq < Wq) {
        _Float16* dst = meta + (((size_t)b * Hq + yq) * Wq + xq) * 64 + 4 * g;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
          u2 w;
          w[0] = pack_h2(o[T][0] + tb[T][0], o[T][1] + tb[T][1]);
          w[1] = pack_h2(o[T][2] + tb[T][2], o[T][3] + tb[T][3]);
          *reinterpret_cast<u2*>(dst + 16 * T) = w;
        }
      }
    }
  }
}

int refine_num_tiles(int batch, int Hq, int Wq) {
  return batch * ((Hq + kRTH - 1) / kRTH) * ((Wq + kRTW - 1) / kRTW);
}

hipError_t launch_refine_tail(const void* work, const void* wfrag, const float* rbias, const float* tbias,
                              void* meta, int Hq, int Wq, int batch, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(refine_tail_kernel, dim3(grid), dim3(256), 0, stream, (const _Float16*)work,
                     (const h8*)wfrag, rbias, tbias, (_Float16*)meta, Hq, Wq, batch);
  return hipGetLastError();
}

int refine_blocks_per_cu() {
  int n = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, refine_tail_kernel, 256, 0);
  return e == hipSuccess && n > 0 ? n : 1;
}

}  // namespace aeisu
