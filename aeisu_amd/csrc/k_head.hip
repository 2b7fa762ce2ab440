// Reconstruction head: coefficient clamp, per-pixel filter synthesis, 5x5
// RGB application, 2x phase write -- one fused pass.
//
// Math (aeisu/reconstruction.py:15-83; native ReconstructConstant,
// optimized/native/src/neural/adaptive/AdaptiveReconstruction.cuh:288-417):
//   a_k   = clamp(meta[(Y/2, X/2)][16*rho + k]),  rho = 2*(Y&1) + (X&1) on the padded grid
//   W[t,ph] = base[t,ph] + sum_k a_k * bank[t,k,ph]                (t: 25 taps, ph: 4 phases)
//   out[c, 2y + ph/2, 2x + ph%2] = clamp01( sum_t W[t,ph] * src[c, clamp(y+dy_t), clamp(x+dx_t)] )
//
// gfx950 mapping.  One wave handles 16 consecutive LR pixels of a row.
//  * Synthesis on MFMA (16x16x32 f16): D[112 x 16] = Bank^T[112 x K] . Coef[K x 16],
//    rows = tap*4 + phase (7 row tiles, taps 25..27 zero).  The FP32 bank is
//    split into FP16 hi + lo halves; two MFMAs per row tile compute
//      [K_hi | K_lo] . [a_hi ; a_hi]   and   [K_hi | base_hi, base_lo] . [a_lo ; 1, 1]
//    giving W to ~2^-22 relative accuracy with the base folded in.  a_lo is
//    non-zero only for clamped coefficients; the unclamped fast path feeds the
//    raw FP16 coefficients straight into the MFMA.
//  * Accumulator lane (n, g) holds W for pixel n, tap 4t+g, phases 0..3, so
//    each lane applies 7 taps x 4 phases x 3 channels with FP32 FMAs from an
//    LDS RGB tile; the four lane groups are summed with permlane32/16 swaps.
#include "common.hpp"

namespace aeisu {

constexpr int kHeadTW = 64, kHeadTH = 4;
constexpr int kHeadLW = kHeadTW + 4, kHeadLH = kHeadTH + 4;

template <typename Tin>
__device__ __forceinline__ float load_px(const Tin* p) { return (float)*p; }

template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void head_kernel(
    const Tin* __restrict__ src, const _Float16* __restrict__ meta, const h8* __restrict__ bankA,
    Tout* __restrict__ out, int H, int W, int Hq, int Wq, int py, int px, int batch,
    unsigned* __restrict__ nonfinite) {
  __shared__ float4 tile[kHeadLH][kHeadLW];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  h8 A1[7], A3[7];
#pragma unroll
  for (int t = 0; t < 7; ++t) {
    A1[t] = bankA[t * 64 + lane];
    A3[t] = bankA[(7 + t) * 64 + lane];
  }
  const int tiles_x = (W + kHeadTW - 1) / kHeadTW, tiles_y = (H + kHeadTH - 1) / kHeadTH;
  const int num_tiles = batch * tiles_y * tiles_x;
  const int iters = tile_iters(num_tiles);
  const size_t plane = (size_t)H * W, oplane = (size_t)4 * H * W;
  // constant B operand of the base MFMA: slots 16, 17 = 1 (lane group 2, first two halves)
  h8 bconst = {0, 0, 0, 0, 0, 0, 0, 0};
  if (g == 2) { bconst[0] = (_Float16)1.0f; bconst[1] = (_Float16)1.0f; }

  for (int it = 0; it < iters; ++it) {
    const int tidx = tile_of(it, num_tiles);
    if (tidx >= num_tiles) break;                    // block-uniform
    const int b = tidx / (tiles_y * tiles_x);
    const int rem = tidx - b * tiles_y * tiles_x;
    const int y0 = (rem / tiles_x) * kHeadTH, x0 = (rem % tiles_x) * kHeadTW;
    const Tin* s = src + (size_t)b * 3 * plane;
    __syncthreads();
    for (int q = threadIdx.x; q < kHeadLH * kHeadLW; q += 256) {
      const int ly = q / kHeadLW, lx = q - ly * kHeadLW;
      const int sy = min(max(y0 + ly - 2, 0), H - 1), sx = min(max(x0 + lx - 2, 0), W - 1);
      const size_t o = (size_t)sy * W + sx;
      tile[ly][lx] = make_float4(load_px(s + o), load_px(s + plane + o), load_px(s + 2 * plane + o), 0.f);
    }
    __syncthreads();
    const int y = y0 + wave;
    if (y >= H) continue;                              // wave-uniform
    const _Float16* mrow = meta + (size_t)b * Hq * Wq * 64;
    Tout* ob = out + (size_t)b * 3 * oplane;
#pragma unroll 1
    for (int j = 0; j < kHeadTW / 16; ++j) {
      const int x = x0 + 16 * j + n;
      if (x0 + 16 * j >= W) break;                     // wave-uniform
      const int xc = min(x, W - 1);
      const int Y = y + py, X = xc + px;
      const int rho = ((Y & 1) << 1) | (X & 1);
      const u4 raw = *reinterpret_cast<const u4*>(mrow + ((size_t)(Y >> 1) * Wq + (X >> 1)) * 64 + 16 * rho + 8 * (g & 1));
      unsigned big = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) big |= ((raw[w] & 0x7FFF7FFFu) + 0x3FFF3FFFu) & 0x80008000u;
      h8 b1, b3;
      if (__ballot(big != 0) == 0ull) {
        b1 = __builtin_bit_cast(h8, raw);
        b3 = bconst;
      } else {
        h8 hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const unsigned w = raw[i >> 1];
          const float t = (i & 1) ? h2f_hi(w) : h2f_lo(w);
          const float mag = fabsf(t);
          float c = t;
          if (mag > 2.0f) c = copysignf(fminf(2.5f, fmaf(0.05f, mag - 2.0f, 2.0f)), t);
          hi[i] = (_Float16)c;
          lo[i] = (_Float16)(c - (float)hi[i]);
        }
        b1 = hi;
        b3 = (g < 2) ? lo : bconst;
      }
      f4 acc[7];
#pragma unroll
      for (int t = 0; t < 7; ++t) {
        acc[t] = mfma_f16(A1[t], b1, f4{0.f, 0.f, 0.f, 0.f});
        acc[t] = mfma_f16(A3[t], b3, acc[t]);
      }
      float o[12];
#pragma unroll
      for (int i = 0; i < 12; ++i) o[i] = 0.f;
#pragma unroll
      for (int t = 0; t < 7; ++t) {
        const int tap = min(4 * t + g, 24);            // taps >= 25 carry zero weights
        const int dy = tap / 5, dx = tap - 5 * (tap / 5);
        const float4 L = tile[wave + dy][16 * j + n + dx];
#pragma unroll
        for (int ph = 0; ph < 4; ++ph) {
          o[0 * 4 + ph] = fmaf(acc[t][ph], L.x, o[0 * 4 + ph]);
          o[1 * 4 + ph] = fmaf(acc[t][ph], L.y, o[1 * 4 + ph]);
          o[2 * 4 + ph] = fmaf(acc[t][ph], L.z, o[2 * 4 + ph]);
        }
      }
      // Sum the four lane groups (g = lane >> 4) holding the same pixel.
      float s[6];
#pragma unroll
      for (int i = 0; i < 6; ++i) {
        float x = o[2 * i], z = o[2 * i + 1];
        permlane32_swap(x, z);
        s[i] = x + z;
      }
      float u[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        float x = s[2 * c], z = s[2 * c + 1];
        permlane16_swap(x, z);
        u[c] = x + z;
      }
      // lane row g now holds phase ph = ((g & 1) << 1) | (g >> 1) of pixel n, channels 0..2
      const int ph = ((g & 1) << 1) | (g >> 1);
      if (x < W) {
        const bool bad = !(__builtin_isfinite(u[0]) && __builtin_isfinite(u[1]) && __builtin_isfinite(u[2]));
        if (bad && nonfinite) atomicOr(nonfinite, 1u);
        const size_t o_off = (size_t)(2 * y + (ph >> 1)) * (2 * W) + 2 * x + (ph & 1);
#pragma unroll
        for (int c = 0; c < 3; ++c) ob[c * oplane + o_off] = (Tout)__builtin_amdgcn_fmed3f(u[c], 0.0f, 1.0f);
      }
    }
  }
}

template <typename Tin, typename Tout>
hipError_t launch_head_t(const void* src, const void* meta, const void* bankA, void* out, int H, int W,
                         int Hq, int Wq, int py, int px, int batch, unsigned* nonfinite, int grid,
                         hipStream_t stream) {
  hipLaunchKernelGGL((head_kernel<Tin, Tout>), dim3(grid), dim3(256), 0, stream, (const Tin*)src,
                     (const _Float16*)meta, (const h8*)bankA, (Tout*)out, H, W, Hq, Wq, py, px, batch,
                     nonfinite);
  return hipGetLastError();
}

int head_num_tiles(int batch, int H, int W) {
  return batch * ((H + kHeadTH - 1) / kHeadTH) * ((W + kHeadTW - 1) / kHeadTW);
}

hipError_t launch_head(int in_fp32, int out_fp32, const void* src, const void* meta, const void* bankA,
                       void* out, int H, int W, int Hq, int Wq, int py, int px, int batch,
                       unsigned* nonfinite, int grid, hipStream_t stream) {
  if (in_fp32 && out_fp32)
    return launch_head_t<float, float>(src, meta, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, grid, stream);
  if (in_fp32)
    return launch_head_t<float, _Float16>(src, meta, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, grid, stream);
  if (out_fp32)
    return launch_head_t<_Float16, float>(src, meta, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, grid, stream);
  return launch_head_t<_Float16, _Float16>(src, meta, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, grid, stream);
}

int head_blocks_per_cu(int in_fp32, int out_fp32) {
  int n = 0;
  hipError_t e;
  if (in_fp32 && out_fp32) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<float, float>, 256, 0);
  else if (in_fp32) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<float, _Float16>, 256, 0);
  else if (out_fp32) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<_Float16, float>, 256, 0);
  else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<_Float16, _Float16>, 256, 0);
  return e == hipSuccess && n > 0 ? n : 1;
}

}  // namespace aeisu
