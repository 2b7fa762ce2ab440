// Low-resolution body of the controller: unshuffle + compress 1x1 (128 -> 64),
// four grouped 3x3 layers (2 groups of 32 -> 32), expand 1x1 (64 -> 128) +
// pixel_shuffle + skip add.  Three arithmetic policies share the structure:
//
//  * FP16 : FP16 operands, FP32 accumulation, FP16 activations.
//  * FP8  : OCP E4M3 operands on the FP8 MFMA, per-channel weight scales,
//           per-tensor activation scales, epilogue
//           q = e4m3(leaky(fmaf(acc, s_in*w_scale[c], bias_fp8[c])) * (1/s_out))
//           (SrcPyrNativeFp8Compress.cuh:94-129,222-236; SrcPyrNativeFp8Conv.cuh:414-632;
//            SrcPyrNativeFp8Expand.cuh:68-307, skip add fp16(q*s_out + skip)).
//  * INT8 : symmetric INT8 on the i8 MFMA (INT32 accumulation), epilogue
//           q = clamp(rint(leaky(fmaf(acc, factor[c], bias[c])) / s_out), +-127)
//           (optimized/shader/src/int8_kernels.cuh:2-62).
//
// Reference model: aeisu/model.py:482-489.  Layer order and activation-scale
// indices: compress reads s1 writes s2, bottleneck i reads s(i+2) writes s(i+3),
// expand reads s6 writes s7 (SrcPyrCudaRuntime.cu:4397-4451, 4587-4601).
//
// Layouts: skip/work FP16 [B][2Hl][2Wl][32]; low [B][Hl][Wl][64] (FP16 or bytes).
// Operand K-orders are permuted on the host (see engine.cpp pack_*) so every
// lane reads contiguous channels:
//   compress   K-chunk kappa = unshuffle phase, slots = 32 skip channels of that phase
//   grouped    K-chunk = tap, slots = the group's 32 input channels (i8: 2 taps per chunk)
//   expand     A rows of tile T = 16 channels c (16*(T>>2)+m) of phase T&3
#include "common.hpp"

namespace aeisu {

constexpr int kGTW = 32, kGTH = 4, kGPW = kGTW + 2, kGPH = kGTH + 2;

struct BodyTile {
  int b, y0, x0;
};
__device__ __forceinline__ BodyTile grouped_tile(int tidx, int Hl, int Wl) {
  const int tx = (Wl + kGTW - 1) / kGTW, ty = (Hl + kGTH - 1) / kGTH;
  BodyTile t;
  t.b = tidx / (tx * ty);
  const int rem = tidx - t.b * tx * ty;
  t.y0 = (rem / tx) * kGTH;
  t.x0 = (rem % tx) * kGTW;
  return t;
}

// ---------------------------------------------------------------------------------------------
// compress
// ---------------------------------------------------------------------------------------------
template <int MODE>  // 0 fp16, 1 fp8, 2 int8
__global__ __launch_bounds__(256) void compress_kernel(
    const _Float16* __restrict__ skip, const void* __restrict__ wfrag, const float* __restrict__ bias,
    const float* __restrict__ scale, void* __restrict__ low, float inv_in, float inv_out, int Hl, int Wl,
    int batch) {
  const int lane = lane_id(), wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
  const int Hq = 2 * Hl, Wq = 2 * Wl;
  const int gx = (Wl + 15) / 16, num_groups = batch * Hl * gx;
  float bs[4][4], sc[4][4];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bs[T][r] = bias[16 * T + 4 * g + r];
      sc[T][r] = MODE == 0 ? 0.f : scale[16 * T + 4 * g + r];
    }
  if constexpr (MODE == 0) {
    h8 A[4][4];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int k = 0; k < 4; ++k) A[T][k] = reinterpret_cast<const h8*>(wfrag)[(T * 4 + k) * 64 + lane];
    for (int G = blockIdx.x * 4 + wave; G < num_groups; G += gridDim.x * 4) {
      const int b = G / (Hl * gx), rem = G - b * Hl * gx, ly = rem / gx, lx = (rem - ly * gx) * 16 + n;
      const int lxc = min(lx, Wl - 1);
      f4 acc[4] = {};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const h8 bop = *reinterpret_cast<const h8*>(
            skip + (((size_t)b * Hq + 2 * ly + (k >> 1)) * Wq + 2 * lxc + (k & 1)) * 32 + 8 * g);
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = mfma_f16(A[T][k], bop, acc[T]);
      }
      if (lx < Wl) {
        _Float16* dst = reinterpret_cast<_Float16*>(low) + (((size_t)b * Hl + ly) * Wl + lx) * 64 + 4 * g;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
          u2 w;
          w[0] = pack_h2(leaky(acc[T][0] + bs[T][0], 0.1f), leaky(acc[T][1] + bs[T][1], 0.1f));
          w[1] = pack_h2(leaky(acc[T][2] + bs[T][2], 0.1f), leaky(acc[T][3] + bs[T][3], 0.1f));
          *reinterpret_cast<u2*>(dst + 16 * T) = w;
        }
      }
    }
  } else if constexpr (MODE == 1 || MODE == 3) {
    // MODE 1: E4M3 operands on the FP8 MFMA.  MODE 3: the same E4M3 values widened
    // (exactly) to FP16 for the FP16 MFMA, whose FP32 accumulation is exact per product.
    typedef typename std::conditional<MODE == 1, long, h8>::type Frag;
    Frag A[4][4];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int k = 0; k < 4; ++k) A[T][k] = reinterpret_cast<const Frag*>(wfrag)[(T * 4 + k) * 64 + lane];
    for (int G = blockIdx.x * 4 + wave; G < num_groups; G += gridDim.x * 4) {
      const int b = G / (Hl * gx), rem = G - b * Hl * gx, ly = rem / gx, lx = (rem - ly * gx) * 16 + n;
      const int lxc = min(lx, Wl - 1);
      f4 acc[4] = {};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const _Float16* px = skip + (((size_t)b * Hq + 2 * ly + (k >> 1)) * Wq + 2 * lxc + (k & 1)) * 32;
        // K slot 8g + j = channel 4g + j (j < 4) or 16 + 4g + j - 4: the project accumulator order in
        // which the frame-input fused body feeds its compress (engine.cpp packs the weights so)
        const u2 a = *reinterpret_cast<const u2*>(px + 4 * g), c = *reinterpret_cast<const u2*>(px + 16 + 4 * g);
        const u4 raw = u4{a[0], a[1], c[0], c[1]};
        const unsigned lo = pack_e4m3x4(h2f_lo_mul(raw[0], inv_in), h2f_hi_mul(raw[0], inv_in),
                                        h2f_lo_mul(raw[1], inv_in), h2f_hi_mul(raw[1], inv_in));
        const unsigned hi = pack_e4m3x4(h2f_lo_mul(raw[2], inv_in), h2f_hi_mul(raw[2], inv_in),
                                        h2f_lo_mul(raw[3], inv_in), h2f_hi_mul(raw[3], inv_in));
        if constexpr (MODE == 1) {
          const long bop = (long)(((unsigned long)hi << 32) | lo);
#pragma unroll
          for (int T = 0; T < 4; ++T) acc[T] = mfma_fp8(A[T][k], bop, acc[T]);
        } else {
          const h8 bop = e4m3x8_to_h8(lo, hi);
#pragma unroll
          for (int T = 0; T < 4; ++T) acc[T] = mfma_f16(A[T][k], bop, acc[T]);
        }
      }
      if (lx < Wl) {
        unsigned char* dst = reinterpret_cast<unsigned char*>(low) + (((size_t)b * Hl + ly) * Wl + lx) * 64 + 4 * g;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = leaky(fmaf(acc[T][r], sc[T][r], bs[T][r]), 0.1f) * inv_out;
          *reinterpret_cast<unsigned*>(dst + 16 * T) = pack_e4m3x4(v[0], v[1], v[2], v[3]);
        }
      }
    }
  } else {
    i4 A[4][2];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int k = 0; k < 2; ++k) A[T][k] = reinterpret_cast<const i4*>(wfrag)[(T * 2 + k) * 64 + lane];
    for (int G = blockIdx.x * 4 + wave; G < num_groups; G += gridDim.x * 4) {
      const int b = G / (Hl * gx), rem = G - b * Hl * gx, ly = rem / gx, lx = (rem - ly * gx) * 16 + n;
      const int lxc = min(lx, Wl - 1);
      i4 acc[4] = {};
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ph = 2 * k + (g >> 1);
        const _Float16* p = skip + (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lxc + (ph & 1)) * 32 + 16 * (g & 1);
        const u4 r0 = *reinterpret_cast<const u4*>(p), r1 = *reinterpret_cast<const u4*>(p + 8);
        i4 bop;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          bop[w] = (int)pack_s8x4(quant_s8(h2f_lo(r0[2 * w]), inv_in), quant_s8(h2f_hi(r0[2 * w]), inv_in),
                                  quant_s8(h2f_lo(r0[2 * w + 1]), inv_in), quant_s8(h2f_hi(r0[2 * w + 1]), inv_in));
          bop[2 + w] = (int)pack_s8x4(quant_s8(h2f_lo(r1[2 * w]), inv_in), quant_s8(h2f_hi(r1[2 * w]), inv_in),
                                      quant_s8(h2f_lo(r1[2 * w + 1]), inv_in), quant_s8(h2f_hi(r1[2 * w + 1]), inv_in));
        }
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = mfma_i8(A[T][k], bop, acc[T]);
      }
      if (lx < Wl) {
        unsigned char* dst = reinterpret_cast<unsigned char*>(low) + (((size_t)b * Hl + ly) * Wl + lx) * 64 + 4 * g;
#pragma unroll
        for (int T = 0; T < 4; ++T) {
          int q[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) q[r] = quant_s8(leaky(fmaf((float)acc[T][r], sc[T][r], bs[T][r]), 0.1f), inv_out);
          *reinterpret_cast<unsigned*>(dst + 16 * T) = pack_s8x4(q[0], q[1], q[2], q[3]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// grouped 3x3 (2 groups of 32 -> 32), zero padding
// ---------------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void grouped_kernel(
    const void* __restrict__ in, const void* __restrict__ wfrag, const float* __restrict__ bias,
    const float* __restrict__ scale, void* __restrict__ out, float inv_out, int Hl, int Wl, int batch) {
  constexpr int ES = MODE == 0 ? 2 : 1;                  // element size in HBM
  constexpr bool H16 = MODE == 0 || MODE == 3;           // FP16 operands in LDS / on the MFMA
  constexpr int PIX = H16 ? 144 : 80;                    // LDS bytes per pixel (64 ch + pad)
  __shared__ __attribute__((aligned(16))) unsigned char patch[kGPH * kGPW * PIX];
  const int lane = lane_id(), wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
  const int grp = wave & 1, rowbase = (wave >> 1) * 2;
  float bs[2][4], sc[2][4];
#pragma unroll
  for (int T = 0; T < 2; ++T)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = 32 * grp + 16 * T + 4 * g + r;
      bs[T][r] = bias[c];
      sc[T][r] = MODE == 0 ? 0.f : scale[c];
    }
  constexpr int NK = MODE == 2 ? 5 : 9;                  // K-chunks (taps; i8 packs 2 taps)
  typedef typename std::conditional<H16, h8, typename std::conditional<MODE == 1, long, i4>::type>::type Frag;
  Frag A[2][NK];
#pragma unroll
  for (int T = 0; T < 2; ++T)
#pragma unroll
    for (int k = 0; k < NK; ++k) A[T][k] = reinterpret_cast<const Frag*>(wfrag)[((grp * 2 + T) * NK + k) * 64 + lane];

  const int tx = (Wl + kGTW - 1) / kGTW, ty = (Hl + kGTH - 1) / kGTH;
  const int num_tiles = batch * tx * ty;
  const int iters = tile_iters(num_tiles);
  constexpr int CHUNKS = 64 * ES / 16;                   // 16-byte chunks per pixel
  for (int it = 0; it < iters; ++it) {
    const int tidx = tile_of(it, num_tiles);
    if (tidx >= num_tiles) break;
    const BodyTile t = grouped_tile(tidx, Hl, Wl);
    const unsigned char* src = reinterpret_cast<const unsigned char*>(in) + (size_t)t.b * Hl * Wl * 64 * ES;
    __syncthreads();
    for (int q = threadIdx.x; q < kGPH * kGPW * CHUNKS; q += 256) {
      const int pix = q / CHUNKS, ch = q - pix * CHUNKS;
      const int ly = pix / kGPW, lx = pix - ly * kGPW;
      const int gy = t.y0 + ly - 1, gx = t.x0 + lx - 1;
      u4 v = {0u, 0u, 0u, 0u};
      if (gy >= 0 && gy < Hl && gx >= 0 && gx < Wl)
        v = *reinterpret_cast<const u4*>(src + ((size_t)gy * Wl + gx) * 64 * ES + 16 * ch);
      if constexpr (MODE == 3) {   // 16 E4M3 codes -> 16 FP16 values (32 bytes of LDS)
        *reinterpret_cast<h8*>(patch + pix * PIX + 32 * ch) = e4m3x8_to_h8(v[0], v[1]);
        *reinterpret_cast<h8*>(patch + pix * PIX + 32 * ch + 16) = e4m3x8_to_h8(v[2], v[3]);
      } else {
        *reinterpret_cast<u4*>(patch + pix * PIX + 16 * ch) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int row = rowbase + rr, ly = t.y0 + row;
      if (ly >= Hl) break;
#pragma unroll
      for (int j = 0; j < kGTW / 16; ++j) {
        const int lx = t.x0 + 16 * j + n;
        if (t.x0 + 16 * j >= Wl) break;
        typedef typename std::conditional<MODE == 2, i4, f4>::type Acc;
        Acc acc[2] = {};
#pragma unroll
        for (int k = 0; k < NK; ++k) {
          if constexpr (MODE == 2) {
            const int tap = min(2 * k + (g >> 1), 8);
            const int p = (row + tap / 3) * kGPW + 16 * j + n + tap % 3;
            const i4 bop = *reinterpret_cast<const i4*>(patch + p * PIX + 32 * grp + 16 * (g & 1));
#pragma unroll
            for (int T = 0; T < 2; ++T) acc[T] = mfma_i8(A[T][k], bop, acc[T]);
          } else {
            const int p = (row + k / 3) * kGPW + 16 * j + n + k % 3;
            if constexpr (H16) {
              const h8 bop = *reinterpret_cast<const h8*>(patch + p * PIX + 2 * (32 * grp + 8 * g));
#pragma unroll
              for (int T = 0; T < 2; ++T) acc[T] = mfma_f16(A[T][k], bop, acc[T]);
            } else {
              const long bop = *reinterpret_cast<const long*>(patch + p * PIX + 32 * grp + 8 * g);
#pragma unroll
              for (int T = 0; T < 2; ++T) acc[T] = mfma_fp8(A[T][k], bop, acc[T]);
            }
          }
        }
        if (lx < Wl) {
          const size_t pix = ((size_t)t.b * Hl + ly) * Wl + lx;
#pragma unroll
          for (int T = 0; T < 2; ++T) {
            const int c0 = 32 * grp + 16 * T + 4 * g;
            if constexpr (MODE == 0) {
              u2 w;
              w[0] = pack_h2(leaky(acc[T][0] + bs[T][0], 0.1f), leaky(acc[T][1] + bs[T][1], 0.1f));
              w[1] = pack_h2(leaky(acc[T][2] + bs[T][2], 0.1f), leaky(acc[T][3] + bs[T][3], 0.1f));
              *reinterpret_cast<u2*>(reinterpret_cast<_Float16*>(out) + pix * 64 + c0) = w;
            } else if constexpr (MODE == 1 || MODE == 3) {
              float v[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) v[r] = leaky(fmaf(acc[T][r], sc[T][r], bs[T][r]), 0.1f) * inv_out;
              *reinterpret_cast<unsigned*>(reinterpret_cast<unsigned char*>(out) + pix * 64 + c0) =
                  pack_e4m3x4(v[0], v[1], v[2], v[3]);
            } else {
              int q[4];
#pragma unroll
              for (int r = 0; r < 4; ++r)
                q[r] = quant_s8(leaky(fmaf((float)acc[T][r], sc[T][r], bs[T][r]), 0.1f), inv_out);
              *reinterpret_cast<unsigned*>(reinterpret_cast<unsigned char*>(out) + pix * 64 + c0) =
                  pack_s8x4(q[0], q[1], q[2], q[3]);
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// expand 1x1 (64 -> 128) + pixel_shuffle + skip add -> FP16 work
// ---------------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void expand_kernel(
    const void* __restrict__ low, const _Float16* __restrict__ skip, const void* __restrict__ wfrag,
    const float* __restrict__ bias, const float* __restrict__ scale, _Float16* __restrict__ work,
    float inv_out, float s_out, int Hl, int Wl, int batch) {
  const int lane = lane_id(), wave = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
  const int Hq = 2 * Hl, Wq = 2 * Wl;
  const int gx = (Wl + 15) / 16, num_groups = batch * Hl * gx;
  float bs[8][4], sc[8][4];
#pragma unroll
  for (int T = 0; T < 8; ++T)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = (16 * (T >> 2) + 4 * g + r) * 4 + (T & 3);   // expand output channel c*4 + phase
      bs[T][r] = bias[o];
      sc[T][r] = MODE == 0 ? 0.f : scale[o];
    }
  constexpr int NK = MODE == 2 ? 1 : 2;
  typedef typename std::conditional<MODE == 0 || MODE == 3, h8,
                                    typename std::conditional<MODE == 1, long, i4>::type>::type Frag;
  Frag A[8][NK];
#pragma unroll
  for (int T = 0; T < 8; ++T)
#pragma unroll
    for (int k = 0; k < NK; ++k) A[T][k] = reinterpret_cast<const Frag*>(wfrag)[(T * NK + k) * 64 + lane];
  for (int G = blockIdx.x * 4 + wave; G < num_groups; G += gridDim.x * 4) {
    const int b = G / (Hl * gx), rem = G - b * Hl * gx, ly = rem / gx, lx = (rem - ly * gx) * 16 + n;
    const int lxc = min(lx, Wl - 1);
    const size_t pix = ((size_t)b * Hl + ly) * Wl + lxc;
    typedef typename std::conditional<MODE == 2, i4, f4>::type Acc;
    Acc acc[8] = {};
    if constexpr (MODE == 0) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const h8 bop = *reinterpret_cast<const h8*>(reinterpret_cast<const _Float16*>(low) + pix * 64 + 32 * k + 8 * g);
#pragma unroll
        for (int T = 0; T < 8; ++T) acc[T] = mfma_f16(A[T][k], bop, acc[T]);
      }
    } else if constexpr (MODE == 1) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const long bop = *reinterpret_cast<const long*>(reinterpret_cast<const unsigned char*>(low) + pix * 64 + 32 * k + 8 * g);
#pragma unroll
        for (int T = 0; T < 8; ++T) acc[T] = mfma_fp8(A[T][k], bop, acc[T]);
      }
    } else if constexpr (MODE == 3) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const u2 raw = *reinterpret_cast<const u2*>(reinterpret_cast<const unsigned char*>(low) + pix * 64 + 32 * k + 8 * g);
        const h8 bop = e4m3x8_to_h8(raw[0], raw[1]);
#pragma unroll
        for (int T = 0; T < 8; ++T) acc[T] = mfma_f16(A[T][k], bop, acc[T]);
      }
    } else {
      const i4 bop = *reinterpret_cast<const i4*>(reinterpret_cast<const unsigned char*>(low) + pix * 64 + 16 * g);
#pragma unroll
      for (int T = 0; T < 8; ++T) acc[T] = mfma_i8(A[T][0], bop, acc[T]);
    }
    if (lx >= Wl) continue;
#pragma unroll
    for (int T = 0; T < 8; ++T) {
      const int ph = T & 3, c0 = 16 * (T >> 2) + 4 * g;
      const size_t dst = (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + c0;
      const u2 sk = *reinterpret_cast<const u2*>(skip + dst);
      const float s[4] = {h2f_lo(sk[0]), h2f_hi(sk[0]), h2f_lo(sk[1]), h2f_hi(sk[1])};
      float v[4];
      if constexpr (MODE == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = (float)(_Float16)leaky(acc[T][r] + bs[T][r], 0.1f);
          v[r] = e + s[r];
        }
      } else if constexpr (MODE == 1 || MODE == 3) {
        const unsigned q = pack_e4m3x4(leaky(fmaf(acc[T][0], sc[T][0], bs[T][0]), 0.1f) * inv_out,
                                       leaky(fmaf(acc[T][1], sc[T][1], bs[T][1]), 0.1f) * inv_out,
                                       leaky(fmaf(acc[T][2], sc[T][2], bs[T][2]), 0.1f) * inv_out,
                                       leaky(fmaf(acc[T][3], sc[T][3], bs[T][3]), 0.1f) * inv_out);
        v[0] = fmaf(e4m3_to_f32<0>(q), s_out, s[0]);
        v[1] = fmaf(e4m3_to_f32<1>(q), s_out, s[1]);
        v[2] = fmaf(e4m3_to_f32<2>(q), s_out, s[2]);
        v[3] = fmaf(e4m3_to_f32<3>(q), s_out, s[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int q = quant_s8(leaky(fmaf((float)acc[T][r], sc[T][r], bs[T][r]), 0.1f), inv_out);
          v[r] = fmaf((float)q, s_out, s[r]);
        }
      }
      u2 w;
      w[0] = pack_h2(v[0], v[1]);
      w[1] = pack_h2(v[2], v[3]);
      *reinterpret_cast<u2*>(work + dst) = w;
    }
  }
}

// ---------------------------------------------------------------------------------------------
int grouped_num_tiles(int batch, int Hl, int Wl) {
  return batch * ((Hl + kGTH - 1) / kGTH) * ((Wl + kGTW - 1) / kGTW);
}

hipError_t launch_compress(int mode, const void* skip, const void* wfrag, const float* bias, const float* scale,
                           void* low, float inv_in, float inv_out, int Hl, int Wl, int batch, int grid,
                           hipStream_t stream) {
#define AEISU_COMPRESS(M)                                                                                \
  hipLaunchKernelGGL(compress_kernel<M>, dim3(grid), dim3(256), 0, stream, (const _Float16*)skip, wfrag, \
                     bias, scale, low, inv_in, inv_out, Hl, Wl, batch)
  switch (mode) {
    case 0: AEISU_COMPRESS(0); break;
    case 1: AEISU_COMPRESS(1); break;
    case 2: AEISU_COMPRESS(2); break;
    default: AEISU_COMPRESS(3); break;
  }
#undef AEISU_COMPRESS
  return hipGetLastError();
}

hipError_t launch_grouped(int mode, const void* in, const void* wfrag, const float* bias, const float* scale,
                          void* out, float inv_out, int Hl, int Wl, int batch, int grid, hipStream_t stream) {
#define AEISU_GROUPED(M)                                                                                     \
  hipLaunchKernelGGL(grouped_kernel<M>, dim3(grid), dim3(256), 0, stream, in, wfrag, bias, scale, out, inv_out, \
                     Hl, Wl, batch)
  switch (mode) {
    case 0: AEISU_GROUPED(0); break;
    case 1: AEISU_GROUPED(1); break;
    case 2: AEISU_GROUPED(2); break;
    default: AEISU_GROUPED(3); break;
  }
#undef AEISU_GROUPED
  return hipGetLastError();
}

hipError_t launch_expand(int mode, const void* low, const void* skip, const void* wfrag, const float* bias,
                         const float* scale, void* work, float inv_out, float s_out, int Hl, int Wl, int batch,
                         int grid, hipStream_t stream) {
#define AEISU_EXPAND(M)                                                                                    \
  hipLaunchKernelGGL(expand_kernel<M>, dim3(grid), dim3(256), 0, stream, low, (const _Float16*)skip, wfrag, \
                     bias, scale, (_Float16*)work, inv_out, s_out, Hl, Wl, batch)
  switch (mode) {
    case 0: AEISU_EXPAND(0); break;
    case 1: AEISU_EXPAND(1); break;
    case 2: AEISU_EXPAND(2); break;
    default: AEISU_EXPAND(3); break;
  }
#undef AEISU_EXPAND
  return hipGetLastError();
}

int body_blocks_per_cu(int kind, int mode) {
  int n = 0;
  hipError_t e = hipErrorInvalidValue;
#define AEISU_OCC(K)                                                                  \
  (mode == 0   ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K<0>, 256, 0)       \
   : mode == 1 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K<1>, 256, 0)       \
   : mode == 2 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K<2>, 256, 0)       \
               : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K<3>, 256, 0))
  if (kind == 0) e = AEISU_OCC(compress_kernel);
  else if (kind == 1) e = AEISU_OCC(grouped_kernel);
  else e = AEISU_OCC(expand_kernel);
#undef AEISU_OCC
  return e == hipSuccess && n > 0 ? n : 1;
}

}  // namespace aeisu
