// FP32 policy: the controller and the reconstruction head in FP32 arithmetic, one kernel per stage
// (the reference's PyTorch path, aeisu/model.py:473-496 and aeisu/reconstruction.py:15-83, which
// users of aeisu/runtime.py run).  Activations stay FP32 in device memory (NHWC):
//   skip  [B][Hq][Wq][32]   project output (analysis features -> project 1x1 -> LeakyReLU)
//   low   [B][Hl][Wl][64]   compress and the four grouped 3x3 layers (ping-pong)
//   work  [B][Hq][Wq][32]   pixel_shuffle(expand) + skip
//   meta  [B][Hq][Wq][64]   refine 3x3 + LeakyReLU -> tail 1x1 (the packed coefficients)
// and the head writes the clipped 2x frame.
//
// One thread per output pixel holds all its output channels in registers and walks the input
// channels; the weights, laid out [tap][ci][co] (kernels.hpp kF32*), are read at wave-uniform
// addresses, so they come through the scalar cache and feed the FMAs as scalar operands.  Every
// product is an FP32 fmaf; the sums run over input channels (and taps) in a fixed order, which
// differs from the reference's convolution order only by FP32 rounding.
#include "common.hpp"
#include "features.hpp"
#include "kernels.hpp"

namespace aeisu {

constexpr int kF32Threads = 256;

__device__ __forceinline__ float leaky01(float v) { return v < 0.f ? v * 0.1f : v; }

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

// ---- analysis features + project 1x1 + LeakyReLU: one packed pixel per thread ---------------------
template <typename Tin>
__global__ __launch_bounds__(kF32Threads) void f32_project_kernel(const Tin* __restrict__ src, const float* __restrict__ wimg,
                                                                  float* __restrict__ skip, int H, int W, int Hq, int Wq,
                                                                  int py, int px, int batch) {
  const long idx = (long)blockIdx.x * kF32Threads + threadIdx.x;
  if (idx >= (long)batch * Hq * Wq) return;
  const int b = (int)(idx / ((long)Hq * Wq));
  const int rem = (int)(idx - (long)b * Hq * Wq);
  const int qy = rem / Wq, qx = rem - qy * Wq;
  const size_t plane = (size_t)H * W;
  const Tin* s = src + (size_t)b * 3 * plane;
  // 4x4 LR window on the padded grid (one halo pixel each side), replicate-clamped into the source
  float w[3][4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int sy = min(max(2 * qy - 1 + a - py, 0), H - 1);
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
      const int sx = min(max(2 * qx - 1 + c4 - px, 0), W - 1);
      const size_t o = (size_t)sy * W + sx;
#pragma unroll
      for (int c = 0; c < 3; ++c) w[c][a][c4] = to_f32(s[c * plane + o]);
    }
  }
  const Analysis an = analysis_from(wimg + kF32Analysis);
  float f[8][4];
  window_features(w, an, f);
  const float* wp = wimg + kF32Project;
  float acc[32];
#pragma unroll
  for (int co = 0; co < 32; ++co) acc[co] = 0.f;
#pragma unroll
  for (int ci = 0; ci < 32; ++ci) {                // input channel = feature * 4 + phase (pixel_unshuffle)
    const float x = f[ci >> 2][ci & 3];
#pragma unroll
    for (int co = 0; co < 32; ++co) acc[co] = fmaf(x, wp[ci * 32 + co], acc[co]);
  }
  float* out = skip + (size_t)idx * 32;
#pragma unroll
  for (int co = 0; co < 32; co += 4)
    *reinterpret_cast<float4*>(out + co) = make_float4(leaky01(acc[co] + wp[1024 + co]), leaky01(acc[co + 1] + wp[1025 + co]),
                                                       leaky01(acc[co + 2] + wp[1026 + co]), leaky01(acc[co + 3] + wp[1027 + co]));
}

// ---- pixel_unshuffle + compress 1x1 (128 -> 64) + LeakyReLU: one low pixel per thread ---------------
__global__ __launch_bounds__(kF32Threads) void f32_compress_kernel(const float* __restrict__ skip, const float* __restrict__ wimg,
                                                                   float* __restrict__ low, int Hl, int Wl, int batch) {
  const long idx = (long)blockIdx.x * kF32Threads + threadIdx.x;
  if (idx >= (long)batch * Hl * Wl) return;
  const int b = (int)(idx / ((long)Hl * Wl));
  const int rem = (int)(idx - (long)b * Hl * Wl);
  const int ly = rem / Wl, lx = rem - ly * Wl;
  const int Hq = 2 * Hl, Wq = 2 * Wl;
  const float* wc = wimg + kF32Compress;
  float acc[64];
#pragma unroll
  for (int co = 0; co < 64; ++co) acc[co] = 0.f;
  for (int ph = 0; ph < 4; ++ph) {                 // unshuffled input channel = skip channel * 4 + phase
    const float* in = skip + (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32;
    for (int c0 = 0; c0 < 32; c0 += 4) {
      const float4 x4 = *reinterpret_cast<const float4*>(in + c0);
      const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* wr = wc + ((c0 + e) * 4 + ph) * 64;
#pragma unroll
        for (int co = 0; co < 64; ++co) acc[co] = fmaf(xs[e], wr[co], acc[co]);
      }
    }
  }
  float* out = low + (size_t)idx * 64;
#pragma unroll
  for (int co = 0; co < 64; co += 4)
    *reinterpret_cast<float4*>(out + co) =
        make_float4(leaky01(acc[co] + wc[8192 + co]), leaky01(acc[co + 1] + wc[8193 + co]),
                    leaky01(acc[co + 2] + wc[8194 + co]), leaky01(acc[co + 3] + wc[8195 + co]));
}

// ---- grouped 3x3 (2 groups of 32 -> 32, zero padding) + LeakyReLU: a 16 x 16 tile of low pixels
// per block (one pixel per thread) and one conv group (blockIdx.y), its 18 x 18 input halo staged in
// LDS with coalesced loads (the group's 32 channels of a pixel, 36 floats apart: conflict-free
// 16-byte reads), the weight rows block-uniform (scalar loads).  Read straight from memory, each
// thread's 72 strided 16-byte loads made the layer 4x slower.
constexpr int kF32GT = 16, kF32GH = kF32GT + 2, kF32GPix = 36;
__global__ __launch_bounds__(kF32Threads) void f32_grouped_kernel(const float* __restrict__ in, const float* __restrict__ wl,
                                                                  float* __restrict__ out, int Hl, int Wl, int batch) {
  __shared__ __attribute__((aligned(16))) float tile[kF32GH * kF32GH * kF32GPix];
  const int tx_n = (Wl + kF32GT - 1) / kF32GT, ty_n = (Hl + kF32GT - 1) / kF32GT;
  const int b = (int)blockIdx.x / (tx_n * ty_n), rem = (int)blockIdx.x - b * tx_n * ty_n;
  const int y0 = (rem / tx_n) * kF32GT, x0 = (rem % tx_n) * kF32GT;
  const int grp = blockIdx.y, tid = threadIdx.x;
  // stage: 18 x 18 pixels x 8 float4 (the group's 32 channels), zero outside the low grid
  for (int i = tid; i < kF32GH * kF32GH * 8; i += kF32Threads) {
    const int pix = i >> 3, q = i & 7, py = pix / kF32GH, px = pix - py * kF32GH;
    const int y = y0 + py - 1, x = x0 + px - 1;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (y >= 0 && y < Hl && x >= 0 && x < Wl)
      v = *reinterpret_cast<const float4*>(in + (((size_t)b * Hl + y) * Wl + x) * 64 + 32 * grp + 4 * q);
    *reinterpret_cast<float4*>(&tile[pix * kF32GPix + 4 * q]) = v;
  }
  __syncthreads();
  const int ty = tid / kF32GT, tx = tid - ty * kF32GT;
  float acc[32];
#pragma unroll
  for (int o = 0; o < 32; ++o) acc[o] = 0.f;
  for (int tap = 0; tap < 9; ++tap) {
    const float* src = &tile[((ty + tap / 3) * kF32GH + tx + tap % 3) * kF32GPix];
    for (int c0 = 0; c0 < 32; c0 += 4) {
      const float4 x4 = *reinterpret_cast<const float4*>(src + c0);
      const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* wr = wl + (tap * 32 + c0 + e) * 64 + 32 * grp;
#pragma unroll
        for (int o = 0; o < 32; ++o) acc[o] = fmaf(xs[e], wr[o], acc[o]);
      }
    }
  }
  const int ly = y0 + ty, lx = x0 + tx;
  if (ly >= Hl || lx >= Wl) return;
  float* dst = out + (((size_t)b * Hl + ly) * Wl + lx) * 64 + 32 * grp;
#pragma unroll
  for (int o = 0; o < 32; o += 4)
    *reinterpret_cast<float4*>(dst + o) = make_float4(
        leaky01(acc[o] + wl[18432 + 32 * grp + o]), leaky01(acc[o + 1] + wl[18433 + 32 * grp + o]),
        leaky01(acc[o + 2] + wl[18434 + 32 * grp + o]), leaky01(acc[o + 3] + wl[18435 + 32 * grp + o]));
}

// ---- expand 1x1 (64 -> 128) + LeakyReLU, pixel_shuffle, + skip: one low pixel per thread ----------
// Expand output channel c * 4 + 2i + j goes to channel c of packed pixel (2ly + i, 2lx + j).
__global__ __launch_bounds__(kF32Threads) void f32_expand_kernel(const float* __restrict__ low, const float* __restrict__ skip,
                                                                 const float* __restrict__ wimg, float* __restrict__ work,
                                                                 int Hl, int Wl, int batch) {
  const long idx = (long)blockIdx.x * kF32Threads + threadIdx.x;
  if (idx >= (long)batch * Hl * Wl) return;
  const int b = (int)(idx / ((long)Hl * Wl));
  const int rem = (int)(idx - (long)b * Hl * Wl);
  const int ly = rem / Wl, lx = rem - ly * Wl;
  const int Hq = 2 * Hl, Wq = 2 * Wl;
  const float* we = wimg + kF32Expand;
  const float* in = low + (size_t)idx * 64;
  for (int half = 0; half < 2; ++half) {           // output channels 64 half .. 64 half + 63
    float acc[64];
#pragma unroll
    for (int co = 0; co < 64; ++co) acc[co] = 0.f;
    for (int c0 = 0; c0 < 64; c0 += 4) {
      const float4 x4 = *reinterpret_cast<const float4*>(in + c0);
      const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* wr = we + (c0 + e) * 128 + 64 * half;
#pragma unroll
        for (int co = 0; co < 64; ++co) acc[co] = fmaf(xs[e], wr[co], acc[co]);
      }
    }
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
      const size_t o = (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + 16 * half;
#pragma unroll
      for (int c = 0; c < 16; c += 4) {
        const float4 sk = *reinterpret_cast<const float4*>(skip + o + c);
        const int e0 = 4 * c + ph;                 // acc index of output channel (16 half + c) * 4 + ph
        *reinterpret_cast<float4*>(work + o + c) =
            make_float4(leaky01(acc[e0] + we[8192 + 64 * half + e0]) + sk.x,
                        leaky01(acc[e0 + 4] + we[8192 + 64 * half + e0 + 4]) + sk.y,
                        leaky01(acc[e0 + 8] + we[8192 + 64 * half + e0 + 8]) + sk.z,
                        leaky01(acc[e0 + 12] + we[8192 + 64 * half + e0 + 12]) + sk.w);
      }
    }
  }
}

// ---- refine 3x3 (32 -> 64) + LeakyReLU + tail 1x1 (64 -> 64): a 16 x 16 tile of packed pixels per
// block (one pixel per thread), its 18 x 18 input halo (32 channels, 36 floats apart) staged in LDS
// as in the grouped layers; the tail in two halves of 32 outputs (64 + 32 accumulators within 128
// VGPRs: four waves per SIMD; all 64 + 64 took 129)
__global__ __launch_bounds__(kF32Threads) void f32_refine_tail_kernel(const float* __restrict__ work,
                                                                      const float* __restrict__ wimg,
                                                                      float* __restrict__ meta, int Hq, int Wq, int batch) {
  __shared__ __attribute__((aligned(16))) float tile[kF32GH * kF32GH * kF32GPix];
  const int tx_n = (Wq + kF32GT - 1) / kF32GT, ty_n = (Hq + kF32GT - 1) / kF32GT;
  const int b = (int)blockIdx.x / (tx_n * ty_n), rem = (int)blockIdx.x - b * tx_n * ty_n;
  const int y0 = (rem / tx_n) * kF32GT, x0 = (rem % tx_n) * kF32GT;
  const int tid = threadIdx.x;
  for (int i = tid; i < kF32GH * kF32GH * 8; i += kF32Threads) {
    const int pix = i >> 3, q = i & 7, py = pix / kF32GH, px = pix - py * kF32GH;
    const int y = y0 + py - 1, x = x0 + px - 1;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (y >= 0 && y < Hq && x >= 0 && x < Wq)
      v = *reinterpret_cast<const float4*>(work + (((size_t)b * Hq + y) * Wq + x) * 32 + 4 * q);
    *reinterpret_cast<float4*>(&tile[pix * kF32GPix + 4 * q]) = v;
  }
  __syncthreads();
  const int ty = tid / kF32GT, tx = tid - ty * kF32GT;
  const float* wr = wimg + kF32Refine;
  const float* wt = wimg + kF32Tail;
  float r[64];
#pragma unroll
  for (int co = 0; co < 64; ++co) r[co] = 0.f;
  for (int tap = 0; tap < 9; ++tap) {
    const float* src = &tile[((ty + tap / 3) * kF32GH + tx + tap % 3) * kF32GPix];
    for (int c0 = 0; c0 < 32; c0 += 4) {
      const float4 x4 = *reinterpret_cast<const float4*>(src + c0);
      const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* w = wr + (tap * 32 + c0 + e) * 64;
#pragma unroll
        for (int co = 0; co < 64; ++co) r[co] = fmaf(xs[e], w[co], r[co]);
      }
    }
  }
  const int qy = y0 + ty, qx = x0 + tx;
  if (qy >= Hq || qx >= Wq) return;
#pragma unroll
  for (int ci = 0; ci < 64; ++ci) r[ci] = leaky01(r[ci] + wr[18432 + ci]);
  float* out = meta + (((size_t)b * Hq + qy) * Wq + qx) * 64;
  for (int h = 0; h < 64; h += 32) {
    float t[32];
#pragma unroll
    for (int co = 0; co < 32; ++co) t[co] = 0.f;
#pragma unroll
    for (int ci = 0; ci < 64; ++ci)
#pragma unroll
      for (int co = 0; co < 32; ++co) t[co] = fmaf(r[ci], wt[ci * 64 + h + co], t[co]);
#pragma unroll
    for (int co = 0; co < 32; co += 4)
      *reinterpret_cast<float4*>(out + h + co) = make_float4(t[co] + wt[4096 + h + co], t[co + 1] + wt[4097 + h + co],
                                                             t[co + 2] + wt[4098 + h + co], t[co + 3] + wt[4099 + h + co]);
  }
}

// ---- head: clamp, polyphase filter synthesis, 5x5 application, clip: one LR pixel per thread -------
// coefficient_clamp (aeisu/reconstruction.py:15-17) in FP32 with the reference's separate multiply
// and add; a NaN coefficient stays NaN (so does the output, which raises the non-finite flag).
__device__ __forceinline__ float clamp_coef(float a) {
#pragma clang fp contract(off)
  const float m = fabsf(a);
  if (m <= 2.f) return a;
  float v = 2.f + 0.05f * (m - 2.f);
  v = v > 2.5f ? 2.5f : v;
  return copysignf(v, a);
}
template <typename Tout>
__device__ __forceinline__ Tout from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }

template <typename Tin, typename Tout>
__global__ __launch_bounds__(kF32Threads) void f32_head_kernel(const Tin* __restrict__ src, const float* __restrict__ meta,
                                                               const float* __restrict__ wimg, Tout* __restrict__ out, int H,
                                                               int W, int Hq, int Wq, int py, int px, int batch,
                                                               unsigned* __restrict__ nonfinite) {
  const long idx = (long)blockIdx.x * kF32Threads + threadIdx.x;
  const bool live = idx < (long)batch * H * W;
  const long id = live ? idx : 0;
  const int b = (int)(id / ((long)H * W));
  const int rem = (int)(id - (long)b * H * W);
  const int y = rem / W, x = rem - y * W;
  const size_t plane = (size_t)H * W;
  const Tin* s = src + (size_t)b * 3 * plane;
  // coefficients of this LR pixel: channel 16 rho + k of its packed pixel on the padded grid
  const int Y = y + py, X = x + px, rho = ((Y & 1) << 1) | (X & 1);
  const float* mp = meta + (((size_t)b * Hq + (Y >> 1)) * Wq + (X >> 1)) * 64 + 16 * rho;
  float a[16];
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    const float4 v = *reinterpret_cast<const float4*>(mp + k);
    a[k] = clamp_coef(v.x);
    a[k + 1] = clamp_coef(v.y);
    a[k + 2] = clamp_coef(v.z);
    a[k + 3] = clamp_coef(v.w);
  }
  // 5x5 RGB window, replicate-clamped
  float L[25][3];
#pragma unroll
  for (int t = 0; t < 25; ++t) {
    const int sy = min(max(y + t / 5 - 2, 0), H - 1), sx = min(max(x + t % 5 - 2, 0), W - 1);
    const size_t o = (size_t)sy * W + sx;
#pragma unroll
    for (int c = 0; c < 3; ++c) L[t][c] = to_f32(s[c * plane + o]);
  }
  const float* base = wimg + kF32Base;     // [25][4]
  const float* basis = wimg + kF32Basis;   // [25][16][4]
  const size_t oplane = (size_t)4 * H * W;
  Tout* o = out + (size_t)b * 3 * oplane;
  float chk = 0.f;
#pragma unroll
  for (int ph = 0; ph < 4; ++ph) {
    float u[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 25; ++t) {
      float wt = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) wt = fmaf(a[k], basis[(t * 16 + k) * 4 + ph], wt);
      wt += base[t * 4 + ph];
#pragma unroll
      for (int c = 0; c < 3; ++c) u[c] = fmaf(wt, L[t][c], u[c]);
    }
    chk = fmaf(u[0] + u[1] + u[2], 0.f, chk);
    if (live) {
      const size_t op = (size_t)(2 * y + (ph >> 1)) * (2 * W) + 2 * x + (ph & 1);
#pragma unroll
      for (int c = 0; c < 3; ++c) o[c * oplane + op] = from_f32<Tout>(__builtin_amdgcn_fmed3f(u[c], 0.f, 1.f));
    }
  }
  if (nonfinite && __ballot(live && chk != chk) != 0ull && (threadIdx.x & 63) == 0) atomicOr(nonfinite, 1u);
}

// ---- launchers ---------------------------------------------------------------------------------------
static int f32_grid(long n) { return (int)((n + kF32Threads - 1) / kF32Threads); }

hipError_t launch_f32_controller(int in_fp32, const void* src, const float* wimg, float* skip, float* low0, float* low1,
                                 float* const* lows, float* work, float* meta, int H, int W, int Hq, int Wq, int py, int px,
                                 int batch, hipStream_t stream, hipEvent_t* ev) {
  const int Hl = Hq / 2, Wl = Wq / 2;
  const long packed = (long)batch * Hq * Wq, lowpx = (long)batch * Hl * Wl;
  if (in_fp32)
    hipLaunchKernelGGL(f32_project_kernel<float>, dim3(f32_grid(packed)), dim3(kF32Threads), 0, stream,
                       (const float*)src, wimg, skip, H, W, Hq, Wq, py, px, batch);
  else
    hipLaunchKernelGGL(f32_project_kernel<_Float16>, dim3(f32_grid(packed)), dim3(kF32Threads), 0, stream,
                       (const _Float16*)src, wimg, skip, H, W, Hq, Wq, py, px, batch);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[1], stream)) != hipSuccess) return e;
  // layer outputs: lows[i] when every layer is kept, else ping-pong between low0 and low1
  float* dst[5];
  for (int i = 0; i < 5; ++i) dst[i] = lows ? lows[i] : (i % 2 ? low1 : low0);
  hipLaunchKernelGGL(f32_compress_kernel, dim3(f32_grid(lowpx)), dim3(kF32Threads), 0, stream, (const float*)skip, wimg,
                     dst[0], Hl, Wl, batch);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[2], stream)) != hipSuccess) return e;
  for (int l = 0; l < 4; ++l) {
    const int gtiles = batch * ((Hl + kF32GT - 1) / kF32GT) * ((Wl + kF32GT - 1) / kF32GT);
    hipLaunchKernelGGL(f32_grouped_kernel, dim3(gtiles, 2), dim3(kF32Threads), 0, stream, (const float*)dst[l],
                       wimg + kF32Grouped + l * kF32GroupedStride, dst[l + 1], Hl, Wl, batch);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (ev && (e = hipEventRecord(ev[3], stream)) != hipSuccess) return e;
  hipLaunchKernelGGL(f32_expand_kernel, dim3(f32_grid(lowpx)), dim3(kF32Threads), 0, stream, (const float*)dst[4],
                     (const float*)skip, wimg, work, Hl, Wl, batch);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[4], stream)) != hipSuccess) return e;
  const int rtiles = batch * ((Hq + kF32GT - 1) / kF32GT) * ((Wq + kF32GT - 1) / kF32GT);
  hipLaunchKernelGGL(f32_refine_tail_kernel, dim3(rtiles), dim3(kF32Threads), 0, stream, (const float*)work,
                     wimg, meta, Hq, Wq, batch);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (ev && (e = hipEventRecord(ev[5], stream)) != hipSuccess) return e;
  return hipSuccess;
}

hipError_t launch_f32_head(int in_fp32, int out_fp32, const void* src, const float* meta, const float* wimg, void* out,
                           int H, int W, int Hq, int Wq, int py, int px, int batch, unsigned* nonfinite,
                           hipStream_t stream) {
  const int grid = f32_grid((long)batch * H * W);
#define AEISU_F32_HEAD(TI, TO)                                                                                     \
  hipLaunchKernelGGL((f32_head_kernel<TI, TO>), dim3(grid), dim3(kF32Threads), 0, stream, (const TI*)src, meta, wimg, \
                     (TO*)out, H, W, Hq, Wq, py, px, batch, nonfinite)
  if (in_fp32 && out_fp32) AEISU_F32_HEAD(float, float);
  else if (in_fp32) AEISU_F32_HEAD(float, _Float16);
  else if (out_fp32) AEISU_F32_HEAD(_Float16, float);
  else AEISU_F32_HEAD(_Float16, _Float16);
#undef AEISU_F32_HEAD
  return hipGetLastError();
}

}  // namespace aeisu
