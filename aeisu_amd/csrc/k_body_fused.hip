// Fused low-resolution body: unshuffle + compress 1x1 (128 -> 64), the four grouped 3x3
// layers (2 groups of 32 -> 32) and expand 1x1 (64 -> 128) + pixel_shuffle + skip add, in one
// kernel.  The 64-channel activations of a tile never leave the CU: they ping-pong between
// two LDS buffers, and only the FP16 skip tensor is read and the FP16 work tensor written.
//
// Reference: aeisu/model.py:482-489; the Mixed deployment's per-layer kernels
// SrcPyrNativeFp8Compress.cuh:94-129,222-236, SrcPyrNativeFp8Conv.cuh:414-632,
// SrcPyrNativeFp8Expand.cuh:68-307 (one launch per layer, activations through device memory);
// INT8: optimized/shader/src/int8_kernels.cuh:2-62.
//
// Arithmetic is that of the per-layer kernels in k_body.hip (same MFMA operands and K order,
// same epilogues), so the work tensor is bit-identical to compress -> 4 x grouped -> expand.
//
// Tiling: one block per output tile of T x T low pixels.  A 3x3 layer shrinks its input
// region by one pixel per side, so compress computes the (T+8)^2 region R0, bottleneck i the
// (T+8-2i)^2 region Ri, expand the T^2 tile.  Region pixels outside the low grid hold zero:
// that is the zero padding the grouped convolutions see at the frame edge.  Regions are
// flattened and cut into 16-pixel MFMA column groups, so no MFMA work is lost to row ends.
//  * byte activations (E4M3 codes, INT8): T = 24 (252 tiles at 1080p, one per CU), 72 bytes
//    per LDS pixel; the Mixed policy widens codes to FP16 operands with
//    v_cvt_scalef32_pk_f16_fp8 as it reads them.
//  * FP16 activations: T = 16, 144 bytes per LDS pixel.
// 16 waves: compress and expand split the pixel groups over all waves; in a grouped layer,
// wave w serves group w & 1 (its 18 weight fragments stay in registers for the layer).
#include "common.hpp"
#include "kernels.hpp"

namespace aeisu {

template <int MODE>
struct BodyFusedCfg {
  static constexpr int T = MODE == 0 ? 16 : 24;     // output tile side (low pixels)
  static constexpr int PIX = MODE == 0 ? 144 : 72;  // LDS bytes per pixel: 64 channels + pad
  static constexpr int S0 = T + 8;                  // compress region side
  static constexpr int SizeA = S0 * S0 * PIX;
  static constexpr int SizeB = (S0 - 2) * (S0 - 2) * PIX;
  static constexpr int Consts = 896;                // per-channel bias/scale of all six layers
  static constexpr int Lds = SizeA + SizeB + Consts * 4;
  static constexpr int Threads = 768, Waves = Threads / 64;
  static_assert(Lds <= 160 * 1024, "fused body LDS exceeds the CU's 160 KB");
  typedef typename std::conditional<MODE == 0 || MODE == 3, h8,
                                    typename std::conditional<MODE == 1, long, i4>::type>::type Frag;
  typedef typename std::conditional<MODE == 2, i4, f4>::type Acc;
};

// LDS constant table (floats): compress bias/scale, grouped l bias/scale, expand bias/scale.
constexpr int kCstCompress = 0, kCstGrouped = 128, kCstExpand = 640;

struct BodyTileF {
  int b, y0, x0;
};

// ---- operand and epilogue helpers ---------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ typename BodyFusedCfg<MODE>::Acc mma(typename BodyFusedCfg<MODE>::Frag a,
                                                                typename BodyFusedCfg<MODE>::Frag b,
                                                                typename BodyFusedCfg<MODE>::Acc c) {
  if constexpr (MODE == 0 || MODE == 3) return mfma_f16(a, b, c);
  else if constexpr (MODE == 1) return mfma_fp8(a, b, c);
  else return mfma_i8(a, b, c);
}

// B operand of K-chunk (8 channels for f16/fp8 K = 32; 16 channels for i8 K = 64) at LDS byte
// address p; ch = first channel.
template <int MODE>
__device__ __forceinline__ typename BodyFusedCfg<MODE>::Frag lds_operand(const unsigned char* p) {
  if constexpr (MODE == 0) return *reinterpret_cast<const h8*>(p);
  else if constexpr (MODE == 1) return *reinterpret_cast<const long*>(p);
  else if constexpr (MODE == 3) {
    const u2 raw = *reinterpret_cast<const u2*>(p);
    return e4m3x8_to_h8(raw[0], raw[1]);
  } else return *reinterpret_cast<const i4*>(p);
}

// Byte offset of channel c inside an LDS pixel.
template <int MODE>
__device__ __forceinline__ int ch_off(int c) { return MODE == 0 ? 2 * c : c; }

// Epilogue of compress / bottleneck outputs for 4 consecutive channels: the value stored
// in LDS (FP16 pair of dwords, or 4 codes in one dword); 0 outside the frame.
template <int MODE>
__device__ __forceinline__ void store_act4(unsigned char* dst, typename BodyFusedCfg<MODE>::Acc acc,
                                           const float* bs, const float* sc, float inv_out, bool inside) {
  if constexpr (MODE == 0) {
    u2 w;
    w[0] = pack_h2(leaky(acc[0] + bs[0], 0.1f), leaky(acc[1] + bs[1], 0.1f));
    w[1] = pack_h2(leaky(acc[2] + bs[2], 0.1f), leaky(acc[3] + bs[3], 0.1f));
    if (!inside) w = u2{0u, 0u};
    *reinterpret_cast<u2*>(dst) = w;
  } else if constexpr (MODE == 1 || MODE == 3) {
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = leaky(fmaf(acc[r], sc[r], bs[r]), 0.1f) * inv_out;
    const unsigned w = pack_e4m3x4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<unsigned*>(dst) = inside ? w : 0u;
  } else {
    int q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = quant_s8(leaky(fmaf((float)acc[r], sc[r], bs[r]), 0.1f), inv_out);
    const unsigned w = pack_s8x4(q[0], q[1], q[2], q[3]);
    *reinterpret_cast<unsigned*>(dst) = inside ? w : 0u;
  }
}

// ---- compress: skip (HBM, FP16) -> region R0 -----------------------------------------------------
template <int MODE>
__device__ __forceinline__ void fb_compress(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst,
                                            const float* cst, int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Frag Frag;
  typedef typename C::Acc Acc;
  constexpr int S = C::S0, N = S * S, G = (N + 15) / 16;
  constexpr int NK = MODE == 2 ? 2 : 4;
  const int n = lane & 15, g = lane >> 4;
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  const _Float16* skip = P.skip + (size_t)t.b * Hq * Wq * 32;
  Frag A[4][NK];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int k = 0; k < NK; ++k) A[T][k] = reinterpret_cast<const Frag*>(P.frag[0])[(T * NK + k) * 64 + lane];
  const float inv_in = P.inv_in, inv_out = P.inv_out[0];
  for (int pg = wave; pg < G; pg += C::Waves) {
    const int q = pg * 16 + n, qc = min(q, N - 1);
    const int r = qc / S, c = qc - r * S;
    const int gy = t.y0 - 4 + r, gx = t.x0 - 4 + c;
    const bool inside = gy >= 0 && gy < P.Hl && gx >= 0 && gx < P.Wl;
    const int ly = min(max(gy, 0), P.Hl - 1), lx = min(max(gx, 0), P.Wl - 1);
    Acc acc[4] = {};
    if constexpr (MODE == 2) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int ph = 2 * k + (g >> 1);
        const _Float16* p = skip + (((size_t)2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + 16 * (g & 1);
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
    } else {
      u4 raw[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        raw[k] = *reinterpret_cast<const u4*>(skip + (((size_t)2 * ly + (k >> 1)) * Wq + 2 * lx + (k & 1)) * 32 + 8 * g);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        Frag bop;
        if constexpr (MODE == 0) {
          bop = __builtin_bit_cast(h8, raw[k]);
        } else {
          const unsigned lo = pack_e4m3x4(h2f_lo_mul(raw[k][0], inv_in), h2f_hi_mul(raw[k][0], inv_in),
                                          h2f_lo_mul(raw[k][1], inv_in), h2f_hi_mul(raw[k][1], inv_in));
          const unsigned hi = pack_e4m3x4(h2f_lo_mul(raw[k][2], inv_in), h2f_hi_mul(raw[k][2], inv_in),
                                          h2f_lo_mul(raw[k][3], inv_in), h2f_hi_mul(raw[k][3], inv_in));
          if constexpr (MODE == 1) bop = (long)(((unsigned long)hi << 32) | lo);
          else bop = e4m3x8_to_h8(lo, hi);
        }
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = mma<MODE>(A[T][k], bop, acc[T]);
      }
    }
    if (q < N) {
#pragma unroll
      for (int T = 0; T < 4; ++T) {
        const int c0 = 16 * T + 4 * g;
        const f4 bs = *reinterpret_cast<const f4*>(cst + kCstCompress + c0);
        const f4 sc = *reinterpret_cast<const f4*>(cst + kCstCompress + 64 + c0);
        const float b4[4] = {bs[0], bs[1], bs[2], bs[3]}, s4[4] = {sc[0], sc[1], sc[2], sc[3]};
        store_act4<MODE>(dst + q * C::PIX + ch_off<MODE>(c0), acc[T], b4, s4, inv_out, inside);
      }
    }
  }
}

// ---- bottleneck L (1..4): region R(L-1) -> region RL ----------------------------------------------
template <int MODE, int L>
__device__ __forceinline__ void fb_grouped(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                           unsigned char* dst, const float* cst, int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Frag Frag;
  typedef typename C::Acc Acc;
  constexpr int Sin = C::S0 - 2 * (L - 1), Sout = Sin - 2, N = Sout * Sout, G = (N + 15) / 16;
  constexpr int NK = MODE == 2 ? 5 : 9;               // K-chunks (taps; i8 packs 2 taps)
  constexpr int GW = C::Waves / 2;                     // waves per group
  const int n = lane & 15, g = lane >> 4, grp = wave & 1;
  Frag A[2][NK];
#pragma unroll
  for (int T = 0; T < 2; ++T)
#pragma unroll
    for (int k = 0; k < NK; ++k) A[T][k] = reinterpret_cast<const Frag*>(P.frag[L])[((grp * 2 + T) * NK + k) * 64 + lane];
  const float inv_out = P.inv_out[L];
  const float* cb = cst + kCstGrouped + 128 * (L - 1);
  // lane's operand byte offset inside an LDS pixel
  const int opo = MODE == 2 ? 32 * grp + 16 * (g & 1) : ch_off<MODE>(32 * grp + 8 * g);
  float bs[2][4], sc[2][4];
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    const f4 b = *reinterpret_cast<const f4*>(cb + 32 * grp + 16 * T + 4 * g);
    const f4 s4 = *reinterpret_cast<const f4*>(cb + 64 + 32 * grp + 16 * T + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bs[T][r] = b[r];
      sc[T][r] = s4[r];
    }
  }
  for (int pg = wave >> 1; pg < G; pg += GW) {
    const int q = pg * 16 + n, qc = min(q, N - 1);
    const int r = qc / Sout, c = qc - r * Sout;
    const unsigned char* base = src + (r * Sin + c) * C::PIX + opo;
    // all taps' raw operands are read before the first MFMA, so one LDS latency per item
    typedef typename std::conditional<MODE == 3, u2, Frag>::type Raw;
    Raw raw[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int tap = MODE == 2 ? min(2 * k + (g >> 1), 8) : k;
      raw[k] = *reinterpret_cast<const Raw*>(base + ((tap / 3) * Sin + tap % 3) * C::PIX);
    }
    __builtin_amdgcn_sched_barrier(0);                 // keep the reads ahead of the MFMA chain
    Acc acc[2] = {};
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      Frag bop;
      if constexpr (MODE == 3) bop = e4m3x8_to_h8(raw[k][0], raw[k][1]);
      else bop = raw[k];
#pragma unroll
      for (int T = 0; T < 2; ++T) acc[T] = mma<MODE>(A[T][k], bop, acc[T]);
    }
    if (q < N) {
      const int gy = t.y0 - 4 + L + r, gx = t.x0 - 4 + L + c;
      const bool inside = gy >= 0 && gy < P.Hl && gx >= 0 && gx < P.Wl;
#pragma unroll
      for (int T = 0; T < 2; ++T)
        store_act4<MODE>(dst + q * C::PIX + ch_off<MODE>(32 * grp + 16 * T + 4 * g), acc[T], bs[T], sc[T], inv_out,
                         inside);
    }
  }
}

// ---- expand: tile (LDS) -> work = fp16(dequant(e) + skip) (HBM) ------------------------------------
template <int MODE>
__device__ __forceinline__ void fb_expand(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                          const float* cst, int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Frag Frag;
  typedef typename C::Acc Acc;
  constexpr int S = C::T, N = S * S, G = (N + 15) / 16;
  constexpr int NK = MODE == 2 ? 1 : 2;
  const int n = lane & 15, g = lane >> 4;
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  const float inv_out = P.inv_out[5], s_out = P.s_out;
#pragma unroll
  for (int half = 0; half < 2; ++half) {               // output tiles T = 4*half .. 4*half+3
    Frag A[4][NK];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int k = 0; k < NK; ++k)
        A[j][k] = reinterpret_cast<const Frag*>(P.frag[5])[((4 * half + j) * NK + k) * 64 + lane];
    for (int pg = wave; pg < G; pg += C::Waves) {
      const int q = pg * 16 + n, qc = min(q, N - 1);
      const int r = qc / S, c = qc - r * S;
      const int ly = t.y0 + r, lx = t.x0 + c;
      Acc acc[4] = {};
#pragma unroll
      for (int k = 0; k < NK; ++k) {
        const Frag bop = lds_operand<MODE>(src + qc * C::PIX + (MODE == 2 ? 16 * g : ch_off<MODE>(32 * k + 8 * g)));
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = mma<MODE>(A[j][k], bop, acc[j]);
      }
      if (q >= N || ly >= P.Hl || lx >= P.Wl) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int T = 4 * half + j;
        const int ph = T & 3, c0 = 16 * (T >> 2) + 4 * g;
        const size_t d = ((((size_t)t.b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32) + c0;
        const f4 bs = *reinterpret_cast<const f4*>(cst + kCstExpand + 16 * T + 4 * g);
        const f4 sc = *reinterpret_cast<const f4*>(cst + kCstExpand + 128 + 16 * T + 4 * g);
        const u2 sk = *reinterpret_cast<const u2*>(P.skip + d);
        const float s[4] = {h2f_lo(sk[0]), h2f_hi(sk[0]), h2f_lo(sk[1]), h2f_hi(sk[1])};
        float v[4];
        if constexpr (MODE == 0) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) v[r4] = (float)(_Float16)leaky(acc[j][r4] + bs[r4], 0.1f) + s[r4];
        } else if constexpr (MODE == 1 || MODE == 3) {
          const unsigned qq = pack_e4m3x4(leaky(fmaf(acc[j][0], sc[0], bs[0]), 0.1f) * inv_out,
                                          leaky(fmaf(acc[j][1], sc[1], bs[1]), 0.1f) * inv_out,
                                          leaky(fmaf(acc[j][2], sc[2], bs[2]), 0.1f) * inv_out,
                                          leaky(fmaf(acc[j][3], sc[3], bs[3]), 0.1f) * inv_out);
          v[0] = fmaf(e4m3_to_f32<0>(qq), s_out, s[0]);
          v[1] = fmaf(e4m3_to_f32<1>(qq), s_out, s[1]);
          v[2] = fmaf(e4m3_to_f32<2>(qq), s_out, s[2]);
          v[3] = fmaf(e4m3_to_f32<3>(qq), s_out, s[3]);
        } else {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int qi = quant_s8(leaky(fmaf((float)acc[j][r4], sc[r4], bs[r4]), 0.1f), inv_out);
            v[r4] = fmaf((float)qi, s_out, s[r4]);
          }
        }
        u2 w;
        w[0] = pack_h2(v[0], v[1]);
        w[1] = pack_h2(v[2], v[3]);
        *reinterpret_cast<u2*>(P.work + d) = w;
      }
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(768) void body_fused_kernel(BodyFusedArgs P) {
  typedef BodyFusedCfg<MODE> C;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* bufA = smem;
  unsigned char* bufB = smem + C::SizeA;
  float* cst = reinterpret_cast<float*>(smem + C::SizeA + C::SizeB);
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  // per-channel constants -> LDS (expand's in [T][g][r] order: T = phase + 4 * channel block)
  for (int i = tid; i < C::Consts; i += C::Threads) {
    float v;
    if (i < kCstGrouped) {
      const int j = i & 63;
      v = i < 64 ? P.bias[0][j] : (MODE == 0 ? 0.f : P.scale[0][j]);
    } else if (i < kCstExpand) {
      const int l = (i - kCstGrouped) >> 7, j = (i - kCstGrouped) & 127;
      v = j < 64 ? P.bias[1 + l][j] : (MODE == 0 ? 0.f : P.scale[1 + l][j - 64]);
    } else {
      const int j = (i - kCstExpand) & 127, T = j >> 4, m = j & 15;
      const int o = (16 * (T >> 2) + m) * 4 + (T & 3);
      v = i < kCstExpand + 128 ? P.bias[5][o] : (MODE == 0 ? 0.f : P.scale[5][o]);
    }
    cst[i] = v;
  }
  const int tx = (P.Wl + C::T - 1) / C::T, ty = (P.Hl + C::T - 1) / C::T;
  BodyTileF t;
  const int tidx = blockIdx.x;
  t.b = tidx / (tx * ty);
  const int rem = tidx - t.b * tx * ty;
  t.y0 = (rem / tx) * C::T;
  t.x0 = (rem % tx) * C::T;
  __syncthreads();
  fb_compress<MODE>(P, t, bufA, cst, wave, lane);
  __syncthreads();
  fb_grouped<MODE, 1>(P, t, bufA, bufB, cst, wave, lane);
  __syncthreads();
  fb_grouped<MODE, 2>(P, t, bufB, bufA, cst, wave, lane);
  __syncthreads();
  fb_grouped<MODE, 3>(P, t, bufA, bufB, cst, wave, lane);
  __syncthreads();
  fb_grouped<MODE, 4>(P, t, bufB, bufA, cst, wave, lane);
  __syncthreads();
  fb_expand<MODE>(P, t, bufA, cst, wave, lane);
}

// ------------------------------------------------------------------------------------------------
int body_fused_num_tiles(int mode, int batch, int Hl, int Wl) {
  const int T = mode == 0 ? BodyFusedCfg<0>::T : BodyFusedCfg<3>::T;
  return batch * ((Hl + T - 1) / T) * ((Wl + T - 1) / T);
}

hipError_t body_fused_prepare() {
  const void* k[4] = {reinterpret_cast<const void*>(&body_fused_kernel<0>),
                      reinterpret_cast<const void*>(&body_fused_kernel<1>),
                      reinterpret_cast<const void*>(&body_fused_kernel<2>),
                      reinterpret_cast<const void*>(&body_fused_kernel<3>)};
  const int lds[4] = {BodyFusedCfg<0>::Lds, BodyFusedCfg<1>::Lds, BodyFusedCfg<2>::Lds, BodyFusedCfg<3>::Lds};
  for (int i = 0; i < 4; ++i) {
    const hipError_t e = hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds[i]);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_body_fused(int mode, const BodyFusedArgs& args, int batch, hipStream_t stream) {
  const int tiles = body_fused_num_tiles(mode, batch, args.Hl, args.Wl);
#define AEISU_BODY(M) \
  hipLaunchKernelGGL(body_fused_kernel<M>, dim3(tiles), dim3(BodyFusedCfg<M>::Threads), BodyFusedCfg<M>::Lds, stream, args)
  switch (mode) {
    case 0: AEISU_BODY(0); break;
    case 1: AEISU_BODY(1); break;
    case 2: AEISU_BODY(2); break;
    default: AEISU_BODY(3); break;
  }
#undef AEISU_BODY
  return hipGetLastError();
}

}  // namespace aeisu
