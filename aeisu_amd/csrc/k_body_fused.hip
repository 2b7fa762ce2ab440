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
// 12 waves (3 per SIMD, up to 168 VGPRs each): compress and expand split the pixel groups over
// all waves; in a grouped layer, wave w serves group w & 1 and keeps that group's 18 weight
// fragments in registers for the layer.
//
// Latency: the layers hand over through LDS only, so the barrier between layers waits for LDS
// (lgkmcnt) and not for global loads; each wave issues the next layer's weight fragments
// before the barrier.  Compress prefetches the skip operands of its next pixel group, expand
// issues its skip loads before the MFMAs.  Blocks are mapped to tiles in XCD bands, so the
// tiles whose compress halos overlap run in the same L2.
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
  static constexpr int Lds = SizeA + SizeB + kBodyConsts * 4;
  static constexpr int Threads = 768, Waves = Threads / 64;
  static_assert(Lds <= 160 * 1024, "fused body LDS exceeds the CU's 160 KB");
  typedef typename std::conditional<MODE == 0 || MODE == 3, h8,
                                    typename std::conditional<MODE == 1, long, i4>::type>::type Frag;
  typedef typename std::conditional<MODE == 2, i4, f4>::type Acc;
  static constexpr int NKc = MODE == 2 ? 2 : 4;     // compress K-chunks
  static constexpr int NKg = MODE == 2 ? 5 : 9;     // grouped K-chunks (taps; i8 packs 2 taps)
  static constexpr int NKe = MODE == 2 ? 1 : 2;     // expand K-chunks
};

// LDS constant table (floats), filled from BodyFusedArgs::consts.
constexpr int kCstCompress = 0, kCstGrouped = 128, kCstExpand = 640;

struct BodyTileF {
  int b, y0, x0;
};

template <int MODE, int N>
struct FragSet {
  typename BodyFusedCfg<MODE>::Frag f[N];
};
template <int MODE, int N>
__device__ __forceinline__ FragSet<MODE, N> load_frags(const void* base, int first, int lane) {
  FragSet<MODE, N> r;
#pragma unroll
  for (int i = 0; i < N; ++i) r.f[i] = reinterpret_cast<const typename BodyFusedCfg<MODE>::Frag*>(base)[(first + i) * 64 + lane];
  return r;
}

// ---- operand and epilogue helpers ---------------------------------------------------------------
template <int MODE>
__device__ __forceinline__ typename BodyFusedCfg<MODE>::Acc mma(typename BodyFusedCfg<MODE>::Frag a,
                                                                typename BodyFusedCfg<MODE>::Frag b,
                                                                typename BodyFusedCfg<MODE>::Acc c) {
  if constexpr (MODE == 0 || MODE == 3) return mfma_f16(a, b, c);
  else if constexpr (MODE == 1) return mfma_fp8(a, b, c);
  else return mfma_i8(a, b, c);
}

// Byte offset of channel c inside an LDS pixel.
template <int MODE>
__device__ __forceinline__ int ch_off(int c) { return MODE == 0 ? 2 * c : c; }

// Raw LDS operand (E4M3 codes stay bytes until the MFMA needs them) and its MFMA form.
template <int MODE>
using RawOp = typename std::conditional<MODE == 3, u2, typename BodyFusedCfg<MODE>::Frag>::type;
template <int MODE>
__device__ __forceinline__ typename BodyFusedCfg<MODE>::Frag widen(RawOp<MODE> r) {
  if constexpr (MODE == 3) return e4m3x8_to_h8(r[0], r[1]);
  else return r;
}

// Epilogue of compress / bottleneck outputs, split in two so the per-value part can be spread
// between MFMAs: act_value is the FP32 value before packing (the per-layer kernels' arithmetic:
// FP16 leaky(acc + b); E4M3 leaky(fmaf(acc, s, b)) * (1/s_out); INT8 the same, rounded half to
// even), pack_store writes 4 consecutive channels to LDS (0 outside the frame).
template <int MODE>
__device__ __forceinline__ float act_value(typename BodyFusedCfg<MODE>::Acc acc, int r, float bs, float sc,
                                           float inv_out) {
  if constexpr (MODE == 0) return leaky(acc[r] + bs, 0.1f);
  else if constexpr (MODE == 1 || MODE == 3) return leaky(fmaf(acc[r], sc, bs), 0.1f) * inv_out;
  else return __builtin_rintf(leaky(fmaf((float)acc[r], sc, bs), 0.1f) * inv_out);
}
template <int MODE>
__device__ __forceinline__ void pack_store(unsigned char* dst, const float (&v)[4], bool inside) {
  if constexpr (MODE == 0) {
    u2 w;
    w[0] = pack_h2(v[0], v[1]);
    w[1] = pack_h2(v[2], v[3]);
    if (!inside) w = u2{0u, 0u};
    *reinterpret_cast<u2*>(dst) = w;
  } else if constexpr (MODE == 1 || MODE == 3) {
    const unsigned w = pack_e4m3x4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<unsigned*>(dst) = inside ? w : 0u;
  } else {
    int q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = (int)__builtin_amdgcn_fmed3f(v[r], -127.0f, 127.0f);
    const unsigned w = pack_s8x4(q[0], q[1], q[2], q[3]);
    *reinterpret_cast<unsigned*>(dst) = inside ? w : 0u;
  }
}
template <int MODE>
__device__ __forceinline__ void store_act4(unsigned char* dst, typename BodyFusedCfg<MODE>::Acc acc, f4 bs, f4 sc,
                                           float inv_out, bool inside) {
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] = act_value<MODE>(acc, r, bs[r], sc[r], inv_out);
  pack_store<MODE>(dst, v, inside);
}

// ---- compress: skip (HBM, FP16) -> region R0 -----------------------------------------------------
// Skip operands of one 16-pixel group: 4 phases x 8 channels (f16 / fp8 slots) or, for INT8,
// 2 chunks x (2 phases x 16 channels) -- raw[2k], raw[2k+1] are the two halves of chunk k.
template <int MODE>
__device__ __forceinline__ void compress_fetch(u4 (&raw)[4], const _Float16* __restrict__ skip, BodyTileF t, int pg,
                                               int Hl, int Wl, int lane) {
  typedef BodyFusedCfg<MODE> C;
  constexpr int S = C::S0, N = S * S;
  const int n = lane & 15, g = lane >> 4, Wq = 2 * Wl;
  const int qc = min(pg * 16 + n, N - 1);
  const int r = qc / S, c = qc - r * S;
  const int ly = min(max(t.y0 - 4 + r, 0), Hl - 1), lx = min(max(t.x0 - 4 + c, 0), Wl - 1);
  if constexpr (MODE == 2) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int ph = 2 * k + (g >> 1);
      const _Float16* p = skip + (((size_t)2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + 16 * (g & 1);
      raw[2 * k] = *reinterpret_cast<const u4*>(p);
      raw[2 * k + 1] = *reinterpret_cast<const u4*>(p + 8);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      raw[k] = *reinterpret_cast<const u4*>(skip + (((size_t)2 * ly + (k >> 1)) * Wq + 2 * lx + (k & 1)) * 32 + 8 * g);
  }
}

template <int MODE>
__device__ __forceinline__ void fb_compress(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst, const float* cst,
                                            const FragSet<MODE, 4 * BodyFusedCfg<MODE>::NKc>& F, u4 (&rawN)[4],
                                            int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Frag Frag;
  typedef typename C::Acc Acc;
  constexpr int S = C::S0, N = S * S, G = (N + 15) / 16, NK = C::NKc;
  const int n = lane & 15, g = lane >> 4;
  const _Float16* skip = P.skip + (size_t)t.b * (2 * P.Hl) * (2 * P.Wl) * 32;
  const float inv_in = P.inv_in, inv_out = P.inv_out[0];
  for (int pg = wave; pg < G; pg += C::Waves) {
    u4 raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = rawN[k];
    if (pg + C::Waves < G) compress_fetch<MODE>(rawN, skip, t, pg + C::Waves, P.Hl, P.Wl, lane);
    Acc acc[4] = {};
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      Frag bop;
      if constexpr (MODE == 2) {
        const u4 r0 = raw[2 * k], r1 = raw[2 * k + 1];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          bop[w] = (int)pack_s8x4(quant_s8(h2f_lo(r0[2 * w]), inv_in), quant_s8(h2f_hi(r0[2 * w]), inv_in),
                                  quant_s8(h2f_lo(r0[2 * w + 1]), inv_in), quant_s8(h2f_hi(r0[2 * w + 1]), inv_in));
          bop[2 + w] = (int)pack_s8x4(quant_s8(h2f_lo(r1[2 * w]), inv_in), quant_s8(h2f_hi(r1[2 * w]), inv_in),
                                      quant_s8(h2f_lo(r1[2 * w + 1]), inv_in), quant_s8(h2f_hi(r1[2 * w + 1]), inv_in));
        }
      } else if constexpr (MODE == 0) {
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
      for (int T = 0; T < 4; ++T) acc[T] = mma<MODE>(F.f[T * NK + k], bop, acc[T]);
    }
    const int q = pg * 16 + n;
    if (q < N) {
      const int r = q / S, c = q - r * S;
      const int gy = t.y0 - 4 + r, gx = t.x0 - 4 + c;
      const bool inside = ((unsigned)gy < (unsigned)P.Hl) & ((unsigned)gx < (unsigned)P.Wl);   // no branch
#pragma unroll
      for (int T = 0; T < 4; ++T) {
        const int c0 = 16 * T + 4 * g;
        store_act4<MODE>(dst + q * C::PIX + ch_off<MODE>(c0), acc[T],
                         *reinterpret_cast<const f4*>(cst + kCstCompress + c0),
                         *reinterpret_cast<const f4*>(cst + kCstCompress + 64 + c0), inv_out, inside);
      }
    }
  }
}

// ---- bottleneck L (1..4): region R(L-1) -> region RL ----------------------------------------------
template <int MODE, int L>
__device__ __forceinline__ void fb_grouped(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                           unsigned char* dst, const float* cst,
                                           const FragSet<MODE, 2 * BodyFusedCfg<MODE>::NKg>& F, int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Acc Acc;
  constexpr int Sin = C::S0 - 2 * (L - 1), Sout = Sin - 2, N = Sout * Sout, G = (N + 15) / 16;
  constexpr int NK = C::NKg;
  constexpr int GW = C::Waves / 2;                     // waves per group
  const int n = lane & 15, g = lane >> 4, grp = wave & 1;
  const float inv_out = P.inv_out[L];
  const float* cb = cst + kCstGrouped + 128 * (L - 1);
  const int opo = MODE == 2 ? 32 * grp + 16 * (g & 1) : ch_off<MODE>(32 * grp + 8 * g);   // lane's operand bytes
  const int sto = ch_off<MODE>(32 * grp + 4 * g);                                        // lane's result bytes
  f4 bs[2], sc[2];
#pragma unroll
  for (int T = 0; T < 2; ++T) {
    bs[T] = *reinterpret_cast<const f4*>(cb + 32 * grp + 16 * T + 4 * g);
    sc[T] = *reinterpret_cast<const f4*>(cb + 64 + 32 * grp + 16 * T + 4 * g);
  }
  for (int pg = wave >> 1; pg < G; pg += GW) {
    // lanes past the region end compute the region's last pixel again and store the same bytes
    const int qc = min(pg * 16 + n, N - 1);
    const int r = qc / Sout, c = qc - r * Sout;
    const unsigned char* base = src + (r * Sin + c) * C::PIX + opo;
    // all taps' operands are read before the first MFMA: one LDS latency per group
    RawOp<MODE> raw[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int tap = MODE == 2 ? min(2 * k + (g >> 1), 8) : k;
      raw[k] = *reinterpret_cast<const RawOp<MODE>*>(base + ((tap / 3) * Sin + tap % 3) * C::PIX);
    }
    __builtin_amdgcn_sched_barrier(0);                 // keep the reads ahead of the MFMA chain
    Acc acc[2] = {};
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const typename C::Frag bop = widen<MODE>(raw[k]);
#pragma unroll
      for (int T = 0; T < 2; ++T) acc[T] = mma<MODE>(F.f[T * NK + k], bop, acc[T]);
    }
    const int gy = t.y0 - 4 + L + r, gx = t.x0 - 4 + L + c;
    const bool inside = ((unsigned)gy < (unsigned)P.Hl) & ((unsigned)gx < (unsigned)P.Wl);
#pragma unroll
    for (int T = 0; T < 2; ++T)
      store_act4<MODE>(dst + qc * C::PIX + sto + ch_off<MODE>(16 * T), acc[T], bs[T], sc[T], inv_out, inside);
  }
}

// ---- expand: tile (LDS) -> work = fp16(dequant(e) + skip) (HBM) ------------------------------------
// Skip / work element offset of output tile T of lane group g for low pixel (ly, lx).
__device__ __forceinline__ size_t expand_offset(int b, int ly, int lx, int T, int g, int Hq, int Wq) {
  const int ph = T & 3, c0 = 16 * (T >> 2) + 4 * g;
  return (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + c0;
}

template <int MODE>
__device__ __forceinline__ void fb_expand(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                          const float* cst, const FragSet<MODE, 8 * BodyFusedCfg<MODE>::NKe>& F,
                                          int wave, int lane) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Acc Acc;
  constexpr int S = C::T, N = S * S, G = (N + 15) / 16, NK = C::NKe;
  const int n = lane & 15, g = lane >> 4;
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  const float inv_out = P.inv_out[5], s_out = P.s_out;
  for (int pg = wave; pg < G; pg += C::Waves) {
    const int q = pg * 16 + n, qc = min(q, N - 1);
    const int r = qc / S, c = qc - r * S;
    const int ly = t.y0 + r, lx = t.x0 + c;
    const bool store = q < N && ly < P.Hl && lx < P.Wl;
    const int lyc = min(ly, P.Hl - 1), lxc = min(lx, P.Wl - 1);
    u2 sk[8];                                          // skip operands first: in flight during the MFMAs
#pragma unroll
    for (int T = 0; T < 8; ++T) sk[T] = *reinterpret_cast<const u2*>(P.skip + expand_offset(t.b, lyc, lxc, T, g, Hq, Wq));
    RawOp<MODE> raw[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k)
      raw[k] = *reinterpret_cast<const RawOp<MODE>*>(src + qc * C::PIX + (MODE == 2 ? 16 * g : ch_off<MODE>(32 * k + 8 * g)));
    Acc acc[8] = {};
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const typename C::Frag bop = widen<MODE>(raw[k]);
#pragma unroll
      for (int T = 0; T < 8; ++T) acc[T] = mma<MODE>(F.f[T * NK + k], bop, acc[T]);
    }
    if (!store) continue;
#pragma unroll
    for (int T = 0; T < 8; ++T) {
      const f4 bs = *reinterpret_cast<const f4*>(cst + kCstExpand + 16 * T + 4 * g);
      const f4 sc = *reinterpret_cast<const f4*>(cst + kCstExpand + 128 + 16 * T + 4 * g);
      const float s[4] = {h2f_lo(sk[T][0]), h2f_hi(sk[T][0]), h2f_lo(sk[T][1]), h2f_hi(sk[T][1])};
      float v[4];
      if constexpr (MODE == 0) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) v[r4] = (float)(_Float16)leaky(acc[T][r4] + bs[r4], 0.1f) + s[r4];
      } else if constexpr (MODE == 1 || MODE == 3) {
        const unsigned qq = pack_e4m3x4(leaky(fmaf(acc[T][0], sc[0], bs[0]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][1], sc[1], bs[1]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][2], sc[2], bs[2]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][3], sc[3], bs[3]), 0.1f) * inv_out);
        v[0] = fmaf(e4m3_to_f32<0>(qq), s_out, s[0]);
        v[1] = fmaf(e4m3_to_f32<1>(qq), s_out, s[1]);
        v[2] = fmaf(e4m3_to_f32<2>(qq), s_out, s[2]);
        v[3] = fmaf(e4m3_to_f32<3>(qq), s_out, s[3]);
      } else {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int qi = quant_s8(leaky(fmaf((float)acc[T][r4], sc[r4], bs[r4]), 0.1f), inv_out);
          v[r4] = fmaf((float)qi, s_out, s[r4]);
        }
      }
      u2 w;
      w[0] = pack_h2(v[0], v[1]);
      w[1] = pack_h2(v[2], v[3]);
      *reinterpret_cast<u2*>(P.work + expand_offset(t.b, ly, lx, T, g, Hq, Wq)) = w;
    }
  }
}

// Block -> tile: the hardware hands blocks to the 8 XCDs round-robin (block b on XCD b % 8),
// so XCD x runs blocks x, x + 8, ...; each XCD gets a contiguous run of tiles, and tiles whose
// compress halos overlap share its L2.  A bijection on [0, tiles).
__device__ __forceinline__ int body_tile_of(int b, int tiles) {
  const int x = b & 7;
  int start = 0;
  for (int i = 0; i < x; ++i) start += (tiles - i + 7) >> 3;
  return start + (b >> 3);
}

template <int MODE>
__global__ __launch_bounds__(BodyFusedCfg<MODE>::Threads) void body_fused_kernel(BodyFusedArgs P) {
  typedef BodyFusedCfg<MODE> C;
  constexpr int CPT = (kBodyConsts + C::Threads - 1) / C::Threads;   // constants per thread
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* bufA = smem;
  unsigned char* bufB = smem + C::SizeA;
  float* cst = reinterpret_cast<float*>(smem + C::SizeA + C::SizeB);
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int tx = (P.Wl + C::T - 1) / C::T, ty = (P.Hl + C::T - 1) / C::T;
  const int tidx = body_tile_of((int)blockIdx.x, (int)gridDim.x);
  BodyTileF t;
  t.b = tidx / (tx * ty);
  const int rem = tidx - t.b * tx * ty;
  t.y0 = (rem / tx) * C::T;
  t.x0 = (rem % tx) * C::T;
  // constants, compress weights and the first skip operands are in flight together
  float cv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * C::Threads;
    cv[j] = i < kBodyConsts ? P.consts[i] : 0.f;
  }
  const FragSet<MODE, 4 * C::NKc> Fc = load_frags<MODE, 4 * C::NKc>(P.frag[0], 0, lane);
  u4 rawN[4];
  compress_fetch<MODE>(rawN, P.skip + (size_t)t.b * (2 * P.Hl) * (2 * P.Wl) * 32, t, wave, P.Hl, P.Wl, lane);
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * C::Threads;
    if (i < kBodyConsts) cst[i] = cv[j];
  }
  lds_barrier();
  fb_compress<MODE>(P, t, bufA, cst, Fc, rawN, wave, lane);
  const int gf = (wave & 1) * 2 * C::NKg;              // this wave's group's first fragment
  const FragSet<MODE, 2 * C::NKg> F1 = load_frags<MODE, 2 * C::NKg>(P.frag[1], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 1>(P, t, bufA, bufB, cst, F1, wave, lane);
  const FragSet<MODE, 2 * C::NKg> F2 = load_frags<MODE, 2 * C::NKg>(P.frag[2], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 2>(P, t, bufB, bufA, cst, F2, wave, lane);
  const FragSet<MODE, 2 * C::NKg> F3 = load_frags<MODE, 2 * C::NKg>(P.frag[3], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 3>(P, t, bufA, bufB, cst, F3, wave, lane);
  const FragSet<MODE, 2 * C::NKg> F4 = load_frags<MODE, 2 * C::NKg>(P.frag[4], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 4>(P, t, bufB, bufA, cst, F4, wave, lane);
  const FragSet<MODE, 8 * C::NKe> Fe = load_frags<MODE, 8 * C::NKe>(P.frag[5], 0, lane);
  lds_barrier();
  fb_expand<MODE>(P, t, bufA, cst, Fe, wave, lane);
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
#define AEISU_BODY(M)                                                                                            \
  hipLaunchKernelGGL(body_fused_kernel<M>, dim3(tiles), dim3(BodyFusedCfg<M>::Threads), BodyFusedCfg<M>::Lds, \
                     stream, args)
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
