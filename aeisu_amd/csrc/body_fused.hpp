// Fused low-resolution body: unshuffle + compress 1x1 (128 -> 64), the four grouped 3x3
// layers (2 groups of 32 -> 32) and expand 1x1 (64 -> 128) + pixel_shuffle + skip add, in one
// kernel.  The 64-channel activations of a tile never leave the CU: they ping-pong between
// two LDS buffers; only the FP16 work tensor is written.
//
// Reference: aeisu/model.py:473-489 (analysis, project, body); the Mixed deployment's
// per-layer kernels SrcPyrCudaRuntime.cu:2360-2584 (project), SrcPyrNativeFp8Compress.cuh:
// 94-129,222-236, SrcPyrNativeFp8Conv.cuh:414-632, SrcPyrNativeFp8Expand.cuh:68-307 (one
// launch per layer, activations and the skip tensor through device memory); INT8:
// optimized/shader/src/int8_kernels.cuh:2-62.
//
// Two inputs:
//  * BodySrc::Skip (FP16 policy): the FP16 skip tensor written by project_kernel.
//  * BodySrc::Frames16 / Frames32 (Mixed, FP8-MFMA and INT8 policies): the source frames.  The kernel
//    recomputes the analysis features and the project 1x1 for every packed pixel the compress
//    halo needs, feeds the project accumulators to the compress MFMA as register operands (the
//    compress weights are packed in the project-accumulator K order), and recomputes the tile
//    centre's skip values for the expand residual, so the 35 MB (1080p) skip tensor and its
//    halo re-reads never touch device memory.  Features are those of features.hpp and the
//    project arithmetic that of project_kernel, so the skip values are bit-identical.  The
//    MFMA's FP32 sum of its 32 products depends on their order (the FP16 MFMA rarely, by one
//    ulp), so the E4M3 policies' per-layer and skip-input compress read their operands in the
//    same order.
//
// Arithmetic is that of the per-layer kernels in k_body.hip (same MFMA operands, same
// epilogues), so the work tensor is bit-identical to project -> compress -> 4 x grouped ->
// expand.
//
// Tiling: one block per output tile of T x T low pixels.  A 3x3 layer shrinks its input
// region by one pixel per side, so compress computes the (T+8)^2 region R0, bottleneck i the
// (T+8-2i)^2 region Ri, expand the T^2 tile.  Region pixels outside the low grid hold zero:
// that is the zero padding the grouped convolutions see at the frame edge.  Regions are
// flattened and cut into 16-pixel MFMA column groups, so no MFMA work is lost to row ends.
//  * byte activations (E4M3 codes, INT8): T = 24 (252 tiles at 1080p, one per CU), 72 bytes
//    per LDS pixel; the Mixed policy widens codes to FP16 operands with
//    v_cvt_scalef32_pk_f16_fp8 as it reads them.  The frame-input variants also come with
//    T = 16 for frames whose 24x24 tiles would leave CUs idle (body_fused_plan picks the tiles
//    per shape: trailing frames or right-hand columns on 16x16 tiles, in the same launch).
//  * FP16 activations: T = 16, 144 bytes per LDS pixel.
// Compress exchange (body_fused_xc_kernel, frame input): when a whole-frame launch has no more tiles
// than the device has CUs, every tile is resident at once, so a tile computes compress on its T x T
// core only and takes the 4-pixel ring of R0 from its neighbours' cores through a device-memory
// tensor (exchange_publish / exchange_wait / exchange_ring): the compress work per tile drops from (T+8)^2 to
// T^2 pixels (1080p: 64 to 36 pixel groups).  The codes are the same, so the result is too.
// 12 waves (3 per SIMD, up to 168 VGPRs each): compress and expand split the pixel groups over
// all waves; in a grouped layer, wave w serves group w & 1 and keeps that group's 18 weight
// fragments in registers for the layer.
//
// Frame input, per 16-low-pixel group (64 packed pixels, one per lane): the wave stages the
// group's RGB (6 LR rows x up to 68 columns per channel: one or two row segments when the
// group wraps a region row) in its own 5 KB LDS slice -- the slices live in the second
// activation buffer, which is free during compress and expand (T = 24), or behind the weight
// fragments where that buffer is too small for them (T = 16) -- with the next group's RGB in
// flight in registers.  Each lane computes the 32 features of one packed pixel into the slice
// (over the RGB: a wave's LDS operations execute in order), the project MFMA reads them back
// as operands, and its accumulators become the skip operands.  No workgroup barrier is needed
// inside compress or expand.
//
// Latency: the layers hand over through LDS only, so the barrier between layers waits for LDS
// (lgkmcnt) and not for global loads; each wave issues the next layer's weight fragments
// (raw buffer loads: a scalar offset per fragment, so no address has to survive in a VGPR)
// before the barrier.  The kernel must not spill: a scratch reload waits for every memory load
// issued before it, which would serialise these prefetches.  Compress prefetches the operands of its next pixel group, expand
// issues its global loads before the MFMAs.  Blocks are mapped to tiles in XCD bands, so the
// tiles whose compress halos overlap run in the same L2.
#pragma once
#include <algorithm>
#include <vector>

#include "common.hpp"
#include "features.hpp"
#include "kernels.hpp"

namespace aeisu {

constexpr int kBodySliceBytes = 64 * 40 * 2;
constexpr int kLoadDeviceScope = 16;               // buffer-load cache policy: sc1 (device scope)      // a wave's RGB stage / feature slice (frame input)

template <int MODE, int TT = (MODE == 0 ? 16 : 24)>
struct BodyFusedCfg {
  static constexpr int T = TT;                      // output tile side (low pixels)
  static constexpr int PIX = MODE == 0 ? 144 : 72;  // LDS bytes per pixel: 64 channels + pad
  static constexpr int S0 = T + 8;                  // compress region side
  static constexpr int SizeC = kBodyConsts * 4 + 48;   // constants + 10 group counters (+ pad)
  static constexpr int SizeA = S0 * S0 * PIX;
  static constexpr int SizeB = (S0 - 2) * (S0 - 2) * PIX;
  static constexpr int Lds = SizeC + SizeA + SizeB;  // layout: constants | A | B
  static constexpr int Threads = 768, Waves = Threads / 64;
  static_assert(Lds <= 160 * 1024, "fused body LDS exceeds the CU's 160 KB");
  typedef typename std::conditional<MODE == 0 || MODE == 3, h8,
                                    typename std::conditional<MODE == 1, long, i4>::type>::type Frag;
  typedef typename std::conditional<MODE == 2, i4, f4>::type Acc;
  static constexpr int NKc = MODE == 2 ? 2 : 4;     // compress K-chunks
  static constexpr int NKg = MODE == 2 ? 5 : 9;     // grouped K-chunks (taps; i8 packs 2 taps)
  static constexpr int NKe = MODE == 2 ? 1 : 2;     // expand K-chunks
  // frame input: compress, later expand, weight fragments in LDS after the second buffer
  static constexpr int FragBytes = (4 * NKc > 8 * NKe ? 4 * NKc : 8 * NKe) * 64 * (int)sizeof(Frag);
  // the waves' slices sit in the second buffer when it holds them (24x24 tiles), else behind the
  // fragments (16x16 tiles)
  static constexpr bool SlicesInB = Waves * kBodySliceBytes <= SizeB;
  static constexpr int LdsRgb = Lds + FragBytes + (SlicesInB ? 0 : Waves * kBodySliceBytes);
};

// LDS constant table (floats), filled from BodyFusedArgs::consts.
constexpr int kCstCompress = 0, kCstGrouped = 128, kCstExpand = 640, kCstProject = 896;

struct BodyTileF {
  int b, y0, x0;
};

template <int MODE, int N>
struct FragSet {
  typename BodyFusedCfg<MODE>::Frag f[N];
};
// Weight fragments are read with raw buffer loads: the fragment offset is a scalar and the
// lane offset the only VGPR, so no per-fragment 64-bit address has to stay live (or be
// spilled) between the phases that prefetch fragments and the phases that use them.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t frag_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRawBufferWord3);
}
template <typename F>
__device__ __forceinline__ F buffer_frag(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  if constexpr (sizeof(F) == 16) return __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  else return __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
template <int MODE, int N>
__device__ __forceinline__ FragSet<MODE, N> load_frags(const void* base, int first, int lane) {
  typedef typename BodyFusedCfg<MODE>::Frag F;
  const int f0 = __builtin_amdgcn_readfirstlane(first);   // wave-uniform
  const __amdgpu_buffer_rsrc_t r = frag_rsrc(base, (f0 + N) * 64 * (int)sizeof(F));
  const int voff = fresh(lane) * (int)sizeof(F);
  FragSet<MODE, N> out;
#pragma unroll
  for (int i = 0; i < N; ++i) out.f[i] = buffer_frag<F>(r, voff, (f0 + i) * 64 * (int)sizeof(F));
  return out;
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
// LDS operand of a lane.  Byte-activation pixels are 72 bytes apart, so a 16-byte operand (INT8)
// is only 8-byte aligned: it is read as two 8-byte halves (ds_read2_b64), since a 16-byte LDS read
// of an address that is not 16-byte aligned runs at a fraction of the LDS rate.
template <int MODE>
__device__ __forceinline__ RawOp<MODE> lds_operand(const unsigned char* p) {
  if constexpr (sizeof(RawOp<MODE>) == 16 && BodyFusedCfg<MODE>::PIX % 16 != 0) {
    const u2* q = reinterpret_cast<const u2*>(p);
    const u2 lo = q[0], hi = q[1];
    return __builtin_bit_cast(RawOp<MODE>, u4{lo[0], lo[1], hi[0], hi[1]});
  } else {
    return *reinterpret_cast<const RawOp<MODE>*>(p);
  }
}
template <int MODE>
__device__ __forceinline__ typename BodyFusedCfg<MODE>::Frag widen(RawOp<MODE> r) {
  if constexpr (MODE == 3) return e4m3x8_to_h8(r[0], r[1]);
  else return r;
}

// Epilogue of compress / bottleneck outputs, split in two so the per-value part can be spread
// between MFMAs: act_value is the FP32 value before packing (the per-layer kernels' arithmetic:
// FP16 leaky(acc + b); E4M3 and INT8 leaky(fmaf(acc, s, b)) * (1/s_out)), pack_store writes 4
// consecutive channels to LDS (0 outside the frame).
template <int MODE>
__device__ __forceinline__ float act_value(typename BodyFusedCfg<MODE>::Acc acc, int r, float bs, float sc,
                                           float inv_out) {
  if constexpr (MODE == 0) return leaky(acc[r] + bs, 0.1f);
  else if constexpr (MODE == 1 || MODE == 3) return leaky(fmaf(acc[r], sc, bs), 0.1f) * inv_out;
  else return leaky(fmaf((float)acc[r], sc, bs), 0.1f) * inv_out;
}
// Byte codes of 4 consecutive channels (E4M3 saturating RNE, or INT8 rounded half to even and
// clamped to +-127: quant_s8x4).
template <int MODE>
__device__ __forceinline__ unsigned pack_codes4(const float (&v)[4]) {
  static_assert(MODE != 0, "byte-activation policies");
  if constexpr (MODE == 1 || MODE == 3) return pack_e4m3x4(v[0], v[1], v[2], v[3]);
  else return quant_s8x4(v[0], v[1], v[2], v[3]);
}
template <int MODE>
__device__ __forceinline__ void pack_store(unsigned char* dst, const float (&v)[4], bool inside) {
  if constexpr (MODE == 0) {
    u2 w;
    w[0] = pack_h2(v[0], v[1]);
    w[1] = pack_h2(v[2], v[3]);
    if (!inside) w = u2{0u, 0u};
    *reinterpret_cast<u2*>(dst) = w;
  } else {
    const unsigned w = pack_codes4<MODE>(v);
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
template <int MODE, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void compress_fetch(u4 (&raw)[4], const _Float16* __restrict__ skip, BodyTileF t, int pg,
                                               int Hl, int Wl, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
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
    for (int k = 0; k < 4; ++k) {
      const _Float16* px = skip + (((size_t)2 * ly + (k >> 1)) * Wq + 2 * lx + (k & 1)) * 32;
      if constexpr (MODE == 1 || MODE == 3) {          // project accumulator order (see compress_kernel)
        const u2 a = *reinterpret_cast<const u2*>(px + 4 * g), c = *reinterpret_cast<const u2*>(px + 16 + 4 * g);
        raw[k] = u4{a[0], a[1], c[0], c[1]};
      } else {
        raw[k] = *reinterpret_cast<const u4*>(px + 8 * g);
      }
    }
  }
}

// Compress MFMAs of one 16-pixel group from its skip operands raw[] (FP16 skip values, 8 per
// u4 in the lane's K-slot order).
template <int MODE>
__device__ __forceinline__ void compress_mma(const u4 (&raw)[4], const FragSet<MODE, 4 * BodyFusedCfg<MODE>::NKc>& F,
                                             float inv_in, typename BodyFusedCfg<MODE>::Acc (&acc)[4]) {
  typedef BodyFusedCfg<MODE> C;
  typedef typename C::Frag Frag;
  constexpr int NK = C::NKc;
#pragma unroll
  for (int T = 0; T < 4; ++T) acc[T] = typename C::Acc{};
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    Frag bop;
    if constexpr (MODE == 2) {
      const u4 r0 = raw[2 * k], r1 = raw[2 * k + 1];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        bop[w] = (int)quant_s8x4(h2f_lo_mul(r0[2 * w], inv_in), h2f_hi_mul(r0[2 * w], inv_in),
                                 h2f_lo_mul(r0[2 * w + 1], inv_in), h2f_hi_mul(r0[2 * w + 1], inv_in));
        bop[2 + w] = (int)quant_s8x4(h2f_lo_mul(r1[2 * w], inv_in), h2f_hi_mul(r1[2 * w], inv_in),
                                     h2f_lo_mul(r1[2 * w + 1], inv_in), h2f_hi_mul(r1[2 * w + 1], inv_in));
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
}

// Compress epilogue of group pg of region R0 into LDS (zero outside the low grid).
template <int MODE, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void compress_store(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst, const float* cst,
                                               const typename BodyFusedCfg<MODE>::Acc (&acc)[4], int pg, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int S = C::S0, N = S * S;
  const int n = lane & 15, g = lane >> 4;
  const int q = pg * 16 + n;
  if (q < N) {
    const int r = q / S, c = q - r * S;
    const int gy = t.y0 - 4 + r, gx = t.x0 - 4 + c;
    const bool inside = ((unsigned)gy < (unsigned)P.Hl) & ((unsigned)gx < (unsigned)P.Wl);   // no branch
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      const int c0 = 16 * T + 4 * g;
      store_act4<MODE>(dst + q * C::PIX + ch_off<MODE>(c0), acc[T], *reinterpret_cast<const f4*>(cst + kCstCompress + c0),
                       *reinterpret_cast<const f4*>(cst + kCstCompress + 64 + c0), P.inv_out[0], inside);
    }
  }
}

// Compress epilogue of group pg of the T x T tile core (compress exchange): into its place in
// region R0 and, for the pixels within 4 of the core's edge that lie in the low grid, into the
// exchange tensor, from which the neighbouring tiles take their ring of R0.
template <int MODE, int TT>
__device__ __forceinline__ void compress_store_core(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst,
                                                    const float* cst, const typename BodyFusedCfg<MODE>::Acc (&acc)[4],
                                                    int pg, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  static_assert((C::T * C::T) % 16 == 0, "core groups cover whole tiles");
  const int n = lane & 15, g = lane >> 4;
  const int q = pg * 16 + n;
  const int r = q / C::T, c = q - r * C::T;
  const int gy = t.y0 + r, gx = t.x0 + c;
  const bool inside = (gy < P.Hl) & (gx < P.Wl);
  const bool border = (r < 4) | (r >= C::T - 4) | (c < 4) | (c >= C::T - 4);
  unsigned char* ld = dst + ((r + 4) * C::S0 + c + 4) * C::PIX;
  unsigned char* gd = P.xbuf + (((size_t)t.b * P.Hl + min(gy, P.Hl - 1)) * P.Wl + min(gx, P.Wl - 1)) * 64;
#pragma unroll
  for (int T = 0; T < 4; ++T) {
    const int c0 = 16 * T + 4 * g;
    const f4 bs = *reinterpret_cast<const f4*>(cst + kCstCompress + c0);
    const f4 sc = *reinterpret_cast<const f4*>(cst + kCstCompress + 64 + c0);
    float v[4];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) v[r4] = act_value<MODE>(acc[T], r4, bs[r4], sc[r4], P.inv_out[0]);
    const unsigned w = pack_codes4<MODE>(v);
    *reinterpret_cast<unsigned*>(ld + c0) = inside ? w : 0u;
    // device-scope store (sc1): written through to the device's coherence point, past this XCD's L2
    if (inside & border) __hip_atomic_store(reinterpret_cast<unsigned*>(gd + c0), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int MODE, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void fb_compress(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst, const float* cst,
                                            const FragSet<MODE, 4 * BodyFusedCfg<MODE>::NKc>& F, u4 (&rawN)[4],
                                            int wave, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int S = C::S0, N = S * S, G = (N + 15) / 16;
  const _Float16* skip = P.skip + (size_t)t.b * (2 * P.Hl) * (2 * P.Wl) * 32;
  for (int pg = wave; pg < G; pg += C::Waves) {
    u4 raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = rawN[k];
    if (pg + C::Waves < G) compress_fetch<MODE, TT>(rawN, skip, t, pg + C::Waves, P.Hl, P.Wl, lane);
    typename C::Acc acc[4];
    compress_mma<MODE>(raw, F, P.inv_in, acc);
    compress_store<MODE, TT>(P, t, dst, cst, acc, pg, lane);
  }
}

// ---- frame input: RGB staging, analysis features and project per 16-pixel group -----------------
// A group of a flattened region (side S >= 16, low-grid origin (oy, ox)) covers at most two row
// segments: m pixels of region row r from column c, then 16 - m pixels of row r + 1 from column 0.
// Its stage covers the 6 padded-LR rows 4 ly - 1 .. 4 ly + 4 of each segment's low row ly, side by
// side: segment 1 in stage columns 0 .. 4m + 1, segment 2 after it (68 columns in all).  The stage
// holds the luma of every stage pixel (kSR rows of kSW floats), computed once per LR pixel, and the
// RGB of the four middle rows, the packed pixels' own (channel-major, rows of kRW floats, stage
// column j at j + 1, so that each packed pixel's 2 x 2 RGB starts on an even float).
constexpr int kSW = 68, kSR = 6;                      // stage row width, rows
constexpr int kSPlane = kSR * kSW;                   // luma floats
constexpr int kRW = kSW + 2, kRPlane = 4 * kRW;      // RGB row width, floats per RGB channel
constexpr int kFRow = 40;                            // halves per feature row (32 + 8 pad)
constexpr int kSlice = 64 * kFRow * 2;               // bytes of a wave's slice (features >= stage)
static_assert(kSlice == kBodySliceBytes, "slice size");
static_assert((kSPlane + 3 * kRPlane) * 4 <= kSlice, "stage must fit the slice");
constexpr int kStageLoads = 3 * kSR + 3;             // per lane: column `lane` (6 rows x 3 channels)
                                                     // and one pixel of columns 64..67 (lanes < 24)

struct GroupGeom {
  int ly, lx1, lx2, m;                               // segment 1 row / first column, segment 2 first column
};
__device__ __forceinline__ GroupGeom group_geom(int oy, int ox, int S, int pg) {
  const int q0 = 16 * pg, r = q0 / S, c = q0 - r * S;
  GroupGeom gg;
  gg.ly = oy + r;
  gg.lx1 = ox + c;
  gg.lx2 = ox;
  gg.m = min(16, S - c);
  return gg;
}

// Raw staged values in flight, one 32-bit word each (FP16 frames: zero-extended).  They pass
// through an empty asm statement before stage_store reads them: packed two FP16 values per
// register, the compiler waited for the loads right after issuing them.
template <typename Tin>
struct RgbStage {
  unsigned v[kStageLoads];
  __device__ __forceinline__ void set(int e, unsigned x) { v[e] = x; }
  __device__ __forceinline__ float get(int e) const {
    if constexpr (sizeof(Tin) == 2) return (float)__builtin_bit_cast(_Float16, (unsigned short)v[e]);
    else return __builtin_bit_cast(float, v[e]);
  }
  __device__ __forceinline__ void settle() {
#pragma unroll
    for (int e = 0; e < kStageLoads; ++e) asm volatile("" : "+v"(v[e]));
  }
};
// Lane L takes stage column L (rows 0..5, value c * kSR + row) and, for L < 24, the pixel (row
// L >> 2, column 64 + (L & 3)) (values 3 kSR + c).  Loads are unconditional with clamped
// coordinates (replicate padding of aeisu/runtime.py:84), held raw, through one raw buffer per
// frame (three planes < 2^31 bytes): 32-bit offsets, the plane as a scalar offset.
__device__ __forceinline__ int stage_src_x(const GroupGeom& gg, int j, int px, int W) {
  const int seg2 = j >= 4 * gg.m + 2;
  const int X = seg2 ? 4 * gg.lx2 - 1 + (j - 4 * gg.m - 2) : 4 * gg.lx1 - 1 + j;
  return min(max(X - px, 0), W - 1);
}
template <typename Tin>
__device__ __forceinline__ unsigned stage_load(__amdgpu_buffer_rsrc_t rs, int off, int soff) {
  if constexpr (sizeof(Tin) == 2) return (unsigned)__builtin_amdgcn_raw_buffer_load_b16(rs, off, soff, 0);
  else return __builtin_amdgcn_raw_buffer_load_b32(rs, off, soff, 0);
}
template <typename Tin>
__device__ __forceinline__ void stage_fetch(RgbStage<Tin>& st, const Tin* __restrict__ frame, const GroupGeom& gg,
                                            const BodyFusedArgs& P, int lane) {
  const int plane = P.H * P.W * (int)sizeof(Tin), rowb = P.W * (int)sizeof(Tin);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<Tin*>(frame), 0, 3 * plane, kRawBufferWord3);
  {
    const int j = lane;
    const int sx = stage_src_x(gg, j, P.px, P.W) * (int)sizeof(Tin);
    const int Y0 = 4 * gg.ly - 1 + (j >= 4 * gg.m + 2 ? 4 : 0) - P.py;
#pragma unroll
    for (int row = 0; row < kSR; ++row) {
      const int o = min(max(Y0 + row, 0), P.H - 1) * rowb + sx;
#pragma unroll
      for (int c = 0; c < 3; ++c) st.set(c * kSR + row, stage_load<Tin>(rs, o, c * plane));
    }
  }
  {
    const int v = min(lane, 4 * kSR - 1), row = v >> 2, j = 64 + (v & 3);
    const int sx = stage_src_x(gg, j, P.px, P.W) * (int)sizeof(Tin);
    const int Y = 4 * gg.ly - 1 + (j >= 4 * gg.m + 2 ? 4 : 0) + row - P.py;
    const int o = min(max(Y, 0), P.H - 1) * rowb + sx;
#pragma unroll
    for (int c = 0; c < 3; ++c) st.set(3 * kSR + c, stage_load<Tin>(rs, o, c * plane));
  }
}
template <typename Tin>
__device__ __forceinline__ void stage_store(RgbStage<Tin>& st, float* stg, const Analysis& an, int lane) {
  st.settle();
  float* rgb = stg + kSPlane;
#pragma unroll
  for (int row = 0; row < kSR; ++row) {
    const float r = st.get(row), g = st.get(kSR + row), b = st.get(2 * kSR + row);
    stg[row * kSW + lane] = luma(r, g, b, an);
    if (row >= 1 && row <= 4) {
      float* d = rgb + (row - 1) * kRW + lane + 1;
      d[0] = r;
      d[kRPlane] = g;
      d[2 * kRPlane] = b;
    }
  }
  if (lane < 4 * kSR) {
    const int row = lane >> 2, j = 64 + (lane & 3);
    const float r = st.get(3 * kSR), g = st.get(3 * kSR + 1), b = st.get(3 * kSR + 2);
    stg[row * kSW + j] = luma(r, g, b, an);
    if (row >= 1 && row <= 4) {
      float* d = rgb + (row - 1) * kRW + j + 1;
      d[0] = r;
      d[kRPlane] = g;
      d[2 * kRPlane] = b;
    }
  }
}

// Features of the lane's packed pixel (phase g of low pixel n of the group) from the stage into
// feature row `lane` of the slice.  The rows overwrite the stage: every lane's stage reads were
// issued before (a wave's LDS operations execute in order).
__device__ __forceinline__ void features_to_slice(unsigned char* slice, int m, const Analysis& an, int lane) {
  const int n = lane & 15, g = lane >> 4;
  // window origin: an even stage column, so each luma row is two aligned float2 reads and each
  // RGB row of the 2 x 2 pixels one; all 14 reads are issued before the arithmetic
  const int col = 4 * n + 2 * (g & 1) + (n >= m ? 2 : 0), r0 = 2 * (g >> 1);
  const float* lp = reinterpret_cast<const float*>(slice) + r0 * kSW + col;
  const float* cp = reinterpret_cast<const float*>(slice) + kSPlane + r0 * kRW + col + 2;
  float lw[4][4], c[3][2][2];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const float2 lo = *reinterpret_cast<const float2*>(lp + a * kSW);
    const float2 hi = *reinterpret_cast<const float2*>(lp + a * kSW + 2);
    lw[a][0] = lo.x; lw[a][1] = lo.y; lw[a][2] = hi.x; lw[a][3] = hi.y;
  }
#pragma unroll
  for (int ch = 0; ch < 3; ++ch)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float2 v = *reinterpret_cast<const float2*>(cp + ch * kRPlane + i * kRW);
      c[ch][i][0] = v.x; c[ch][i][1] = v.y;
    }
  __builtin_amdgcn_sched_barrier(0);
  float f[8][4];
  luma_features(lw, c, an, f);
  h8 hi[4], lo[4];
  feature_slices<false>(f, hi, lo);
  _Float16* feat = reinterpret_cast<_Float16*>(slice);
#pragma unroll
  for (int q = 0; q < 4; ++q) *reinterpret_cast<h8*>(feat + lane * kFRow + 8 * q) = hi[q];
}

// Project 1x1 + LeakyReLU of phase k of the group (FP16 operands as in the Mixed / INT8
// deployment, project_kernel<., false>): the lane's 8 skip channels 4g..4g+3, 16+4g..16+4g+3
// of phase k of low pixel n as FP16 pairs -- the project accumulator layout, which is the
// compress operand order of the frame-input weights and the expand residual layout.
__device__ __forceinline__ u4 project_phase(const unsigned char* slice, const h8 (&pf)[2], f4 bs0, f4 bs1, int k,
                                            int lane) {
  const int n = lane & 15, g = lane >> 4;
  const h8 b = *reinterpret_cast<const h8*>(reinterpret_cast<const _Float16*>(slice) + (16 * k + n) * kFRow + 8 * g);
  const f4 a0 = mfma_f16(pf[0], b, f4{0.f, 0.f, 0.f, 0.f});
  const f4 a1 = mfma_f16(pf[1], b, f4{0.f, 0.f, 0.f, 0.f});
  u4 sk;
  sk[0] = pack_h2(leaky(a0[0] + bs0[0], 0.1f), leaky(a0[1] + bs0[1], 0.1f));
  sk[1] = pack_h2(leaky(a0[2] + bs0[2], 0.1f), leaky(a0[3] + bs0[3], 0.1f));
  sk[2] = pack_h2(leaky(a1[0] + bs1[0], 0.1f), leaky(a1[1] + bs1[1], 0.1f));
  sk[3] = pack_h2(leaky(a1[2] + bs1[2], 0.1f), leaky(a1[3] + bs1[3], 0.1f));
  return sk;
}

// Skip hand-over between the frame-input compress and expand of a tile.  Compress computes the
// skip values (the project output) of every pixel of its region, and the tile's expand needs them
// again for the core's residual.  Compress stores them for the core pixels into the block's own
// part of the work tensor -- the 64 bytes of each packed pixel, in the project accumulator layout
// (lane group g's 16 bytes at byte 16g: channels 4g..4g+3, 16+4g..16+4g+3) -- and expand reads
// them back before it overwrites the same bytes with its output (each pixel's reads precede its
// writes through the data dependence).  The cores of a launch's tiles are disjoint, so a pixel is
// written and read by one block only; its stores are complete (vmcnt(0)) before the barrier that
// ends compress, and no CU has the lines cached before (none reads them earlier in the kernel).
__device__ __forceinline__ _Float16* skip_slot(const BodyFusedArgs& P, int b, int ly, int lx, int ph, int g) {
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  return P.work + ((((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + 8 * g);
}

// Frame-input compress (quantized policies).  Per group: stage -> features -> next group's RGB
// loads issued -> per compress K-chunk, the project MFMAs of its phases (their FP16 outputs of
// core pixels kept for expand, skip_slot) and the compress MFMAs.
// CORE: the T x T core only (compress exchange), else the whole region R0.
template <int MODE, typename Tin, int TT = BodyFusedCfg<MODE>::T, bool CORE = false>
__device__ __forceinline__ void fb_compress_rgb(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst,
                                                const float* cst, const typename BodyFusedCfg<MODE>::Frag* fr,
                                                const h8 (&pf)[2], const Analysis& an, RgbStage<Tin>& stN,
                                                unsigned char* slice, int* counter, int wave, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int S = CORE ? C::T : C::S0, N = S * S, G = (N + 15) / 16, NK = C::NKc, O = CORE ? 0 : 4;
  static_assert(MODE != 0, "frame input serves the quantized policies");
  const int g = lane >> 4;
  const Tin* frame = reinterpret_cast<const Tin*>(P.frames) + (size_t)t.b * 3 * P.H * P.W;
  for (int pg = wave, next; pg < G; pg = next) {
    stage_store<Tin>(stN, reinterpret_cast<float*>(slice), an, lane);
    features_to_slice(slice, group_geom(t.y0 - O, t.x0 - O, S, pg).m, an, lane);
    next = claim_group(counter, lane);
    if (next < G) stage_fetch<Tin>(stN, frame, group_geom(t.y0 - O, t.x0 - O, S, next), P, lane);
    const f4 bs0 = *reinterpret_cast<const f4*>(cst + kCstProject + 4 * g);
    const f4 bs1 = *reinterpret_cast<const f4*>(cst + kCstProject + 16 + 4 * g);
    // the lane's low pixel; is it a core pixel of this tile inside the low grid?
    const int q = pg * 16 + (lane & 15), r = q / S, c = q - r * S;
    const int ly = t.y0 - O + r, lx = t.x0 - O + c;
    const bool keep = (q < N) & (r >= O) & (r < O + C::T) & (c >= O) & (c < O + C::T) & (ly < P.Hl) & (lx < P.Wl);
    typename C::Acc acc[4];
#pragma unroll
    for (int T = 0; T < 4; ++T) acc[T] = typename C::Acc{};
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      typename C::Frag bop;
      if constexpr (MODE == 2) {
        const u4 r0 = project_phase(slice, pf, bs0, bs1, 2 * k, lane);
        const u4 r1 = project_phase(slice, pf, bs0, bs1, 2 * k + 1, lane);
        if (keep) {
          *reinterpret_cast<u4*>(skip_slot(P, t.b, ly, lx, 2 * k, g)) = r0;
          *reinterpret_cast<u4*>(skip_slot(P, t.b, ly, lx, 2 * k + 1, g)) = r1;
        }
        const float inv_in = P.inv_in;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          bop[w] = (int)quant_s8x4(h2f_lo_mul(r0[2 * w], inv_in), h2f_hi_mul(r0[2 * w], inv_in),
                                   h2f_lo_mul(r0[2 * w + 1], inv_in), h2f_hi_mul(r0[2 * w + 1], inv_in));
          bop[2 + w] = (int)quant_s8x4(h2f_lo_mul(r1[2 * w], inv_in), h2f_hi_mul(r1[2 * w], inv_in),
                                       h2f_lo_mul(r1[2 * w + 1], inv_in), h2f_hi_mul(r1[2 * w + 1], inv_in));
        }
      } else {
        const u4 r = project_phase(slice, pf, bs0, bs1, k, lane);
        if (keep) *reinterpret_cast<u4*>(skip_slot(P, t.b, ly, lx, k, g)) = r;
        const float inv_in = P.inv_in;
        const unsigned lo = pack_e4m3x4(h2f_lo_mul(r[0], inv_in), h2f_hi_mul(r[0], inv_in), h2f_lo_mul(r[1], inv_in),
                                        h2f_hi_mul(r[1], inv_in));
        const unsigned hi = pack_e4m3x4(h2f_lo_mul(r[2], inv_in), h2f_hi_mul(r[2], inv_in), h2f_lo_mul(r[3], inv_in),
                                        h2f_hi_mul(r[3], inv_in));
        if constexpr (MODE == 1) bop = (long)(((unsigned long)hi << 32) | lo);
        else bop = e4m3x8_to_h8(lo, hi);
      }
#pragma unroll
      for (int T = 0; T < 4; ++T) acc[T] = mma<MODE>(fr[(T * NK + k) * 64 + lane], bop, acc[T]);
    }
    if constexpr (CORE) compress_store_core<MODE, TT>(P, t, dst, cst, acc, pg, lane);
    else compress_store<MODE, TT>(P, t, dst, cst, acc, pg, lane);
  }
}

// Compress exchange.  Each tile has computed compress on its core and stored the codes within 4
// pixels of the core's edge to the exchange tensor with device-scope stores (sc1: written through
// to the device's coherence point).  exchange_publish waits until this wave's stores are complete,
// and after the block barrier stores the tile's launch count to its counter (device scope);
// exchange_wait polls the up to eight neighbours' counters until they reach the same count, and
// exchange_ring then reads the 4-pixel ring of region R0 with device-scope loads (zero outside the
// low grid).  The stores are complete before the counter is written and the loads are issued after
// the counters were seen, and device-scope accesses are coherent across the XCDs' L2 caches, so no
// cache-wide writeback or invalidate is needed.  Counters only grow: a tile reads its count at the
// start of the launch (the launches before) and publishes one more, so nothing is reset between
// launches or graph replays.  Every block of the launch is resident at once (one block per CU, no
// more tiles than CUs), and the wait is bounded all the same: after P.xspins polls (none if
// P.xspins <= 0) the tile computes the ring itself, as without the exchange, so the result never
// depends on the neighbours arriving in time.
__device__ __forceinline__ void exchange_publish(const BodyFusedArgs& P, int tidx, const int* counters, int tid) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  if (tid == 0) __hip_atomic_store(P.xflags + tidx, (unsigned)counters[10], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Block-uniform: true when every neighbour published this launch's count within the poll budget.
__device__ __forceinline__ bool exchange_wait(const BodyFusedArgs& P, int tidx, int tx, int ty, int* counters,
                                              int tid, int wave, int lane) {
  if (wave == 0) {
    const unsigned target = (unsigned)counters[10];
    const int per_frame = tx * ty, rem = tidx % per_frame, tyi = rem / tx, txi = rem - tyi * tx;
    const int ny = tyi + lane / 3 - 1, nx = txi + lane % 3 - 1;
    bool late = false;
    if (lane < 9 && lane != 4 && ny >= 0 && ny < ty && nx >= 0 && nx < tx) {
      const unsigned* f = P.xflags + (tidx - rem) + ny * tx + nx;
      late = P.xspins <= 0;
      // counts wrap after 2^32 launches: compare the difference, which is -1 (behind) or 0
      for (int spin = 0; !late && (int)(__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0;
           ++spin) {
        if (spin >= P.xspins) late = true;
        else __builtin_amdgcn_s_sleep(2);
      }
    }
    const bool ready = __ballot(late) == 0ull;
    if (tid == 0) counters[11] = ready;
  }
  lds_barrier();
  return counters[11] != 0;
}
template <int MODE, int TT>
__device__ __forceinline__ void exchange_ring(const BodyFusedArgs& P, BodyTileF t, unsigned char* dst, int tid) {
  typedef BodyFusedCfg<MODE, TT> C;
  // ring pixels: 4 rows above and 4 below the core (S0 wide), 4 columns left and right of it;
  // 16-byte chunks, 4 per pixel.  Pixels outside the low grid get an offset past the frame's
  // range, which a raw buffer load returns as zero.
  constexpr int S = C::S0, T = C::T, NR = 8 * S + 8 * T, Chunks = 4 * NR;
  constexpr int PerT = (Chunks + C::Threads - 1) / C::Threads;
  const int frame_bytes = P.Hl * P.Wl * 64;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(P.xbuf + (size_t)t.b * frame_bytes, 0, frame_bytes, kRawBufferWord3);
  u4 v[PerT];
  int at[PerT];
#pragma unroll
  for (int j = 0; j < PerT; ++j) {
    const int idx = min(tid + j * C::Threads, Chunks - 1), i = idx >> 2, k = idx & 3;
    int r, c;
    if (i < 8 * S) {                                   // rows 0..3 and T+4..T+7
      const int row = i / S;
      r = row < 4 ? row : T + row;
      c = i - row * S;
    } else {                                           // columns 0..3 and T+4..T+7 of rows 4..T+3
      const int e = i - 8 * S, row = e >> 3, col = e & 7;
      r = 4 + row;
      c = col < 4 ? col : T + col;
    }
    const int gy = t.y0 - 4 + r, gx = t.x0 - 4 + c;
    const bool inside = ((unsigned)gy < (unsigned)P.Hl) & ((unsigned)gx < (unsigned)P.Wl);
    const int off = inside ? (gy * P.Wl + gx) * 64 + 16 * k : frame_bytes;
    v[j] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, kLoadDeviceScope));
    at[j] = (r * S + c) * C::PIX + 16 * k;
  }
#pragma unroll
  for (int j = 0; j < PerT; ++j) {
    if (tid + j * C::Threads < Chunks) {
      u2* d = reinterpret_cast<u2*>(dst + at[j]);      // 8-byte aligned (72-byte pixels)
      d[0] = u2{v[j][0], v[j][1]};
      d[1] = u2{v[j][2], v[j][3]};
    }
  }
}

// ---- bottleneck L (1..4): region R(L-1) -> region RL ----------------------------------------------
template <int MODE, int L, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void fb_grouped(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                           unsigned char* dst, const float* cst,
                                           const FragSet<MODE, 2 * BodyFusedCfg<MODE>::NKg>& F, int* counter, int wave,
                                           int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  typedef typename C::Acc Acc;
  constexpr int Sin = C::S0 - 2 * (L - 1), Sout = Sin - 2, N = Sout * Sout, G = (N + 15) / 16;
  constexpr int NK = C::NKg;
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
  for (int pg = wave >> 1, next; pg < G; pg = next) {
    next = claim_group(counter, lane);               // this conv group's next pixel group
    // lanes past the region end compute the region's last pixel again and store the same bytes
    const int qc = min(pg * 16 + n, N - 1);
    const int r = qc / Sout, c = qc - r * Sout;
    const unsigned char* base = src + (r * Sin + c) * C::PIX + opo;
    // all taps' operands are issued before the first MFMA (one LDS latency per group); the
    // scheduler may interleave the widening with the reads (a scheduling barrier between them
    // measured 0.3 us slower)
    RawOp<MODE> raw[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int tap = MODE == 2 ? min(2 * k + (g >> 1), 8) : k;
      raw[k] = lds_operand<MODE>(base + ((tap / 3) * Sin + tap % 3) * C::PIX);
    }
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

// Expand MFMAs of the group's LDS pixel qc.
template <int MODE, typename FragAt>
__device__ __forceinline__ void expand_mma(const unsigned char* src, int qc, FragAt F, int g,
                                           typename BodyFusedCfg<MODE>::Acc (&acc)[8]) {
  typedef BodyFusedCfg<MODE> C;
  constexpr int NK = C::NKe;
  RawOp<MODE> raw[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k)
    raw[k] = lds_operand<MODE>(src + qc * C::PIX + (MODE == 2 ? 16 * g : ch_off<MODE>(32 * k + 8 * g)));
#pragma unroll
  for (int T = 0; T < 8; ++T) acc[T] = typename C::Acc{};
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const typename C::Frag bop = widen<MODE>(raw[k]);
#pragma unroll
    for (int T = 0; T < 8; ++T) acc[T] = mma<MODE>(F(T * NK + k), bop, acc[T]);
  }
}

// work = fp16(dequant(expand output) + skip) for low pixel (ly, lx); sk[T] = the lane's four skip
// channels of output tile T.  Tile T holds phase T & 3, channels 16 (T >> 2) + 4g .. + 3 in lane
// group g; one v_permlane16_swap per register pairs tiles T and T + 4 between groups 2k and 2k + 1,
// after which group g holds 8 consecutive channels 16 (g & 1) + 8 (g >> 1) .. + 7 of phase T, and
// the four groups of a pixel store the phase's 64 bytes in one 16-byte store each (the 8-byte stores
// of the unpaired tiles write the same 33 MB at 1080p about 1.4 times slower).  Lanes of a pixel are
// all active or all inactive, so the swap never reads an inactive partner.
template <int MODE>
__device__ __forceinline__ void expand_store(const BodyFusedArgs& P, int b, int ly, int lx, const float* cst,
                                             const typename BodyFusedCfg<MODE>::Acc (&acc)[8], const u2 (&sk)[8], int g) {
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  const float inv_out = P.inv_out[5], s_out = P.s_out;
  u2 wt[8];
#pragma unroll
  for (int T = 0; T < 8; ++T) {
    const f4 bs = *reinterpret_cast<const f4*>(cst + kCstExpand + 16 * T + 4 * g);
    const f4 sc = *reinterpret_cast<const f4*>(cst + kCstExpand + 128 + 16 * T + 4 * g);
    // the FP16 skip values enter as mixed-precision addends (v_fma_mix_f32, exact widening)
    const unsigned s01 = sk[T][0], s23 = sk[T][1];
    float v[4];
    if constexpr (MODE == 0) {
      // fl32(fp16(leaky(acc + b)) + skip): both FP16 operands of one v_fma_mix_f32
      const unsigned e01 = pack_h2(leaky(acc[T][0] + bs[0], 0.1f), leaky(acc[T][1] + bs[1], 0.1f));
      const unsigned e23 = pack_h2(leaky(acc[T][2] + bs[2], 0.1f), leaky(acc[T][3] + bs[3], 0.1f));
      v[0] = add_h16_h16<false, false>(e01, s01);
      v[1] = add_h16_h16<true, true>(e01, s01);
      v[2] = add_h16_h16<false, false>(e23, s23);
      v[3] = add_h16_h16<true, true>(e23, s23);
    } else {
      float q[4];
      if constexpr (MODE == 1 || MODE == 3) {
        const unsigned qq = pack_e4m3x4(leaky(fmaf(acc[T][0], sc[0], bs[0]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][1], sc[1], bs[1]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][2], sc[2], bs[2]), 0.1f) * inv_out,
                                        leaky(fmaf(acc[T][3], sc[3], bs[3]), 0.1f) * inv_out);
        q[0] = e4m3_to_f32<0>(qq);
        q[1] = e4m3_to_f32<1>(qq);
        q[2] = e4m3_to_f32<2>(qq);
        q[3] = e4m3_to_f32<3>(qq);
      } else {
        // the INT8 code as a float: clamp(rint(x), -127, 127) = float(quant_s8)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          q[r4] = __builtin_amdgcn_fmed3f(__builtin_rintf(leaky(fmaf((float)acc[T][r4], sc[r4], bs[r4]), 0.1f) * inv_out),
                                          -127.0f, 127.0f);
      }
      v[0] = fma_h16_addend<false>(q[0], s_out, s01);
      v[1] = fma_h16_addend<true>(q[1], s_out, s01);
      v[2] = fma_h16_addend<false>(q[2], s_out, s23);
      v[3] = fma_h16_addend<true>(q[3], s_out, s23);
    }
    wt[T][0] = pack_h2(v[0], v[1]);
    wt[T][1] = pack_h2(v[2], v[3]);
  }
  const int c0 = 16 * (g & 1) + 8 * (g >> 1);
#pragma unroll
  for (int ph = 0; ph < 4; ++ph) {
    unsigned x0 = wt[ph][0], x1 = wt[ph][1], y0 = wt[ph + 4][0], y1 = wt[ph + 4][1];
    permlane16_swap_u(x0, y0);
    permlane16_swap_u(x1, y1);
    const size_t o = (((size_t)b * Hq + 2 * ly + (ph >> 1)) * Wq + 2 * lx + (ph & 1)) * 32 + c0;
    *reinterpret_cast<u4*>(P.work + o) = u4{x0, x1, y0, y1};
  }
}

template <int MODE, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void fb_expand(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                          const float* cst, const FragSet<MODE, 8 * BodyFusedCfg<MODE>::NKe>& F,
                                          int wave, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int S = C::T, N = S * S, G = (N + 15) / 16;
  const int n = lane & 15, g = lane >> 4;
  const int Hq = 2 * P.Hl, Wq = 2 * P.Wl;
  for (int pg = wave; pg < G; pg += C::Waves) {
    const int q = pg * 16 + n, qc = min(q, N - 1);
    const int r = qc / S, c = qc - r * S;
    const int ly = t.y0 + r, lx = t.x0 + c;
    const bool store = q < N && ly < P.Hl && lx < P.Wl;
    const int lyc = min(ly, P.Hl - 1), lxc = min(lx, P.Wl - 1);
    // skip operands first (in flight during the MFMAs), as 16-byte loads of the channels
    // 16 (g & 1) + 8 (g >> 1) .. + 7 of each phase, regrouped afterwards by the store's swap in
    // reverse: lane group g then holds channels 4g..4g+3 (tile T) and 16+4g.. (tile T + 4)
    u4 skr[4];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph)
      skr[ph] = *reinterpret_cast<const u4*>(
          P.skip + (((size_t)t.b * Hq + 2 * lyc + (ph >> 1)) * Wq + 2 * lxc + (ph & 1)) * 32 + 16 * (g & 1) + 8 * (g >> 1));
    typename C::Acc acc[8];
    expand_mma<MODE>(src, qc, [&](int i) { return F.f[i]; }, g, acc);
    u2 sk[8];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
      unsigned x0 = skr[ph][0], x1 = skr[ph][1], y0 = skr[ph][2], y1 = skr[ph][3];
      permlane16_swap_u(x0, y0);
      permlane16_swap_u(x1, y1);
      sk[ph] = u2{x0, x1};
      sk[ph + 4] = u2{y0, y1};
    }
    if (store) expand_store<MODE>(P, t.b, ly, lx, cst, acc, sk, g);
  }
}

// Frame-input expand: the skip residual of each core pixel is the one compress kept (skip_slot).
template <int MODE, int TT = BodyFusedCfg<MODE>::T>
__device__ __forceinline__ void fb_expand_rgb(const BodyFusedArgs& P, BodyTileF t, const unsigned char* src,
                                              const float* cst, const typename BodyFusedCfg<MODE>::Frag* fr,
                                              int* counter, int wave, int lane) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int S = C::T, N = S * S, G = (N + 15) / 16;
  static_assert(N % 16 == 0, "expand groups cover whole tiles");
  const int n = lane & 15, g = lane >> 4;
  for (int pg = wave, next; pg < G; pg = next) {
    next = claim_group(counter, lane);
    const int q = pg * 16 + n;
    const int r = q / S, c = q - r * S;
    const int ly = t.y0 + r, lx = t.x0 + c;
    const bool store = ly < P.Hl && lx < P.Wl;
    // the kept skip values first (in flight during the MFMAs); pixels past the low grid read
    // the grid's last pixel and store nothing
    const int lyc = min(ly, P.Hl - 1), lxc = min(lx, P.Wl - 1);
    u4 kept[4];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) kept[ph] = *reinterpret_cast<const u4*>(skip_slot(P, t.b, lyc, lxc, ph, g));
    typename C::Acc acc[8];
    expand_mma<MODE>(src, q, [&](int i) { return fr[i * 64 + lane]; }, g, acc);
    u2 sk[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sk[k] = u2{kept[k][0], kept[k][1]};            // output tile k: phase k, channels 4g..4g+3
      sk[k + 4] = u2{kept[k][2], kept[k][3]};        // output tile k + 4: channels 16 + 4g..
    }
    if (store) expand_store<MODE>(P, t.b, ly, lx, cst, acc, sk, g);
  }
}

// Block -> tile: the hardware hands blocks to the 8 XCDs round-robin (block g on XCD g % 8),
// so each XCD gets a contiguous run of tiles, and tiles whose compress halos overlap share its L2.
// Local block b of a launch part whose first block is `first` (global index first + b), of
// `tiles` blocks: the part's blocks on XCD x are b = f(x), f(x) + 8, ... with f(x) = (x - first)
// mod 8.  A bijection on [0, tiles).
__device__ __forceinline__ int body_tile_of(int b, int tiles, int first) {
  const int x = (first + b) & 7;
  int start = 0;
  for (int i = 0; i < x; ++i) start += (tiles - ((i - first) & 7) + 7) >> 3;
  return start + (b >> 3);
}

// One output tile (tile index tidx of the launch part described by P).
template <int MODE, int SRC, int TT, bool XC = false>
__device__ __forceinline__ void body_tile(const BodyFusedArgs& P, int tidx) {
  typedef BodyFusedCfg<MODE, TT> C;
  typedef typename std::conditional<SRC == (int)BodySrc::Frames32, float, _Float16>::type Tin;
  constexpr bool RGB = SRC != (int)BodySrc::Skip;
  static_assert(!RGB || MODE != 0, "frame input serves the quantized policies (FP16 project operands)");
  static_assert(!XC || RGB, "the compress exchange serves the frame-input body");
  constexpr int CPT = (kBodyConsts + C::Threads - 1) / C::Threads;   // constants per thread
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* cst = reinterpret_cast<float*>(smem);
  // group counters: frame-input compress, expand; then bottleneck l = 1..4, conv group 0 / 1
  int* counters = reinterpret_cast<int*>(smem + kBodyConsts * 4);
  unsigned char* bufA = smem + C::SizeC;
  unsigned char* bufB = bufA + C::SizeA;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  unsigned char* slice = (C::SlicesInB ? bufB : bufB + C::SizeB + C::FragBytes) + wave * kSlice;   // frame input
  const int tx = ((P.cols ? P.cols : P.Wl) + C::T - 1) / C::T, ty = ((P.rows ? P.rows : P.Hl) + C::T - 1) / C::T;
  BodyTileF t;
  t.b = tidx / (tx * ty);
  const int rem = tidx - t.b * tx * ty;
  t.y0 = P.row0 + (rem / tx) * C::T;
  t.x0 = P.col0 + (rem % tx) * C::T;
  // constants, compress weights and the first group's operands are in flight together
  float cv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * C::Threads;
    cv[j] = i < kBodyConsts ? P.consts[i] : 0.f;
  }
  FragSet<MODE, 4 * C::NKc> Fc;
  if constexpr (!RGB) Fc = load_frags<MODE, 4 * C::NKc>(P.frag[0], 0, lane);
  // frame input: weight fragments of compress, then expand, in LDS (registers go to the
  // feature and project work); the block copies them in 16-byte chunks
  static_assert(!RGB || C::LdsRgb <= 160 * 1024, "frame-input body LDS exceeds the CU's 160 KB");
  constexpr int FragChunks = C::FragBytes / 16, FCPT = (FragChunks + C::Threads - 1) / C::Threads;
  u4* fr_lds = reinterpret_cast<u4*>(bufB + C::SizeB);
  const typename C::Frag* fr = reinterpret_cast<const typename C::Frag*>(fr_lds);
  u4 fchunk[FCPT];
  if constexpr (RGB) {                                 // chunks past the end read as zero
    const __amdgpu_buffer_rsrc_t r = frag_rsrc(P.frag[0], C::FragBytes);
#pragma unroll
    for (int j = 0; j < FCPT; ++j) fchunk[j] = buffer_frag<u4>(r, tid * 16, j * C::Threads * 16);
  }
  u4 rawN[4];
  h8 pf[2];
  Analysis an;
  RgbStage<Tin> stN;
  const Tin* frame = reinterpret_cast<const Tin*>(P.frames) + (size_t)t.b * 3 * P.H * P.W;
  if constexpr (RGB) {
#pragma unroll
    for (int i = 0; i < 2; ++i) pf[i] = reinterpret_cast<const h8*>(P.pfrag)[i * 64 + lane];
    an = analysis_from(P.analysis);
    if constexpr (XC) stage_fetch<Tin>(stN, frame, group_geom(t.y0, t.x0, C::T, wave), P, lane);
    else stage_fetch<Tin>(stN, frame, group_geom(t.y0 - 4, t.x0 - 4, C::S0, wave), P, lane);
  } else {
    compress_fetch<MODE, TT>(rawN, P.skip + (size_t)t.b * (2 * P.Hl) * (2 * P.Wl) * 32, t, wave, P.Hl, P.Wl, lane);
  }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * C::Threads;
    if (i < kBodyConsts) cst[i] = cv[j];
  }
  if constexpr (RGB) {
#pragma unroll
    for (int j = 0; j < FCPT; ++j)
      if (tid + j * C::Threads < FragChunks) fr_lds[tid + j * C::Threads] = fchunk[j];
  }
  if (tid < 10) counters[tid] = tid < 2 ? C::Waves : C::Waves / 2;
  if (XC && tid == 0)                                  // this launch's count: the launches before + 1
    counters[10] = (int)(__hip_atomic_load(P.xflags + tidx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u);
  lds_barrier();
  if constexpr (XC) {
    fb_compress_rgb<MODE, Tin, TT, true>(P, t, bufA, cst, fr, pf, an, stN, slice, counters, wave, lane);
    exchange_publish(P, tidx, counters, tid);
  } else if constexpr (RGB) {
    fb_compress_rgb<MODE, Tin, TT>(P, t, bufA, cst, fr, pf, an, stN, slice, counters, wave, lane);
  } else {
    fb_compress<MODE, TT>(P, t, bufA, cst, Fc, rawN, wave, lane);
  }
  if constexpr (RGB) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // kept skip values stored before the barrier
    // expand weights: in flight during the barrier
    const __amdgpu_buffer_rsrc_t r = frag_rsrc(P.frag[5], C::FragBytes);
    const int voff = fresh(tid) * 16;
#pragma unroll
    for (int j = 0; j < FCPT; ++j) fchunk[j] = buffer_frag<u4>(r, voff, j * C::Threads * 16);
  }
  const int gf = (wave & 1) * 2 * C::NKg;              // this wave's group's first fragment
  FragSet<MODE, 2 * C::NKg> F1 = load_frags<MODE, 2 * C::NKg>(P.frag[1], gf, lane);
  if constexpr (XC) {                                  // the weight loads above are in flight during the wait
    if (exchange_wait(P, tidx, tx, ty, counters, tid, wave, lane)) {
      exchange_ring<MODE, TT>(P, t, bufA, tid);
    } else {                                           // block-uniform: compress the whole region here
      if (tid == 0) counters[0] = C::Waves;
      stage_fetch<Tin>(stN, frame, group_geom(t.y0 - 4, t.x0 - 4, C::S0, wave), P, fresh(lane));
      lds_barrier();
      fb_compress_rgb<MODE, Tin, TT>(P, t, bufA, cst, fr, pf, an, stN, slice, counters, wave, lane);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // its kept skip values are stored too
      // the weights are loaded again rather than kept live through that compress
      const __amdgpu_buffer_rsrc_t r = frag_rsrc(P.frag[5], C::FragBytes);
      const int voff = fresh(tid) * 16;
#pragma unroll
      for (int j = 0; j < FCPT; ++j) fchunk[j] = buffer_frag<u4>(r, voff, j * C::Threads * 16);
      F1 = load_frags<MODE, 2 * C::NKg>(P.frag[1], gf, fresh(lane));
    }
  }
  lds_barrier();
  if constexpr (RGB) {                                 // compress no longer reads the region
#pragma unroll
    for (int j = 0; j < FCPT; ++j)
      if (tid + j * C::Threads < FragChunks) fr_lds[tid + j * C::Threads] = fchunk[j];
  }
  fb_grouped<MODE, 1, TT>(P, t, bufA, bufB, cst, F1, counters + 2 + (wave & 1), wave, lane);
  const FragSet<MODE, 2 * C::NKg> F2 = load_frags<MODE, 2 * C::NKg>(P.frag[2], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 2, TT>(P, t, bufB, bufA, cst, F2, counters + 4 + (wave & 1), wave, lane);
  const FragSet<MODE, 2 * C::NKg> F3 = load_frags<MODE, 2 * C::NKg>(P.frag[3], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 3, TT>(P, t, bufA, bufB, cst, F3, counters + 6 + (wave & 1), wave, lane);
  const FragSet<MODE, 2 * C::NKg> F4 = load_frags<MODE, 2 * C::NKg>(P.frag[4], gf, lane);
  lds_barrier();
  fb_grouped<MODE, 4, TT>(P, t, bufB, bufA, cst, F4, counters + 8 + (wave & 1), wave, lane);
  FragSet<MODE, 8 * C::NKe> Fe;
  if constexpr (!RGB) Fe = load_frags<MODE, 8 * C::NKe>(P.frag[5], 0, lane);
  lds_barrier();
  if constexpr (RGB) fb_expand_rgb<MODE, TT>(P, t, bufA, cst, fr, counters + 1, wave, lane);
  else fb_expand<MODE, TT>(P, t, bufA, cst, Fe, wave, lane);
}

template <int MODE, int SRC, int TT = BodyFusedCfg<MODE>::T>
__global__ __launch_bounds__(BodyFusedCfg<MODE>::Threads) void body_fused_kernel(BodyFusedArgs P) {
  body_tile<MODE, SRC, TT>(P, body_tile_of((int)blockIdx.x, (int)gridDim.x, 0));
}

// Frame-input body with the compress exchange (every block resident at once).
template <int MODE, int SRC, int TT>
__global__ __launch_bounds__(BodyFusedCfg<MODE>::Threads) void body_fused_xc_kernel(BodyFusedArgs P) {
  body_tile<MODE, SRC, TT, true>(P, body_tile_of((int)blockIdx.x, (int)gridDim.x, 0));
}

// Two tile sides in one launch: blocks [0, n1) run tiles of side T1 for P1, the rest tiles of side
// T2 for P2.  The hardware starts blocks in order as CUs free up, so the small tiles fill the CUs
// that the last round of large tiles leaves idle, where two launches would run one after the other.
template <int MODE, int SRC, int T1, int T2>
__global__ __launch_bounds__(BodyFusedCfg<MODE>::Threads) void body_fused_pair_kernel(BodyFusedArgs P1, int n1,
                                                                                      BodyFusedArgs P2) {
  const int b = (int)blockIdx.x;
  if (b < n1) body_tile<MODE, SRC, T1>(P1, body_tile_of(b, n1, 0));
  else body_tile<MODE, SRC, T2>(P2, body_tile_of(b - n1, (int)gridDim.x - n1, n1));
}

// The FP16 policy's skip-input kernels are instantiated in k_body_fused_fp16.hip (compiled with
// the default instruction scheduler), the frame-input kernels in k_body_fused.hip (iterative ILP).
hipError_t body_fused_prepare_fp16();
void launch_body_fused_fp16(const BodyFusedArgs& args, int tile, int tiles, hipStream_t stream);
void launch_body_fused_pair_fp16(const BodyFusedArgs& a1, int n1, const BodyFusedArgs& a2, int n2, hipStream_t stream);

template <int MODE, int SRC, int TT>
const void* body_kernel_ptr() { return reinterpret_cast<const void*>(&body_fused_kernel<MODE, SRC, TT>); }
template <int MODE, int SRC, int TT>
const void* body_xc_ptr() { return reinterpret_cast<const void*>(&body_fused_xc_kernel<MODE, SRC, TT>); }
template <int MODE, int SRC, int T1, int T2>
const void* body_pair_ptr() { return reinterpret_cast<const void*>(&body_fused_pair_kernel<MODE, SRC, T1, T2>); }
// dynamic LDS of a launch of tile side TT
template <int MODE, int SRC, int TT>
constexpr int body_lds() { return SRC ? BodyFusedCfg<MODE, TT>::LdsRgb : BodyFusedCfg<MODE, TT>::Lds; }
template <int MODE, int SRC, int T1, int T2>
constexpr int body_pair_lds() {
  return body_lds<MODE, SRC, T1>() > body_lds<MODE, SRC, T2>() ? body_lds<MODE, SRC, T1>() : body_lds<MODE, SRC, T2>();
}
template <int MODE, int SRC, int TT>
void launch_body_t(const BodyFusedArgs& args, int tiles, hipStream_t stream) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int lds = SRC ? C::LdsRgb : C::Lds;
  hipLaunchKernelGGL((body_fused_kernel<MODE, SRC, TT>), dim3(tiles), dim3(C::Threads), lds, stream, args);
}
template <int MODE, int SRC, int T1, int T2>
void launch_pair_t(const BodyFusedArgs& a1, int n1, const BodyFusedArgs& a2, int n2, hipStream_t stream) {
  constexpr int lds = body_pair_lds<MODE, SRC, T1, T2>();
  hipLaunchKernelGGL((body_fused_pair_kernel<MODE, SRC, T1, T2>), dim3(n1 + n2), dim3(BodyFusedCfg<MODE>::Threads),
                     lds, stream, a1, n1, a2);
}

}  // namespace aeisu
