// Fused refine 3x3 (32 -> 64) + LeakyReLU + linear tail 1x1 (64 -> 64) + reconstruction
// head: the 64-channel FP16 coefficient tensor lives only in LDS.
//
// Reference: aeisu/model.py:489-490 (refine_540, metadata_head) and
// aeisu/reconstruction.py:15-83 (clamp, parity unpacking, polyphase 5x5 synthesis);
// native fused_native_fp16_refine_tail_conv_kernel (optimized/native/src/neural/srcpyr/
// SrcPyrNativeFp16Refine.cuh:334-557) followed by ReconstructConstant
// (optimized/native/src/neural/adaptive/AdaptiveReconstruction.cuh:288-417), which exchange
// the coefficients through a 70 MB (1080p) FP16 tensor in device memory.
//
// Arithmetic is that of the unfused kernels (k_refine_tail.hip, k_head.hip): FP16 operands
// with FP32 accumulation, FP32 refine bias, FP16-rounded tail bias, coefficients rounded to
// FP16, then the head's exact clamp split and hi/lo bank synthesis.  The result is
// bit-identical to refine_tail_kernel followed by head_kernel.
//
// gfx950 mapping: one persistent block of 12 waves per CU walks tiles of 32x4 packed pixels
// (64x8 LR pixels) on the padded grid.
//  * Waves 0-3 (producers) run refine + tail on the MFMA for tile i+1: the 44 weight
//    fragments sit in LDS (45 KB, loaded once) and each fragment read feeds two 16-pixel
//    groups; the refine accumulators become the tail's B operand in registers (the tail K
//    order is permuted on the host); FP16 coefficients go to an LDS buffer.  They also
//    load the zero-padded 34x6 work patch of tile i+2.
//  * Waves 4-11 (consumers) run the head on tile i, one LR row each, reading coefficients
//    and a clamped RGB tile from LDS, and load the RGB tile of tile i+1.
//  * Work patch, coefficients and RGB tile are double-buffered; one barrier per tile.
//    MFMA-bound producers and VALU-bound consumers share each SIMD.
#include "common.hpp"

namespace aeisu {

constexpr int kFQW = 32, kFQH = 4;                   // packed tile
constexpr int kFPW = kFQW + 2, kFPH = kFQH + 2;      // work patch (1-pixel zero halo)
constexpr int kFPix = 40;                            // halves per patch pixel (32 + 8 pad)
constexpr int kFMPix = 72;                           // halves per coefficient pixel (64 + 8 pad)
constexpr int kFLW = 2 * kFQW, kFLH = 2 * kFQH;      // LR tile
constexpr int kFRW = kFLW + 4, kFRH = kFLH + 4;      // RGB tile (2-pixel clamped halo)
constexpr int kFRPos = kFRW * kFRH;
constexpr int kFThreads = 768, kFProducers = 4;
constexpr int kFConsumerThreads = kFThreads - 64 * kFProducers;
constexpr int kFRgbPer = (kFRPos + kFConsumerThreads - 1) / kFConsumerThreads;
constexpr int kFPatchChunks = kFPH * kFPW * 4;       // 16-byte chunks of one work patch
constexpr int kFPatchPer = (kFPatchChunks + 64 * kFProducers - 1) / (64 * kFProducers);
constexpr int kFRefineFrags = 36, kFTailFrags = 8;

// LDS layout (bytes)
constexpr int kFOffW = 0;
constexpr int kFSizeW = (kFRefineFrags + kFTailFrags) * 64 * 16;
constexpr int kFOffPatch = kFOffW + kFSizeW;
constexpr int kFSizePatch = kFPH * kFPW * kFPix * 2;
constexpr int kFOffMeta = kFOffPatch + 2 * kFSizePatch;
constexpr int kFSizeMeta = kFQH * kFQW * kFMPix * 2;
constexpr int kFOffRgb = kFOffMeta + 2 * kFSizeMeta;
constexpr int kFSizeRgb = kFRPos * 16;
constexpr int kFLds = kFOffRgb + 2 * kFSizeRgb;
static_assert(kFLds <= 160 * 1024, "fused kernel LDS exceeds the CU's 160 KB");

struct FusedGeom {
  int H, W, Hq, Wq, py, px, batch;
  int qy_lo, qx_lo;            // first packed row / column covering source pixels
  int tiles_x, tiles_y, num_tiles;
};
struct FusedTile {
  int b, qy0, qx0;
};
__device__ __forceinline__ FusedTile fused_tile(int tidx, const FusedGeom& G) {
  FusedTile t;
  t.b = tidx / (G.tiles_y * G.tiles_x);
  const int rem = tidx - t.b * G.tiles_y * G.tiles_x;
  t.qy0 = G.qy_lo + (rem / G.tiles_x) * kFQH;
  t.qx0 = G.qx_lo + (rem % G.tiles_x) * kFQW;
  return t;
}

template <typename Tin>
__device__ __forceinline__ float fload(const Tin* p) { return (float)*p; }

// ---- producer side ----------------------------------------------------------------------------
struct PatchRegs {
  u4 v[kFPatchPer];
};
__device__ __forceinline__ void patch_fetch(PatchRegs& r, const _Float16* __restrict__ work, FusedTile t,
                                            const FusedGeom& G, int ptid) {
  const _Float16* in = work + (size_t)t.b * G.Hq * G.Wq * 32;
#pragma unroll
  for (int k = 0; k < kFPatchPer; ++k) {
    const int q = ptid + 64 * kFProducers * k;
    u4 v = {0u, 0u, 0u, 0u};
    if (q < kFPatchChunks) {
      const int pix = q >> 2, ch = (q & 3) * 8;
      const int ly = pix / kFPW, lx = pix - ly * kFPW;
      const int gy = t.qy0 + ly - 1, gx = t.qx0 + lx - 1;
      if (gy >= 0 && gy < G.Hq && gx >= 0 && gx < G.Wq)
        v = *reinterpret_cast<const u4*>(in + ((size_t)gy * G.Wq + gx) * 32 + ch);
    }
    r.v[k] = v;
  }
}
__device__ __forceinline__ void patch_store(const PatchRegs& r, unsigned char* lds_patch, int ptid) {
#pragma unroll
  for (int k = 0; k < kFPatchPer; ++k) {
    const int q = ptid + 64 * kFProducers * k;
    if (q < kFPatchChunks) {
      const int pix = q >> 2, ch = (q & 3) * 8;
      *reinterpret_cast<u4*>(lds_patch + (pix * kFPix + ch) * 2) = r.v[k];
    }
  }
}

// refine + tail for packed row `prow` of the tile (two 16-pixel groups) -> FP16 coefficients.
__device__ __forceinline__ void produce_row(const unsigned char* lds_w, const unsigned char* lds_patch,
                                            unsigned char* lds_meta, int prow, int lane,
                                            const float (&rb)[4][4], const float (&tb)[4][4]) {
  const int n = lane & 15, g = lane >> 4;
  const h8* wf = reinterpret_cast<const h8*>(lds_w);
  const _Float16(*patch)[kFPW][kFPix] = reinterpret_cast<const _Float16(*)[kFPW][kFPix]>(lds_patch);
  f4 acc[4][2];
#pragma unroll
  for (int T = 0; T < 4; ++T) acc[T][0] = acc[T][1] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    const h8 b0 = *reinterpret_cast<const h8*>(&patch[prow + k / 3][n + k % 3][8 * g]);
    const h8 b1 = *reinterpret_cast<const h8*>(&patch[prow + k / 3][16 + n + k % 3][8 * g]);
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      const h8 a = wf[(T * 9 + k) * 64 + lane];
      acc[T][0] = mfma_f16(a, b0, acc[T][0]);
      acc[T][1] = mfma_f16(a, b1, acc[T][1]);
    }
  }
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    h8 bt[2];
#pragma unroll
    for (int T = 0; T < 4; ++T)
#pragma unroll
      for (int r = 0; r < 4; ++r) bt[T >> 1][(T & 1) * 4 + r] = (_Float16)leaky(acc[T][J][r] + rb[T][r], 0.1f);
    _Float16* dst = reinterpret_cast<_Float16*>(lds_meta) + ((prow * kFQW) + 16 * J + n) * kFMPix + 4 * g;
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      f4 o = mfma_f16(wf[(kFRefineFrags + T * 2) * 64 + lane], bt[0], f4{0.f, 0.f, 0.f, 0.f});
      o = mfma_f16(wf[(kFRefineFrags + T * 2 + 1) * 64 + lane], bt[1], o);
      u2 w;
      w[0] = pack_h2(o[0] + tb[T][0], o[1] + tb[T][1]);
      w[1] = pack_h2(o[2] + tb[T][2], o[3] + tb[T][3]);
      *reinterpret_cast<u2*>(dst + 16 * T) = w;
    }
  }
}

// ---- consumer side ----------------------------------------------------------------------------
struct RgbRegs {
  float v[kFRgbPer][3];
};
template <typename Tin>
__device__ __forceinline__ void rgb_fetch(RgbRegs& r, const Tin* __restrict__ src, FusedTile t, const FusedGeom& G,
                                          int ctid) {
  const size_t plane = (size_t)G.H * G.W;
  const Tin* s = src + (size_t)t.b * 3 * plane;
  const int y0 = 2 * t.qy0 - G.py - 2, x0 = 2 * t.qx0 - G.px - 2;
#pragma unroll
  for (int k = 0; k < kFRgbPer; ++k) {
    const int q = ctid + kFConsumerThreads * k;
    if (q < kFRPos) {
      const int ly = q / kFRW, lx = q - ly * kFRW;
      const int sy = min(max(y0 + ly, 0), G.H - 1), sx = min(max(x0 + lx, 0), G.W - 1);
      const size_t o = (size_t)sy * G.W + sx;
      r.v[k][0] = fload(s + o);
      r.v[k][1] = fload(s + plane + o);
      r.v[k][2] = fload(s + 2 * plane + o);
    }
  }
}
__device__ __forceinline__ void rgb_store(const RgbRegs& r, float4* lds_rgb, int ctid) {
#pragma unroll
  for (int k = 0; k < kFRgbPer; ++k) {
    const int q = ctid + kFConsumerThreads * k;
    if (q < kFRPos) lds_rgb[q] = make_float4(r.v[k][0], r.v[k][1], r.v[k][2], 0.f);
  }
}

// 2 FP16 coefficients (one dword) -> (u, w) with clamp(v) = u + 0.05 w, both exact in FP16
// (identical to the head kernel's split; see k_head.hip).
__device__ __forceinline__ void fused_clamp_split(unsigned v, unsigned& u, unsigned& w) {
  typedef unsigned short us2 __attribute__((ext_vector_type(2)));
  const unsigned mag = v & 0x7FFF7FFFu;
  const us2 m = __builtin_bit_cast(us2, mag);
  const us2 nanpart = __builtin_elementwise_sub_sat(m, (us2){0x7C00, 0x7C00});
  const us2 mc = __builtin_elementwise_min(m, (us2){0x4A00, 0x4A00});
  const h2 mch = __builtin_bit_cast(h2, mc);
  const h2 e = __builtin_elementwise_max(mch - (h2){2, 2}, (h2){0, 0});
  const h2 um = mch - e;
  unsigned nanbits;
  asm("v_pk_mad_u16 %0, %1, %2, 0 clamp" : "=v"(nanbits) : "v"(__builtin_bit_cast(unsigned, nanpart)),
      "s"(0x7E007E00u));
  u = ((__builtin_bit_cast(unsigned, um) | nanbits) & 0x7FFF7FFFu) | (v & 0x80008000u);
  w = (__builtin_bit_cast(unsigned, e) & 0x7FFF7FFFu) | (v & 0x80008000u);
}

template <typename Tout>
__device__ __forceinline__ void fstore_pair(Tout* p, float left, float right);
template <>
__device__ __forceinline__ void fstore_pair<_Float16>(_Float16* p, float left, float right) {
  *reinterpret_cast<unsigned*>(p) = pack_h2(left, right);
}
template <>
__device__ __forceinline__ void fstore_pair<float>(float* p, float left, float right) {
  *reinterpret_cast<float2*>(p) = make_float2(left, right);
}

// Head on LR row `r` of the tile.
template <typename Tout>
__device__ __forceinline__ void consume_row(const unsigned char* lds_meta, const float4* lds_rgb, Tout* __restrict__ out,
                                            FusedTile t, const FusedGeom& G, int r, int lane, const h8 (&A1)[7],
                                            const h8 (&A2)[7], const f4 (&base)[7], const int (&toff)[6],
                                            float& chk) {
  const int n = lane & 15, g = lane >> 4;
  const int y = 2 * t.qy0 + r - G.py;
  if (y < 0 || y >= G.H) return;                      // wave-uniform
  const size_t oplane = (size_t)4 * G.H * G.W;
  Tout* ob = out + (size_t)t.b * 3 * oplane;
  const _Float16* mrow = reinterpret_cast<const _Float16*>(lds_meta) + (r >> 1) * kFQW * kFMPix;
  const int rho_y = (r & 1) << 1;
#pragma unroll
  for (int j = 0; j < kFLW / 16; ++j) {
    const int xs = 2 * t.qx0 + 16 * j - G.px;         // LR column of lane n = 0
    if (xs + 15 < 0 || xs >= G.W) continue;           // wave-uniform
    const int x = xs + n;
    const u2 coef = *reinterpret_cast<const u2*>(mrow + (8 * j + (n >> 1)) * kFMPix + 16 * (rho_y | (n & 1)) + 4 * g);
    unsigned U[2], Wd[2];
    fused_clamp_split(coef[0], U[0], Wd[0]);
    fused_clamp_split(coef[1], U[1], Wd[1]);
#pragma unroll
    for (int w = 0; w < 2; ++w) permlane32_swap_u(U[w], Wd[w]);
#pragma unroll
    for (int w = 0; w < 2; ++w) permlane16_swap_u(U[w], Wd[w]);
    const u4 bw = {U[0], U[1], Wd[0], Wd[1]};
    const h8 bop = __builtin_bit_cast(h8, bw);
    f4 acc[7];
#pragma unroll
    for (int q = 0; q < 7; ++q) {
      acc[q] = mfma_f16(A1[q], bop, base[q]);
      acc[q] = mfma_f16(A2[q], bop, acc[q]);
    }
    const float4* L0 = lds_rgb + r * kFRW + 16 * j + n;
    float o[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) o[i] = 0.f;
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      const float4 L = L0[toff[q]];
#pragma unroll
      for (int ph = 0; ph < 4; ++ph) {
        o[0 * 4 + ph] = fmaf(acc[q][ph], L.x, o[0 * 4 + ph]);
        o[1 * 4 + ph] = fmaf(acc[q][ph], L.y, o[1 * 4 + ph]);
        o[2 * 4 + ph] = fmaf(acc[q][ph], L.z, o[2 * 4 + ph]);
      }
    }
    float s[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      float a = o[2 * i], z = o[2 * i + 1];
      permlane32_swap(a, z);
      s[i] = a + z;
    }
    float u[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      float a = s[2 * c], z = s[2 * c + 1];
      permlane16_swap(a, z);
      u[c] = a + z;
    }
    const float4 L24 = L0[4 * kFRW + 4];
    u[0] = fmaf(acc[6][0], L24.x, u[0]);
    u[1] = fmaf(acc[6][0], L24.y, u[1]);
    u[2] = fmaf(acc[6][0], L24.z, u[2]);
    const bool inside = x >= 0 && x < G.W;
    chk = fmaf(inside ? u[0] + u[1] + u[2] : 0.f, 0.0f, chk);
    float left[3], right[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      left[c] = __builtin_amdgcn_fmed3f(u[c], 0.0f, 1.0f);
      right[c] = left[c];
      permlane32_swap(left[c], right[c]);
    }
    if (g < 2 && inside) {
      Tout* p = ob + (size_t)(2 * y + g) * (2 * G.W) + 2 * x;
#pragma unroll
      for (int c = 0; c < 3; ++c) fstore_pair<Tout>(p + c * oplane, left[c], right[c]);
    }
  }
}

// Producer waves: coefficients of tile i+1, work patch of tile i+2.
__device__ __forceinline__ void producer_main(unsigned char* smem, const _Float16* __restrict__ work,
                                              const float* __restrict__ rbias, const float* __restrict__ tbias,
                                              const FusedGeom& G, int wave, int lane, int ptid) {
  const int g = lane >> 4;
  float rb[4][4], tb[4][4];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rb[T][r] = rbias[16 * T + 4 * g + r];
      tb[T][r] = tbias[16 * T + 4 * g + r];
    }
  unsigned char* const lds_w = smem + kFOffW;
  const int t0 = tile_of(0, G.num_tiles), t1 = tile_of(1, G.num_tiles);
  {
    PatchRegs pr;
    if (t0 < G.num_tiles) {
      patch_fetch(pr, work, fused_tile(t0, G), G, ptid);
      patch_store(pr, smem + kFOffPatch, ptid);
    }
    if (t1 < G.num_tiles) {
      patch_fetch(pr, work, fused_tile(t1, G), G, ptid);
      patch_store(pr, smem + kFOffPatch + kFSizePatch, ptid);
    }
  }
  __syncthreads();                                   // prologue loads visible
  if (t0 < G.num_tiles) produce_row(lds_w, smem + kFOffPatch, smem + kFOffMeta, wave, lane, rb, tb);
  __syncthreads();                                   // coefficients of tile 0 visible
  const int iters = tile_iters(G.num_tiles);
  for (int it = 0; it < iters; ++it) {
    if (tile_of(it, G.num_tiles) >= G.num_tiles) break;   // block-uniform, as in consumer_main
    const int tn = tile_of(it + 1, G.num_tiles), tnn = tile_of(it + 2, G.num_tiles);
    const int cur = it & 1, nxt = cur ^ 1;
    PatchRegs pr;
    if (tnn < G.num_tiles) patch_fetch(pr, work, fused_tile(tnn, G), G, ptid);
    if (tn < G.num_tiles)
      produce_row(lds_w, smem + kFOffPatch + nxt * kFSizePatch, smem + kFOffMeta + nxt * kFSizeMeta, wave, lane, rb, tb);
    if (tnn < G.num_tiles) patch_store(pr, smem + kFOffPatch + cur * kFSizePatch, ptid);
    __syncthreads();
  }
}

// Consumer waves: head of tile i, RGB tile of tile i+1.
template <typename Tin, typename Tout>
__device__ __forceinline__ void consumer_main(unsigned char* smem, const Tin* __restrict__ src,
                                              const h8* __restrict__ bankA, Tout* __restrict__ out,
                                              const FusedGeom& G, int row, int lane, int ctid,
                                              unsigned* __restrict__ nonfinite) {
  const int g = lane >> 4;
  h8 A1[7], A2[7];
  f4 base[7];
  int toff[6];
  const f4* base_src = reinterpret_cast<const f4*>(bankA + 14 * 64);
#pragma unroll
  for (int q = 0; q < 7; ++q) {
    A1[q] = bankA[q * 64 + lane];
    A2[q] = bankA[(7 + q) * 64 + lane];
    base[q] = base_src[q * 4 + g];
  }
#pragma unroll
  for (int q = 0; q < 6; ++q) {
    const int tap = 4 * q + g;
    toff[q] = (tap / 5) * kFRW + tap % 5;
  }
  float chk = 0.f;
  const int t0 = tile_of(0, G.num_tiles);
  if (t0 < G.num_tiles) {
    RgbRegs rr;
    rgb_fetch(rr, src, fused_tile(t0, G), G, ctid);
    rgb_store(rr, reinterpret_cast<float4*>(smem + kFOffRgb), ctid);
  }
  __syncthreads();                                   // prologue loads visible
  __syncthreads();                                   // coefficients of tile 0 visible
  const int iters = tile_iters(G.num_tiles);
  for (int it = 0; it < iters; ++it) {
    const int tc = tile_of(it, G.num_tiles);
    if (tc >= G.num_tiles) break;                    // block-uniform, as in producer_main
    const int tn = tile_of(it + 1, G.num_tiles);
    const int cur = it & 1, nxt = cur ^ 1;
    RgbRegs rr;
    if (tn < G.num_tiles) rgb_fetch(rr, src, fused_tile(tn, G), G, ctid);
    consume_row<Tout>(smem + kFOffMeta + cur * kFSizeMeta, reinterpret_cast<const float4*>(smem + kFOffRgb + cur * kFSizeRgb),
                      out, fused_tile(tc, G), G, row, lane, A1, A2, base, toff, chk);
    if (tn < G.num_tiles) rgb_store(rr, reinterpret_cast<float4*>(smem + kFOffRgb + nxt * kFSizeRgb), ctid);
    __syncthreads();
  }
  if (nonfinite && __ballot(chk != chk) != 0ull && lane == 0) atomicOr(nonfinite, 1u);
}

// Every wave executes the same number of barriers: two in the prologue, one per tile.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kFThreads) void fused_tail_head_kernel(
    const _Float16* __restrict__ work, const Tin* __restrict__ src, const h8* __restrict__ rt_frag,
    const float* __restrict__ rbias, const float* __restrict__ tbias, const h8* __restrict__ bankA,
    Tout* __restrict__ out, FusedGeom G, unsigned* __restrict__ nonfinite) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  {
    const u4* s = reinterpret_cast<const u4*>(rt_frag);
    u4* d = reinterpret_cast<u4*>(smem + kFOffW);
    for (int i = tid; i < kFSizeW / 16; i += kFThreads) d[i] = s[i];
  }
  if (wave < kFProducers)                            // wave-uniform role
    producer_main(smem, work, rbias, tbias, G, wave, lane, tid);
  else
    consumer_main<Tin, Tout>(smem, src, bankA, out, G, wave - kFProducers, lane, tid - 64 * kFProducers, nonfinite);
}

FusedGeom fused_geometry(int H, int W, int Hq, int Wq, int py, int px, int batch) {
  FusedGeom G;
  G.H = H; G.W = W; G.Hq = Hq; G.Wq = Wq; G.py = py; G.px = px; G.batch = batch;
  G.qy_lo = py >> 1;
  G.qx_lo = px >> 1;
  const int qy_hi = (py + H - 1) >> 1, qx_hi = (px + W - 1) >> 1;
  G.tiles_y = (qy_hi - G.qy_lo + kFQH) / kFQH;
  G.tiles_x = (qx_hi - G.qx_lo + kFQW) / kFQW;
  G.num_tiles = batch * G.tiles_y * G.tiles_x;
  return G;
}

int fused_num_tiles(int batch, int H, int W, int Hq, int Wq, int py, int px) {
  return fused_geometry(H, W, Hq, Wq, py, px, batch).num_tiles;
}

template <typename Tin, typename Tout>
static hipError_t launch_fused_t(const void* work, const void* src, const void* rt_frag, const float* rbias,
                                 const float* tbias, const void* bankA, void* out, const FusedGeom& G,
                                 unsigned* nonfinite, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((fused_tail_head_kernel<Tin, Tout>), dim3(grid), dim3(kFThreads), kFLds, stream,
                     (const _Float16*)work, (const Tin*)src, (const h8*)rt_frag, rbias, tbias, (const h8*)bankA,
                     (Tout*)out, G, nonfinite);
  return hipGetLastError();
}

// Allows the kernels' dynamic LDS above the default limit; called once per device at configure.
hipError_t fused_prepare() {
  const void* k[4] = {reinterpret_cast<const void*>(&fused_tail_head_kernel<float, float>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<float, _Float16>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, float>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, _Float16>)};
  for (const void* f : k) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kFLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_fused_tail_head(int in_fp32, int out_fp32, const void* work, const void* src, const void* rt_frag,
                                  const float* rbias, const float* tbias, const void* bankA, void* out, int H, int W,
                                  int Hq, int Wq, int py, int px, int batch, unsigned* nonfinite, int grid,
                                  hipStream_t stream) {
  const FusedGeom G = fused_geometry(H, W, Hq, Wq, py, px, batch);
  if (in_fp32 && out_fp32)
    return launch_fused_t<float, float>(work, src, rt_frag, rbias, tbias, bankA, out, G, nonfinite, grid, stream);
  if (in_fp32)
    return launch_fused_t<float, _Float16>(work, src, rt_frag, rbias, tbias, bankA, out, G, nonfinite, grid, stream);
  if (out_fp32)
    return launch_fused_t<_Float16, float>(work, src, rt_frag, rbias, tbias, bankA, out, G, nonfinite, grid, stream);
  return launch_fused_t<_Float16, _Float16>(work, src, rt_frag, rbias, tbias, bankA, out, G, nonfinite, grid, stream);
}

}  // namespace aeisu
