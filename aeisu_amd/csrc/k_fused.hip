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
// FP16, then the head's exact clamp split and MFMA synthesis.  The result is bit-identical
// to refine_tail_kernel followed by head_kernel.
//
// gfx950 mapping: one persistent block per CU walks tiles of 32 x QH packed pixels
// (64 x 2QH LR pixels) on the padded grid.
//  * 4 producer waves run refine + tail on the MFMA for tile i+1: the 44 weight fragments
//    sit in LDS (45 KB, loaded once) and each fragment read feeds QH/2 16-pixel groups; the
//    refine accumulators become the tail's B operand in registers (the tail K order is
//    permuted on the host); FP16 coefficients go to an LDS buffer.  They also load the
//    zero-padded work patch of tile i+2.
//  * 2QH consumer waves run the head on tile i, one LR row each, reading coefficients and a
//    clamped RGB tile from LDS, and load the RGB tile of tile i+1.  The first tile's
//    coefficients are produced by the consumer waves (one 16-pixel group each).
//  * Output stores carry the non-temporal hint, and with FP16 output two neighbouring chunks'
//    stores are issued together so that each fills whole 128-byte lines.
//  * Work patch, coefficients and RGB tile are double-buffered; one barrier per tile.
//    MFMA-bound producers and VALU-bound consumers share each SIMD.
//  * FP16 frames: QH = 6 (16 waves, 4 per SIMD, <= 128 VGPRs), the RGB tile stays FP16 in
//    LDS and the head's FMAs take it as a mixed-precision operand (v_fma_mix, exact);
//    FP32 frames: QH = 4 (12 waves) with an FP32 RGB tile.
//  * Head synthesis, two forms (QC = false / true), each bit-identical to k_head.hip's:
//    FP16 policy: the exact clamp split u + 0.05 w, two MFMAs per row tile (k_head.hip).
//    Quantized policies (QC): the producers store the clamped coefficients rounded to FP16
//    (common.hpp coef_clamp_h16), the consumer reads its 8 B-operand coefficients with one
//    16-byte LDS read and runs ONE MFMA per row tile, [K_hi | K_lo] . [c ; c], with the FP32
//    base (per lane group, 28 values) as the accumulator input.
#include "common.hpp"
#include "kernels.hpp"

namespace aeisu {

template <typename Tin>
struct FusedCfg;
template <>
struct FusedCfg<_Float16> {
  static constexpr int QH = 6;
  typedef h4 Rgb;
};
template <>
struct FusedCfg<float> {
  static constexpr int QH = 4;
  typedef float4 Rgb;
};

constexpr int kFQW = 32;                             // packed tile width
constexpr int kFPix = 40;                            // halves per patch pixel (32 + 8 pad)
constexpr int kFMPix = 72;                           // halves per coefficient pixel (64 + 8 pad)
constexpr int kFLW = 2 * kFQW, kFRW = kFLW + 4;      // LR tile width, RGB tile width (2-pixel halo)
constexpr int kFProducers = 4;
constexpr int kFRefineFrags = 36, kFTailFrags = 8;
constexpr int kFSizeW = (kFRefineFrags + kFTailFrags) * 64 * 16;

template <typename Tin>
struct FusedLayout {
  static constexpr int QH = FusedCfg<Tin>::QH;
  static constexpr int LH = 2 * QH, RH = LH + 4, RPos = kFRW * RH;
  static constexpr int PH = QH + 2, PW = kFQW + 2;
  static constexpr int Consumers = LH, Threads = 64 * (kFProducers + Consumers);
  static constexpr int ConsumerThreads = 64 * Consumers;
  static constexpr int J = QH / 2;                   // 16-pixel groups per producer (2 per packed row)
  static constexpr int RgbPer = (RPos + ConsumerThreads - 1) / ConsumerThreads;
  static constexpr int PatchChunks = PH * PW * 4;    // 16-byte chunks of one work patch
  static constexpr int PatchPer = (PatchChunks + 64 * kFProducers - 1) / (64 * kFProducers);
  static constexpr int OffW = 0;
  static constexpr int OffBias = OffW + kFSizeW;     // refine bias [64], tail bias [64] (FP32)
  static constexpr int OffPatch = OffBias + 512;
  static constexpr int SizePatch = PH * PW * kFPix * 2;
  static constexpr int OffMeta = OffPatch + 2 * SizePatch;
  static constexpr int SizeMeta = QH * kFQW * kFMPix * 2;
  static constexpr int OffRgb = OffMeta + 2 * SizeMeta;
  static constexpr int SizeRgb = RPos * (int)sizeof(typename FusedCfg<Tin>::Rgb);
  static constexpr int Lds = OffRgb + 2 * SizeRgb;
  static_assert(Lds <= 160 * 1024, "fused kernel LDS exceeds the CU's 160 KB");
  static_assert(J * kFProducers == 2 * QH, "producers must split the tile's 16-pixel groups evenly");
  static_assert(Consumers == 2 * QH, "the consumers produce the first tile, one group each");
};

struct FusedGeom {
  int H, W, Hq, Wq, py, px, batch;
  int qy_lo, qx_lo;            // first packed row / column covering source pixels
  int tiles_x, tiles_y, num_tiles;
};
struct FusedTile {
  int b, qy0, qx0;
};
template <int QH>
__device__ __forceinline__ FusedTile fused_tile(int tidx, const FusedGeom& G) {
  FusedTile t;
  t.b = tidx / (G.tiles_y * G.tiles_x);
  const int rem = tidx - t.b * G.tiles_y * G.tiles_x;
  t.qy0 = G.qy_lo + (rem / G.tiles_x) * QH;
  t.qx0 = G.qx_lo + (rem % G.tiles_x) * kFQW;
  return t;
}

// ---- producer side ----------------------------------------------------------------------------
template <typename LY>
struct PatchRegs {
  u4 v[LY::PatchPer];
};
template <typename LY>
__device__ __forceinline__ void patch_fetch(PatchRegs<LY>& r, const _Float16* __restrict__ work, FusedTile t,
                                            const FusedGeom& G, int ptid) {
  const _Float16* in = work + (size_t)t.b * G.Hq * G.Wq * 32;
#pragma unroll
  for (int k = 0; k < LY::PatchPer; ++k) {
    const int q = ptid + 64 * kFProducers * k;
    u4 v = {0u, 0u, 0u, 0u};
    if (q < LY::PatchChunks) {
      const int pix = q >> 2, ch = (q & 3) * 8;
      const int ly = pix / LY::PW, lx = pix - ly * LY::PW;
      const int gy = t.qy0 + ly - 1, gx = t.qx0 + lx - 1;
      if (gy >= 0 && gy < G.Hq && gx >= 0 && gx < G.Wq)
        v = *reinterpret_cast<const u4*>(in + ((size_t)gy * G.Wq + gx) * 32 + ch);
    }
    r.v[k] = v;
  }
}
template <typename LY>
__device__ __forceinline__ void patch_store(const PatchRegs<LY>& r, unsigned char* lds_patch, int ptid) {
#pragma unroll
  for (int k = 0; k < LY::PatchPer; ++k) {
    const int q = ptid + 64 * kFProducers * k;
    if (q < LY::PatchChunks) {
      const int pix = q >> 2, ch = (q & 3) * 8;
      *reinterpret_cast<u4*>(lds_patch + (pix * kFPix + ch) * 2) = r.v[k];
    }
  }
}

// With two patch rows per producer wave (FP16 frames: PH = 8) the chunks take a row-wise mapping:
// producer wave w loads patch rows 2w and 2w+1, whose 2 x 34 pixels are two contiguous 2176-byte
// segments of the work tensor, and lane l takes chunks c = l + 64k of the two rows (k = 0..4,
// c < 272).  Every chunk's offset is the lane's 16 l plus a wave-uniform row start and a constant,
// and every LDS offset the lane's base plus 1280 k (consecutive patch rows are contiguous in LDS
// too), so the fetch costs about four VALU instructions per chunk where the general mapping
// (patch_fetch: one division, clamps and a 64-bit address per chunk) costs about thirty.  Chunks
// outside the work tensor get an offset past the buffer's range, which the hardware reads as zero
// (the zero padding of the refine convolution).
constexpr int kOutOfRange = 0x7FFFFFF0;            // at or past num_records for every work tensor < 2 GiB
template <typename LY>
__device__ __forceinline__ void patch_fetch_rows(PatchRegs<LY>& r, const _Float16* __restrict__ work, FusedTile t,
                                                 const FusedGeom& G, int wave, int lane) {
  static_assert(LY::PH == 2 * kFProducers && LY::PW * 4 * 2 == 272 && LY::PatchPer == 5,
                "two 34-pixel patch rows per producer wave, five chunks per lane");
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(work) + (size_t)t.b * G.Hq * G.Wq * 32, 0, G.Hq * G.Wq * 64, kRawBufferWord3);
  const int w = __builtin_amdgcn_readfirstlane(wave);
  const int r0 = t.qy0 - 1 + 2 * w;                  // patch rows r0 and r0 + 1 (wave-uniform)
  const bool ok0 = (unsigned)r0 < (unsigned)G.Hq, ok1 = (unsigned)(r0 + 1) < (unsigned)G.Hq;
  const int s0 = r0 * G.Wq * 64, s1 = s0 + G.Wq * 64;
  const int gx = t.qx0 - 1 + (lane >> 2);            // work column of chunk l
  const int cb = (t.qx0 - 1) * 64 + lane * 16;       // chunk l's byte offset from its row's start
  // offset of chunk l + 4 d of a row (d pixels to the right of chunk l), or out of range
  auto at = [&](bool row_ok, int start, int d) {
    return row_ok && (unsigned)(gx + d) < (unsigned)G.Wq ? start + cb + 64 * d : kOutOfRange;
  };
  const int o2 = lane < 8 ? at(ok0, s0, 32) : at(ok1, s1, -2);   // chunk 128 + l of row 0, or l - 8 of row 1
  r.v[0] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, at(ok0, s0, 0), 0, 0));
  r.v[1] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, at(ok0, s0, 16), 0, 0));
  r.v[2] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, o2, 0, 0));
  r.v[3] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, at(ok1, s1, 14), 0, 0));
  // chunks 256..271 of the two rows (lanes 0..15); the other lanes' fifth load is out of range
  r.v[4] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane < 16 ? at(ok1, s1, 30) : kOutOfRange, 0, 0));
}
template <typename LY>
__device__ __forceinline__ void patch_store_rows(const PatchRegs<LY>& r, unsigned char* lds_patch, int wave, int lane) {
  const int w = __builtin_amdgcn_readfirstlane(wave);
  unsigned char* d = lds_patch + 2 * w * LY::PW * kFPix * 2 + ((lane >> 2) * kFPix + (lane & 3) * 8) * 2;
#pragma unroll
  for (int k = 0; k < 4; ++k) *reinterpret_cast<u4*>(d + 1280 * k) = r.v[k];
  if (lane < 16) *reinterpret_cast<u4*>(d + 5120) = r.v[4];
}

// refine + tail for 16-pixel groups p*J .. p*J+J-1 of the tile (group q: packed row q/2, half q%2).
// One producer wave per SIMD runs this, so nothing hides its LDS latency: the operands are pipelined
// by hand, each weight fragment loaded one (tap, T) step ahead of its three MFMAs and each tap's
// patch operands one tap ahead; the tail fragments are loaded once per call and shared by the J
// groups (loaded per group, and waited for right before use, they left the producer at a third of
// its issue rate).
// J = LY::J for the producer waves; the first tile of a launch is produced by the consumer waves
// with J = 1 (one group each), so the consumers do not sit idle for a whole producer tile.
template <typename LY, bool QC, int J = LY::J>
__device__ __forceinline__ void produce(const unsigned char* smem, const unsigned char* lds_patch,
                                        unsigned char* lds_meta, int p, int lane) {
  const int n = lane & 15, g = lane >> 4;
  const h8* wf = reinterpret_cast<const h8*>(smem + LY::OffW);
  const f4* bias = reinterpret_cast<const f4*>(smem + LY::OffBias);
  const _Float16(*patch)[LY::PW][kFPix] = reinterpret_cast<const _Float16(*)[LY::PW][kFPix]>(lds_patch);
  int prow[J], pcol[J];
#pragma unroll
  for (int jj = 0; jj < J; ++jj) {
    const int q = p * J + jj;
    prow[jj] = q >> 1;
    pcol[jj] = 16 * (q & 1);
  }
  f4 acc[4][J];
#pragma unroll
  for (int T = 0; T < 4; ++T)
#pragma unroll
    for (int jj = 0; jj < J; ++jj) acc[T][jj] = f4{0.f, 0.f, 0.f, 0.f};
  // refine fragment of step s = 4k + T is wf[(T * 9 + k) * 64 + lane]
  h8 bcur[J], bnxt[J];
#pragma unroll
  for (int jj = 0; jj < J; ++jj) bcur[jj] = *reinterpret_cast<const h8*>(&patch[prow[jj]][pcol[jj] + n][8 * g]);
  h8 anext = wf[lane];
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    if (k < 8) {
#pragma unroll
      for (int jj = 0; jj < J; ++jj)
        bnxt[jj] = *reinterpret_cast<const h8*>(&patch[prow[jj] + (k + 1) / 3][pcol[jj] + n + (k + 1) % 3][8 * g]);
    }
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      const h8 a = anext;
      const int s = 4 * k + T + 1;
      if (s < 36) anext = wf[((s & 3) * 9 + (s >> 2)) * 64 + lane];
#pragma unroll
      for (int jj = 0; jj < J; ++jj) acc[T][jj] = mfma_f16(a, bcur[jj], acc[T][jj]);
    }
    if (k < 8) {
#pragma unroll
      for (int jj = 0; jj < J; ++jj) bcur[jj] = bnxt[jj];
    }
  }
  // refine epilogue -> the tail's B operands (refine channel order permuted on the host)
  h8 bt[J][2];
#pragma unroll
  for (int jj = 0; jj < J; ++jj)
#pragma unroll
    for (int T = 0; T < 4; ++T) {
      const f4 rb = bias[4 * T + g];                 // refine bias of channels 16T + 4g + r
#pragma unroll
      for (int r = 0; r < 4; ++r) bt[jj][T >> 1][(T & 1) * 4 + r] = (_Float16)leaky(acc[T][jj][r] + rb[r], 0.1f);
    }
#pragma unroll
  for (int T = 0; T < 4; ++T) {
    const h8 t0 = wf[(kFRefineFrags + T * 2) * 64 + lane], t1 = wf[(kFRefineFrags + T * 2 + 1) * 64 + lane];
    const f4 tb = bias[16 + 4 * T + g];              // FP16-rounded tail bias
#pragma unroll
    for (int jj = 0; jj < J; ++jj) {
      f4 o = mfma_f16(t0, bt[jj][0], f4{0.f, 0.f, 0.f, 0.f});
      o = mfma_f16(t1, bt[jj][1], o);
      u2 w;
      w[0] = pack_h2(o[0] + tb[0], o[1] + tb[1]);
      w[1] = pack_h2(o[2] + tb[2], o[3] + tb[3]);
      if constexpr (QC) {                          // coefficients 4g..4g+3 of parity T, clamped
        w[0] = coef_clamp_h16(w[0]);
        w[1] = coef_clamp_h16(w[1]);
      }
      _Float16* dst = reinterpret_cast<_Float16*>(lds_meta) + (prow[jj] * kFQW + pcol[jj] + n) * kFMPix + 4 * g;
      *reinterpret_cast<u2*>(dst + 16 * T) = w;
    }
  }
}

// ---- consumer side ----------------------------------------------------------------------------
// The RGB tile of the next tile is loaded into registers as raw frame values and converted
// only when it is stored to LDS: converting at load time makes the compiler wait for each
// load right away, which would expose the memory latency instead of hiding it behind the
// current tile.  The raw values are held as zero-extended 32-bit words and packed at the store
// by a volatile asm, so that the compiler cannot pack two FP16 channels into one register (and
// wait for both loads) right after the loads.  Loads are unconditional (indices clamped into the
// tile) so they are not split into branches either.
template <typename Tin, typename LY>
struct RgbRegs {
  unsigned v[LY::RgbPer][3];
};
template <typename Tin, typename LY>
__device__ __forceinline__ void rgb_fetch(RgbRegs<Tin, LY>& r, const Tin* __restrict__ src, FusedTile t,
                                          const FusedGeom& G, int ctid) {
  // one raw buffer per frame (3 planes < 2^31 bytes): 32-bit offsets, the plane as a scalar offset
  const int plane = G.H * G.W * (int)sizeof(Tin);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<Tin*>(src) + (size_t)t.b * 3 * G.H * G.W, 0, 3 * plane, kRawBufferWord3);
  const int y0 = 2 * t.qy0 - G.py - 2, x0 = 2 * t.qx0 - G.px - 2;
#pragma unroll
  for (int k = 0; k < LY::RgbPer; ++k) {
    const int q = min(ctid + LY::ConsumerThreads * k, LY::RPos - 1);
    const int ly = q / kFRW, lx = q - ly * kFRW;
    const int sy = min(max(y0 + ly, 0), G.H - 1);
    const int sx = min(max(x0 + lx, 0), G.W - 1);
    const int o = (sy * G.W + sx) * (int)sizeof(Tin);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if constexpr (sizeof(Tin) == 2)
        r.v[k][c] = (unsigned)__builtin_amdgcn_raw_buffer_load_b16(rs, o, c * plane, 0);
      else
        r.v[k][c] = __builtin_amdgcn_raw_buffer_load_b32(rs, o, c * plane, 0);
    }
  }
}
// FP16: (r, g) in the first dword, (b, 0) in the second (the loads zero-extend); the packing is a
// volatile asm so that it stays here.  FP32: the bits.
__device__ __forceinline__ void rgb_put(h4* d, unsigned a, unsigned b, unsigned c) {
  unsigned rg;
  asm volatile("v_perm_b32 %0, %1, %2, %3" : "=v"(rg) : "v"(b), "v"(a), "s"(0x05040100u));
  *reinterpret_cast<u2*>(d) = u2{rg, c};
}
__device__ __forceinline__ void rgb_put(float4* d, unsigned a, unsigned b, unsigned c) {
  *d = make_float4(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b), __builtin_bit_cast(float, c), 0.f);
}
template <typename Tin, typename Rgb, typename LY>
__device__ __forceinline__ void rgb_store(const RgbRegs<Tin, LY>& r, Rgb* lds_rgb, int ctid) {
#pragma unroll
  for (int k = 0; k < LY::RgbPer; ++k) {
    const int q = ctid + LY::ConsumerThreads * k;
    if (q < LY::RPos) rgb_put(lds_rgb + q, r.v[k][0], r.v[k][1], r.v[k][2]);
  }
}


// Output stores through a raw buffer resource covering one frame: lanes whose pixel lies
// outside the frame get an offset past the range and the hardware drops their store, so
// the stores need no branch (raw-buffer range checking: offset >= num_records is not
// written).  A frame is at most 3 x 8192^2 x 4 x 4 bytes < 2^32.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t frame_rsrc(void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)(unsigned)bytes, kRawBufferWord3);
}
// The output frame is written once and not read back by this kernel: its stores carry the
// non-temporal hint (cache-policy bit 1), which keeps them from displacing the work tensor and
// frames that the launch still reads (head -0.8 us at 1080p, A/B on one box).
constexpr int kStoreNonTemporal = 2;
template <typename Tout>
__device__ __forceinline__ void fstore_pair(__amdgpu_buffer_rsrc_t r, unsigned off, float left, float right);
template <>
__device__ __forceinline__ void fstore_pair<_Float16>(__amdgpu_buffer_rsrc_t r, unsigned off, float left, float right) {
  __builtin_amdgcn_raw_buffer_store_b32(pack_h2(left, right), r, (int)off, 0, kStoreNonTemporal);
}
template <>
__device__ __forceinline__ void fstore_pair<float>(__amdgpu_buffer_rsrc_t r, unsigned off, float left, float right) {
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(v2u{__builtin_bit_cast(unsigned, left), __builtin_bit_cast(unsigned, right)},
                                        r, (int)off, 0, kStoreNonTemporal);
}

// Head on LR row `r` of the tile.  The four 16-pixel chunks are computed unconditionally
// (every LDS address stays inside the tile buffers), so the row is one basic block the
// scheduler can interleave; chunks or lanes past the frame edge only lose their stores.
// QC: A23 is unused and BC holds the lane group's FP32 base per row tile; otherwise BC is unused.
// `mid` is called once per row, after the second chunk's arithmetic and before any output store
// is issued (at once for a row outside the frame): the caller stores the next tile's RGB there,
// so that waiting for its loads does not also wait for this row's output stores, which are
// counted by the same counter.
template <typename Tout, typename Rgb, bool QC, typename Mid>
__device__ __forceinline__ void consume_row(const unsigned char* lds_meta, const Rgb* lds_rgb, Tout* __restrict__ out,
                                            FusedTile t, const FusedGeom& G, int r, int lane, const h8 (&A1)[7],
                                            const h8 (&A23)[7], const f4 (&BC)[7], const unsigned ones, float& chk,
                                            Mid&& mid) {
  const int n = lane & 15, g = lane >> 4;
  const int y = 2 * t.qy0 + r - G.py;
  if (y < 0 || y >= G.H) {                            // wave-uniform
    mid();
    return;
  }
  const size_t oplane = (size_t)4 * G.H * G.W;
  const __amdgpu_buffer_rsrc_t ob = frame_rsrc(out + (size_t)t.b * 3 * oplane, 3 * oplane * sizeof(Tout));
  const _Float16* mrow = reinterpret_cast<const _Float16*>(lds_meta) + (r >> 1) * kFQW * kFMPix;
  const int rho_y = (r & 1) << 1;
  unsigned sv01[kFLW / 16], sv2[kFLW / 16], so01[kFLW / 16], so2[kFLW / 16];
#pragma unroll
  for (int j = 0; j < kFLW / 16; ++j) {
    const int x = 2 * t.qx0 + 16 * j - G.px + n;
    const _Float16* cpix = mrow + (8 * j + (n >> 1)) * kFMPix + 16 * (rho_y | (n & 1));
    f4 acc[7];
    if constexpr (QC) {
      // B slots 8g..8g+7 = clamped coefficients 8(g&1)..+7 (slots 16..31 repeat 0..15 for K_lo)
      const h8 bop = *reinterpret_cast<const h8*>(cpix + 8 * (g & 1));
#pragma unroll
      for (int q = 0; q < 7; ++q) acc[q] = mfma_f16(A1[q], bop, BC[q]);
    } else {
      const u2 coef = *reinterpret_cast<const u2*>(cpix + 4 * g);
      unsigned U[2], Wd[2];
      coef_clamp_split(coef[0], U[0], Wd[0]);
      coef_clamp_split(coef[1], U[1], Wd[1]);
      unsigned Ux[2] = {U[0], U[1]}, Uy[2] = {U[0], U[1]};
#pragma unroll
      for (int w = 0; w < 2; ++w) permlane32_swap_mfma(Ux[w], Uy[w]);
#pragma unroll
      for (int w = 0; w < 2; ++w) permlane16_swap_mfma(Ux[w], Uy[w]);
      const u4 bu = {Ux[0], Ux[1], Uy[0], Uy[1]};
      const u4 bw = {Wd[0], Wd[1], ones, 0u};
      const h8 bop_u = __builtin_bit_cast(h8, bu);
      const h8 bop_w = __builtin_bit_cast(h8, bw);
#pragma unroll
      for (int q = 0; q < 7; ++q) {
        acc[q] = mfma_f16(A1[q], bop_u, f4{0.f, 0.f, 0.f, 0.f});
        acc[q] = mfma_f16(A23[q], bop_w, acc[q]);
      }
    }
    const Rgb* L0 = lds_rgb + r * kFRW + 16 * j + n;
    // phase g of pixel n: the 25 taps in order (dy, dx) = (tap / 5, tap % 5)
    float u[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int tap = 0; tap < 25; ++tap) {
      const Rgb L = L0[(tap / 5) * kFRW + tap % 5];
      const float wt = acc[tap >> 2][tap & 3];
      u[0] = fmaf(wt, (float)L.x, u[0]);
      u[1] = fmaf(wt, (float)L.y, u[1]);
      u[2] = fmaf(wt, (float)L.z, u[2]);
    }
    const bool inside = (unsigned)x < (unsigned)G.W;
    chk = fmaf(inside ? u[0] + u[1] + u[2] : 0.f, 0.0f, chk);
    // pair phases (TL, TR) and (BL, BR): after the swap lane groups 0 and 1 both hold
    // (TL, TR), groups 2 and 3 both hold (BL, BR).
    // Both lane groups of a row pair then hold the same values: groups 0 / 2 write channel 0 and
    // groups 1 / 3 channel 1 in one store, then groups 0 / 2 channel 2 (lanes with nothing to write
    // get an out-of-range offset).  FP16 output: a chunk writes 64 bytes per row and channel, so the
    // stores of chunks j - 1 and j are issued together and fill whole 128-byte lines; with the
    // non-temporal hint, half lines written apart were each sent to memory as a partial line
    // (write traffic 1.44x the output).
    const unsigned o0 = (unsigned)(((size_t)(2 * y + (g >> 1)) * (2 * G.W) + 2 * x) * sizeof(Tout));
    const int c01 = g & 1;
    const unsigned off01 = inside ? o0 + (unsigned)(c01 * oplane * sizeof(Tout)) : 0xFFFFFFFFu;
    const unsigned off2 = inside && c01 == 0 ? o0 + (unsigned)(2 * oplane * sizeof(Tout)) : 0xFFFFFFFFu;
    if constexpr (std::is_same<Tout, float>::value) {
      float left[3], right[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        left[c] = __builtin_amdgcn_fmed3f(u[c], 0.0f, 1.0f);
        right[c] = left[c];
        permlane16_swap(left[c], right[c]);
      }
      if (j == 0) mid();
      fstore_pair<Tout>(ob, off01, c01 ? left[1] : left[0], c01 ? right[1] : right[0]);
      fstore_pair<Tout>(ob, off2, left[2], right[2]);
    } else {
      // FP16 output: the lane's own phase is converted (with the [0, 1] clamp) before the swap, so
      // two swaps move (R, G) and (B, B) as FP16 pairs, and one byte permute per store picks the
      // left and right halves: (R_l, R_r) or (G_l, G_r) by the lane's channel, and (B_l, B_r).
      unsigned rgL = pack_h2_clamp01(u[0], u[1]), bbL = pack_h2_clamp01(u[2], u[2]);
      unsigned rgR = rgL, bbR = bbL;
      permlane16_swap_u(rgL, rgR);
      permlane16_swap_u(bbL, bbR);
      sv01[j] = __builtin_amdgcn_perm(rgR, rgL, c01 ? 0x07060302u : 0x05040100u);
      sv2[j] = __builtin_amdgcn_perm(bbR, bbL, 0x05040100u);
      so01[j] = off01;
      so2[j] = off2;
      if (j & 1) {
        if (j == 1) mid();
#pragma unroll
        for (int k = j - 1; k <= j; ++k) __builtin_amdgcn_raw_buffer_store_b32(sv01[k], ob, (int)so01[k], 0, kStoreNonTemporal);
#pragma unroll
        for (int k = j - 1; k <= j; ++k) __builtin_amdgcn_raw_buffer_store_b32(sv2[k], ob, (int)so2[k], 0, kStoreNonTemporal);
      }
    }
  }
}

// Producer waves: coefficients of tile i+1, work patch of tile i+2.
template <typename Tin, bool QC>
__device__ __forceinline__ void producer_main(unsigned char* smem, const _Float16* __restrict__ work,
                                              const FusedGeom& G, int wave, int lane, int ptid) {
  typedef FusedLayout<Tin> LY;
  const int t0 = tile_of(0, G.num_tiles), t1 = tile_of(1, G.num_tiles);
  {
    PatchRegs<LY> pr;
    if (t0 < G.num_tiles) {
      patch_fetch<LY>(pr, work, fused_tile<LY::QH>(t0, G), G, ptid);
      patch_store<LY>(pr, smem + LY::OffPatch, ptid);
    }
    if (t1 < G.num_tiles) {
      patch_fetch<LY>(pr, work, fused_tile<LY::QH>(t1, G), G, ptid);
      patch_store<LY>(pr, smem + LY::OffPatch + LY::SizePatch, ptid);
    }
  }
  lds_barrier();                                   // weights, biases and prologue loads visible
  lds_barrier();                                   // coefficients of tile 0 (the consumers') visible
  const int iters = tile_iters(G.num_tiles);
  for (int it = 0; it < iters; ++it) {
    if (tile_of(it, G.num_tiles) >= G.num_tiles) break;   // block-uniform, as in consumer_main
    const int tn = tile_of(it + 1, G.num_tiles), tnn = tile_of(it + 2, G.num_tiles);
    const int cur = it & 1, nxt = cur ^ 1;
    // patch and coefficient addresses are recomputed every tile (a few VALU ops); hoisted,
    // they were spilled and their reloads waited for the patch prefetch
    const int ptid_it = fresh(ptid), lane_it = fresh(lane);
    PatchRegs<LY> pr;
    if constexpr (LY::PH == 2 * kFProducers) {      // FP16 frames: the row-wise chunk mapping
      if (tnn < G.num_tiles) patch_fetch_rows<LY>(pr, work, fused_tile<LY::QH>(tnn, G), G, wave, lane_it);
    } else {
      if (tnn < G.num_tiles) patch_fetch<LY>(pr, work, fused_tile<LY::QH>(tnn, G), G, ptid_it);
    }
    if (tn < G.num_tiles)
      produce<LY, QC>(smem, smem + LY::OffPatch + nxt * LY::SizePatch, smem + LY::OffMeta + nxt * LY::SizeMeta,
                      wave, lane_it);
    if (tnn < G.num_tiles) {
      if constexpr (LY::PH == 2 * kFProducers) patch_store_rows<LY>(pr, smem + LY::OffPatch + cur * LY::SizePatch, wave, lane_it);
      else patch_store<LY>(pr, smem + LY::OffPatch + cur * LY::SizePatch, ptid_it);
    }
    lds_barrier();
  }
}

// Consumer waves: head of tile i, RGB tile of tile i+1.
template <typename Tin, typename Tout, bool QC>
__device__ __forceinline__ void consumer_main(unsigned char* smem, const Tin* __restrict__ src,
                                              const h8* __restrict__ bankA, Tout* __restrict__ out,
                                              const FusedGeom& G, int row, int lane, int ctid,
                                              unsigned* __restrict__ nonfinite) {
  typedef FusedLayout<Tin> LY;
  typedef typename FusedCfg<Tin>::Rgb Rgb;
  const int g = lane >> 4;
  h8 A1[7], A23[7];
  f4 BC[7];
  const f4* basec = reinterpret_cast<const f4*>(bankA + kHeadBankFrags * 64);
#pragma unroll
  for (int q = 0; q < 7; ++q) {
    A1[q] = bankA[q * 64 + lane];
    if constexpr (QC) BC[q] = basec[g * 7 + q];
    else A23[q] = bankA[(7 + q) * 64 + lane];
  }
  // The bank fragments are used first inside the tile loop.  Waiting for them here, on every
  // path into the loop, keeps the compiler from placing waits for them inside the loop, where
  // they would also wait for the RGB prefetch of the next tile.
#pragma unroll
  for (int q = 0; q < 7; ++q) {
    if constexpr (QC) asm volatile("" ::"v"(A1[q]), "v"(BC[q]));
    else asm volatile("" ::"v"(A1[q]), "v"(A23[q]));
  }
  const unsigned ones = g == 0 ? 0x3C003C00u : 0u;  // FP16 (1, 1) in B slots 4, 5 of lane group 0
  float chk = 0.f;
  const int t0 = tile_of(0, G.num_tiles);
  if (t0 < G.num_tiles) {
    RgbRegs<Tin, LY> rr;
    rgb_fetch<Tin, LY>(rr, src, fused_tile<LY::QH>(t0, G), G, ctid);
    rgb_store<Tin, Rgb, LY>(rr, reinterpret_cast<Rgb*>(smem + LY::OffRgb), ctid);
  }
  lds_barrier();                                   // prologue loads visible
  // tile 0's coefficients: one 16-pixel group per consumer wave (2 QH groups, 2 QH consumers)
  if (t0 < G.num_tiles) produce<LY, QC, 1>(smem, smem + LY::OffPatch, smem + LY::OffMeta, row, fresh(lane));
  lds_barrier();                                   // coefficients of tile 0 visible
  const int iters = tile_iters(G.num_tiles);
  for (int it = 0; it < iters; ++it) {
    const int tc = tile_of(it, G.num_tiles);
    if (tc >= G.num_tiles) break;                    // block-uniform, as in producer_main
    const int tn = tile_of(it + 1, G.num_tiles);
    const int cur = it & 1, nxt = cur ^ 1;
    RgbRegs<Tin, LY> rr;
    if (tn < G.num_tiles) rgb_fetch<Tin, LY>(rr, src, fused_tile<LY::QH>(tn, G), G, ctid);
    // the next tile's RGB buffer was last read before the previous barrier
    consume_row<Tout, Rgb, QC>(smem + LY::OffMeta + cur * LY::SizeMeta,
                               reinterpret_cast<const Rgb*>(smem + LY::OffRgb + cur * LY::SizeRgb), out,
                               fused_tile<LY::QH>(tc, G), G, row, lane, A1, A23, BC, ones, chk, [&]() {
                                 if (tn < G.num_tiles)
                                   rgb_store<Tin, Rgb, LY>(rr, reinterpret_cast<Rgb*>(smem + LY::OffRgb + nxt * LY::SizeRgb), ctid);
                               });
    lds_barrier();
  }
  if (nonfinite && __ballot(chk != chk) != 0ull && lane == 0) atomicOr(nonfinite, 1u);
}

// Every wave executes the same number of barriers: two in the prologue, one per tile.
template <typename Tin, typename Tout, bool QC>
__global__ __launch_bounds__(FusedLayout<Tin>::Threads) void fused_tail_head_kernel(
    const _Float16* __restrict__ work, const Tin* __restrict__ src, const h8* __restrict__ rt_frag,
    const float* __restrict__ rbias, const float* __restrict__ tbias, const h8* __restrict__ bankA,
    Tout* __restrict__ out, FusedGeom G, unsigned* __restrict__ nonfinite) {
  typedef FusedLayout<Tin> LY;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  {
    const u4* s = reinterpret_cast<const u4*>(rt_frag);
    u4* d = reinterpret_cast<u4*>(smem + LY::OffW);
    for (int i = tid; i < kFSizeW / 16; i += LY::Threads) d[i] = s[i];
    float* b = reinterpret_cast<float*>(smem + LY::OffBias);
    if (tid < 64) b[tid] = rbias[tid];
    else if (tid < 128) b[tid] = tbias[tid - 64];
  }
  if (wave < kFProducers)                            // wave-uniform role
    producer_main<Tin, QC>(smem, work, G, wave, lane, tid);
  else
    consumer_main<Tin, Tout, QC>(smem, src, bankA, out, G, wave - kFProducers, lane, tid - 64 * kFProducers,
                                 nonfinite);
}

static FusedGeom fused_geometry(int qh, int H, int W, int Hq, int Wq, int py, int px, int batch) {
  FusedGeom G;
  G.H = H; G.W = W; G.Hq = Hq; G.Wq = Wq; G.py = py; G.px = px; G.batch = batch;
  G.qy_lo = py >> 1;
  G.qx_lo = px >> 1;
  const int qy_hi = (py + H - 1) >> 1, qx_hi = (px + W - 1) >> 1;
  G.tiles_y = (qy_hi - G.qy_lo + qh) / qh;
  G.tiles_x = (qx_hi - G.qx_lo + kFQW) / kFQW;
  G.num_tiles = batch * G.tiles_y * G.tiles_x;
  return G;
}

int fused_num_tiles(int in_fp32, int batch, int H, int W, int Hq, int Wq, int py, int px) {
  const int qh = in_fp32 ? FusedCfg<float>::QH : FusedCfg<_Float16>::QH;
  return fused_geometry(qh, H, W, Hq, Wq, py, px, batch).num_tiles;
}

template <typename Tin, typename Tout, bool QC>
static hipError_t launch_fused_t(const void* work, const void* src, const void* rt_frag, const float* rbias,
                                 const float* tbias, const void* bankA, void* out, int H, int W, int Hq, int Wq,
                                 int py, int px, int batch, unsigned* nonfinite, int grid, hipStream_t stream) {
  typedef FusedLayout<Tin> LY;
  const FusedGeom G = fused_geometry(LY::QH, H, W, Hq, Wq, py, px, batch);
  hipLaunchKernelGGL((fused_tail_head_kernel<Tin, Tout, QC>), dim3(grid), dim3(LY::Threads), LY::Lds, stream,
                     (const _Float16*)work, (const Tin*)src, (const h8*)rt_frag, rbias, tbias, (const h8*)bankA,
                     (Tout*)out, G, nonfinite);
  return hipGetLastError();
}

// Allows the kernels' dynamic LDS above the default limit; called once per device at configure.
hipError_t fused_prepare() {
  const void* k[8] = {reinterpret_cast<const void*>(&fused_tail_head_kernel<float, float, false>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<float, _Float16, false>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, float, false>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, _Float16, false>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<float, float, true>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<float, _Float16, true>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, float, true>),
                      reinterpret_cast<const void*>(&fused_tail_head_kernel<_Float16, _Float16, true>)};
  const int lds[8] = {FusedLayout<float>::Lds,    FusedLayout<float>::Lds,    FusedLayout<_Float16>::Lds,
                      FusedLayout<_Float16>::Lds, FusedLayout<float>::Lds,    FusedLayout<float>::Lds,
                      FusedLayout<_Float16>::Lds, FusedLayout<_Float16>::Lds};
  for (int i = 0; i < 8; ++i) {
    const hipError_t e = hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds[i]);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_fused_tail_head(int in_fp32, int out_fp32, int qclamp, const void* work, const void* src,
                                  const void* rt_frag, const float* rbias, const float* tbias, const void* bankA,
                                  void* out, int H, int W, int Hq, int Wq, int py, int px, int batch,
                                  unsigned* nonfinite, int grid, hipStream_t stream) {
#define AEISU_FUSED(TI, TO, QC) \
  launch_fused_t<TI, TO, QC>(work, src, rt_frag, rbias, tbias, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, \
                             grid, stream)
  if (qclamp) {
    if (in_fp32 && out_fp32) return AEISU_FUSED(float, float, true);
    if (in_fp32) return AEISU_FUSED(float, _Float16, true);
    if (out_fp32) return AEISU_FUSED(_Float16, float, true);
    return AEISU_FUSED(_Float16, _Float16, true);
  }
  if (in_fp32 && out_fp32) return AEISU_FUSED(float, float, false);
  if (in_fp32) return AEISU_FUSED(float, _Float16, false);
  if (out_fp32) return AEISU_FUSED(_Float16, float, false);
  return AEISU_FUSED(_Float16, _Float16, false);
#undef AEISU_FUSED
}

}  // namespace aeisu
