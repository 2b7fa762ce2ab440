// Reconstruction head: coefficient clamp, per-pixel filter synthesis, 5x5
// RGB application, 2x phase write -- one fused pass.
//
// Math (aeisu/reconstruction.py:15-83; native ReconstructConstant,
// optimized/native/src/neural/adaptive/AdaptiveReconstruction.cuh:288-417):
//   a_k   = clamp(meta[(Y/2, X/2)][16*rho + k]),  rho = 2*(Y&1) + (X&1) on the padded grid
//   W[t,ph] = base[t,ph] + sum_k a_k * bank[t,k,ph]                (t: 25 taps, ph: 4 phases)
//   out[c, 2y + ph/2, 2x + ph%2] = clamp01( sum_t W[t,ph] * src[c, clamp(y+dy_t), clamp(x+dx_t)] )
//
// gfx950 mapping.  One wave handles 16 consecutive LR pixels of a row per chunk.
//  * Clamp without FP32 arithmetic: with s = sign(v),
//      clamp(v) = u + 0.05 w,   u = s min(|v|, 2),   w = s max(min(|v|, 12) - 2, 0),
//    where u and w are exact FP16 values computed with packed FP16 / u16 operations
//    (NaN coefficients keep a NaN u).  Lane (n, g) splits coefficients 4g..4g+3 of
//    pixel n, i.e. each coefficient once per wave.
//  * Synthesis on MFMA, two dependent 16x16x32 f16 MFMAs per row tile (FP32 accumulation),
//    D[112 x 16] rows = (tap, phase), columns = pixels:
//      [K_hi | K_lo] . [u ; u]             u regrouped across lane groups by two permlane
//                                          swaps (B slots 8g..8g+7 = u[8(g&1)..+7])
//      A23 . [w_g, (1, 1 if g = 0), 0, 0]  B slots 8g..8g+3 = the lane's own w (no exchange),
//                                          A23 slots 8g..8g+3 = (0.05 K)_hi of coefficients
//                                          4g..4g+3, slots 4, 5 = base_hi, base_lo
//    W = base + K u + 0.05 K w with the FP32 bank and base kept to ~2^-22 relative; only
//    0.05 K is rounded to FP16 (2^-12 relative on the clamp excess, which is <= 0.5 in the
//    coefficient and present only for |a| > 2).  Both MFMAs have the same shape: a chain of
//    different shapes through SrcC needs wait states the compiler does not insert here.
//  * Row layout (packed on the host): row 4g+i of tile t = (phase g, tap 4t+i), taps
//    25..27 zero.  Accumulator lane (n, g) therefore holds W for pixel n, phase g, all 25
//    taps: it applies them to the 3 channels with FP32 FMAs in tap order from an LDS RGB
//    tile (lanes of one pixel read the same LDS words), with no cross-lane reduction.
//  * Pipelining: a block walks tiles of 64x4 LR pixels; the RGB tile (with a
//    2-pixel clamped halo) and each lane's FP16 coefficients of the NEXT tile
//    are loaded into registers while the current tile is computed, and the RGB
//    tile is double-buffered in LDS (one barrier per tile).
//  * Quantized policies (QC): the clamp is coef_clamp_h16 (the clamped coefficient rounded to
//    FP16, <= 1.2e-4 + half an FP16 ulp from the FP32 clamp, only for |a| > 2).  Lane (n, g)
//    reads and clamps coefficients 8(g&1)..+7 itself (no exchange), and each row tile takes ONE
//    MFMA, [K_hi | K_lo] . [c ; c], with the FP32 base of its rows as the accumulator input
//    (bank image: the 14 fragments, then base[g][t] as 4 x 7 float4).
//  * Output: lane groups (0, 1) and (2, 3) hold horizontally adjacent output pixels
//    (phases TL/TR, BL/BR); one permlane16 swap pairs them, so groups 0 and 2 each store
//    two values per channel.  A per-lane
//    running sum 0 * output (NaN for any non-finite output) sets the nonfinite
//    flag once per wave at the end.
#include "common.hpp"
#include "kernels.hpp"

namespace aeisu {

constexpr int kHeadTW = 64, kHeadTH = 4;
constexpr int kHeadLW = kHeadTW + 4, kHeadLH = kHeadTH + 4;
constexpr int kHeadLPos = kHeadLW * kHeadLH;              // RGB positions per tile (with halo)
constexpr int kHeadFill = (kHeadLPos + 255) / 256;        // positions loaded per thread
constexpr int kHeadChunks = kHeadTW / 16;

template <typename Tin>
__device__ __forceinline__ float load_px(const Tin* p) { return (float)*p; }


struct HeadTile {
  int b, y0, x0;
};
__device__ __forceinline__ HeadTile head_tile(int tidx, int tiles_x, int tiles_y) {
  HeadTile t;
  t.b = tidx / (tiles_y * tiles_x);
  const int rem = tidx - t.b * tiles_y * tiles_x;
  t.y0 = (rem / tiles_x) * kHeadTH;
  t.x0 = (rem % tiles_x) * kHeadTW;
  return t;
}

// Registers holding one tile's inputs ahead of its computation.
template <bool QC>
struct HeadPrefetch {
  float rgb[kHeadFill][3];   // this thread's share of the clamped RGB tile
  // this lane's FP16 coefficients for each chunk of its row: 4g..4g+3, or 8(g&1)..+7 (QC)
  typename std::conditional<QC, u4, u2>::type coef[kHeadChunks];
};

template <bool QC, typename Tin>
__device__ __forceinline__ void head_fetch(HeadPrefetch<QC>& p, const Tin* __restrict__ src,
                                           const _Float16* __restrict__ meta, HeadTile t, int H, int W,
                                           int Hq, int Wq, int py, int px, int wave, int n, int g) {
  const size_t plane = (size_t)H * W;
  const Tin* s = src + (size_t)t.b * 3 * plane;
#pragma unroll
  for (int k = 0; k < kHeadFill; ++k) {
    const int q = threadIdx.x + 256 * k;
    if (q < kHeadLPos) {
      const int ly = q / kHeadLW, lx = q - ly * kHeadLW;
      const int sy = min(max(t.y0 + ly - 2, 0), H - 1), sx = min(max(t.x0 + lx - 2, 0), W - 1);
      const size_t o = (size_t)sy * W + sx;
      p.rgb[k][0] = load_px(s + o);
      p.rgb[k][1] = load_px(s + plane + o);
      p.rgb[k][2] = load_px(s + 2 * plane + o);
    }
  }
  // Rows / columns past the frame edge are clamped so every load stays inside the tensor;
  // the clamped chunks are never stored.
  const int Y = min(t.y0 + wave, H - 1) + py;
  const _Float16* mrow = meta + ((size_t)t.b * Hq + (Y >> 1)) * Wq * 64;
#pragma unroll
  for (int j = 0; j < kHeadChunks; ++j) {
    const int X = min(t.x0 + 16 * j + n, W - 1) + px;
    const int rho = ((Y & 1) << 1) | (X & 1);
    const _Float16* c = mrow + (size_t)(X >> 1) * 64 + 16 * rho;
    if constexpr (QC) p.coef[j] = *reinterpret_cast<const u4*>(c + 8 * (g & 1));
    else p.coef[j] = *reinterpret_cast<const u2*>(c + 4 * g);
  }
}

template <typename Tout>
__device__ __forceinline__ void store_pair(Tout* p, float left, float right);
template <>
__device__ __forceinline__ void store_pair<_Float16>(_Float16* p, float left, float right) {
  *reinterpret_cast<unsigned*>(p) = pack_h2(left, right);
}
template <>
__device__ __forceinline__ void store_pair<float>(float* p, float left, float right) {
  *reinterpret_cast<float2*>(p) = make_float2(left, right);
}

template <typename Tin, typename Tout, bool QC>
__global__ __launch_bounds__(256, 3) void head_kernel(
    const Tin* __restrict__ src, const _Float16* __restrict__ meta, const h8* __restrict__ bankA,
    Tout* __restrict__ out, int H, int W, int Hq, int Wq, int py, int px, int batch,
    unsigned* __restrict__ nonfinite) {
  __shared__ float4 tiles[2][kHeadLPos];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  h8 A1[7], A23[7];  // [K_hi | K_lo] and [(0.05K)_hi of 4g..4g+3, base_hi, base_lo, 0, 0] per lane group
  f4 BC[7];          // QC: FP32 base of the lane group's rows per row tile (instead of A23)
  const f4* basec = reinterpret_cast<const f4*>(bankA + kHeadBankFrags * 64);
#pragma unroll
  for (int t = 0; t < 7; ++t) {
    A1[t] = bankA[t * 64 + lane];
    if constexpr (QC) BC[t] = basec[g * 7 + t];
    else A23[t] = bankA[(7 + t) * 64 + lane];
  }
  const unsigned ones = g == 0 ? 0x3C003C00u : 0u;  // FP16 (1, 1) in B slots 4, 5 of lane group 0
  float chk = 0.f;   // 0 * every output of this lane: NaN iff one was not finite

  const int tiles_x = (W + kHeadTW - 1) / kHeadTW, tiles_y = (H + kHeadTH - 1) / kHeadTH;
  const int num_tiles = batch * tiles_y * tiles_x;
  const int iters = tile_iters(num_tiles);
  const size_t oplane = (size_t)4 * H * W;

  int tidx = tile_of(0, num_tiles);
  HeadPrefetch<QC> cur;
  if (tidx < num_tiles)
    head_fetch(cur, src, meta, head_tile(tidx, tiles_x, tiles_y), H, W, Hq, Wq, py, px, wave, n, g);

  for (int it = 0; it < iters; ++it) {
    if (tidx >= num_tiles) break;                    // block-uniform
    const HeadTile t = head_tile(tidx, tiles_x, tiles_y);
    float4* buf = tiles[it & 1];
#pragma unroll
    for (int k = 0; k < kHeadFill; ++k) {
      const int q = threadIdx.x + 256 * k;
      if (q < kHeadLPos) buf[q] = make_float4(cur.rgb[k][0], cur.rgb[k][1], cur.rgb[k][2], 0.f);
    }
    const typename std::conditional<QC, u4, u2>::type coef[kHeadChunks] = {cur.coef[0], cur.coef[1], cur.coef[2],
                                                                            cur.coef[3]};
    const int ntidx = tile_of(it + 1, num_tiles);
    if (ntidx < num_tiles)
      head_fetch(cur, src, meta, head_tile(ntidx, tiles_x, tiles_y), H, W, Hq, Wq, py, px, wave, n, g);
    lds_barrier();                                 // buf complete; the other buffer is free again

    const int y = t.y0 + wave;
    if (y < H) {                                     // wave-uniform
      Tout* ob = out + (size_t)t.b * 3 * oplane;
#pragma unroll
      for (int j = 0; j < kHeadChunks; ++j) {
        if (t.x0 + 16 * j >= W) break;               // wave-uniform
        const int x = t.x0 + 16 * j + n;
        f4 acc[7];
        if constexpr (QC) {
          // coefficients 8(g&1)..+7 of pixel n, clamped: B slots 8g..8g+7 (K_lo repeats K_hi's)
          const u4 cw = {coef_clamp_h16(coef[j][0]), coef_clamp_h16(coef[j][1]), coef_clamp_h16(coef[j][2]),
                         coef_clamp_h16(coef[j][3])};
          const h8 bop = __builtin_bit_cast(h8, cw);
#pragma unroll
          for (int r = 0; r < 7; ++r) acc[r] = mfma_f16(A1[r], bop, BC[r]);
        } else {
          // coefficients 4g..4g+3 of pixel n -> (u, w) halves
          unsigned U[2], Wd[2];
          coef_clamp_split(coef[j][0], U[0], Wd[0]);
          coef_clamp_split(coef[j][1], U[1], Wd[1]);
          // u of groups 0..3 -> group g holds u[8(g&1) .. 8(g&1)+7]
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
          for (int r = 0; r < 7; ++r) {
            acc[r] = mfma_f16(A1[r], bop_u, f4{0.f, 0.f, 0.f, 0.f});
            acc[r] = mfma_f16(A23[r], bop_w, acc[r]);
          }
        }
        const float4* L0 = buf + wave * kHeadLW + 16 * j + n;
        // phase g of pixel n: the 25 taps in order (dy, dx) = (tap / 5, tap % 5)
        float u[3] = {0.f, 0.f, 0.f};
#pragma unroll
        for (int tap = 0; tap < 25; ++tap) {
          const float4 L = L0[(tap / 5) * kHeadLW + tap % 5];
          const float wt = acc[tap >> 2][tap & 3];
          u[0] = fmaf(wt, L.x, u[0]);
          u[1] = fmaf(wt, L.y, u[1]);
          u[2] = fmaf(wt, L.z, u[2]);
        }
        chk = fmaf(u[0] + u[1] + u[2], 0.0f, chk);
        // pair phases (TL, TR) in lane group 0 and (BL, BR) in lane group 2
        float left[3], right[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          left[c] = __builtin_amdgcn_fmed3f(u[c], 0.0f, 1.0f);
          right[c] = left[c];
          permlane16_swap(left[c], right[c]);
        }
        if ((g & 1) == 0 && x < W) {
          Tout* p = ob + (size_t)(2 * y + (g >> 1)) * (2 * W) + 2 * x;
#pragma unroll
          for (int c = 0; c < 3; ++c) store_pair<Tout>(p + c * oplane, left[c], right[c]);
        }
      }
    }
    tidx = ntidx;
  }
  if (nonfinite && __ballot(chk != chk) != 0ull && lane == 0) atomicOr(nonfinite, 1u);
}

template <typename Tin, typename Tout, bool QC>
hipError_t launch_head_t(const void* src, const void* meta, const void* bankA, void* out, int H, int W,
                         int Hq, int Wq, int py, int px, int batch, unsigned* nonfinite, int grid,
                         hipStream_t stream) {
  hipLaunchKernelGGL((head_kernel<Tin, Tout, QC>), dim3(grid), dim3(256), 0, stream, (const Tin*)src,
                     (const _Float16*)meta, (const h8*)bankA, (Tout*)out, H, W, Hq, Wq, py, px, batch,
                     nonfinite);
  return hipGetLastError();
}

int head_num_tiles(int batch, int H, int W) {
  return batch * ((H + kHeadTH - 1) / kHeadTH) * ((W + kHeadTW - 1) / kHeadTW);
}

hipError_t launch_head(int in_fp32, int out_fp32, int qclamp, const void* src, const void* meta, const void* bankA,
                       void* out, int H, int W, int Hq, int Wq, int py, int px, int batch,
                       unsigned* nonfinite, int grid, hipStream_t stream) {
#define AEISU_HEAD(TI, TO, QC) \
  launch_head_t<TI, TO, QC>(src, meta, bankA, out, H, W, Hq, Wq, py, px, batch, nonfinite, grid, stream)
  if (qclamp) {
    if (in_fp32 && out_fp32) return AEISU_HEAD(float, float, true);
    if (in_fp32) return AEISU_HEAD(float, _Float16, true);
    if (out_fp32) return AEISU_HEAD(_Float16, float, true);
    return AEISU_HEAD(_Float16, _Float16, true);
  }
  if (in_fp32 && out_fp32) return AEISU_HEAD(float, float, false);
  if (in_fp32) return AEISU_HEAD(float, _Float16, false);
  if (out_fp32) return AEISU_HEAD(_Float16, float, false);
  return AEISU_HEAD(_Float16, _Float16, false);
#undef AEISU_HEAD
}

template <bool QC>
static hipError_t head_occupancy(int& n, int in_fp32, int out_fp32) {
  if (in_fp32 && out_fp32) return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<float, float, QC>, 256, 0);
  if (in_fp32) return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<float, _Float16, QC>, 256, 0);
  if (out_fp32) return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<_Float16, float, QC>, 256, 0);
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, head_kernel<_Float16, _Float16, QC>, 256, 0);
}

int head_blocks_per_cu(int in_fp32, int out_fp32, int qclamp) {
  int n = 0;
  const hipError_t e = qclamp ? head_occupancy<true>(n, in_fp32, out_fp32) : head_occupancy<false>(n, in_fp32, out_fp32);
  return e == hipSuccess && n > 0 ? n : 1;
}

}  // namespace aeisu
