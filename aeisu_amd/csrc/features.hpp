// Analysis features of one packed pixel: the 8 learned/directional features of each of its
// four LR pixels (aeisu/model.py:273-341, _rgb_to_feature8), in pixel_unshuffle order
// channel = feature * 4 + phase.  Shared by the standalone project kernel and the fused body,
// so both produce bit-identical features.
//
// Learned RGB and luma use explicitly unfused multiplies and adds in the reference's
// evaluation order, and the directional stencils are evaluated without contraction too, so
// the features equal those of the FP32 PyTorch model evaluated on the same input.
#pragma once
#include "common.hpp"

namespace aeisu {

struct Analysis {
  float basis[9], mix[3], dx[3], dy[3], d45[3], d135[3];
};

// Analysis constants from the 24-float table (basis 3x3, luma mix, dx, dy, d45, d135).
__host__ __device__ inline Analysis analysis_from(const float* a) {
  Analysis an;
  for (int i = 0; i < 9; ++i) an.basis[i] = a[i];
  for (int i = 0; i < 3; ++i) {
    an.mix[i] = a[9 + i];
    an.dx[i] = a[12 + i];
    an.dy[i] = a[15 + i];
    an.d45[i] = a[18 + i];
    an.d135[i] = a[21 + i];
  }
  return an;
}

__device__ __forceinline__ float sub_rn(float a, float b) { return a - b; }
// HIP's __fmul_rn / __fadd_rn are plain operators that the compiler may contract into FMAs
// (-ffp-contract=fast is the default): contraction is switched off here explicitly.
__device__ __forceinline__ float dot3_unfused(float3 v, float a, float b, float c) {
#pragma clang fp contract(off)
  return (v.x * a + v.y * b) + v.z * c;
}
// (p*a + q*b) + r*c, unfused, reference order
__device__ __forceinline__ float comb3(float p, float a, float q, float b, float r, float c) {
#pragma clang fp contract(off)
  return (p * a + q * b) + r * c;
}
// (u - d) * a0 - m * a1 + h * a2, evaluated left to right, unfused
__device__ __forceinline__ float d135_unfused(float u, float d, float m, float h, float a0, float a1, float a2) {
#pragma clang fp contract(off)
  return ((u - d) * a0 - m * a1) + h * a2;
}

// Luma of one LR pixel (the window luma of the stencil features).
__device__ __forceinline__ float luma(float r, float g, float b, const Analysis& an) {
  return dot3_unfused(make_float3(r, g, b), an.mix[0], an.mix[1], an.mix[2]);
}

// Features f[feature][phase] of a packed pixel from the luma lw[row][col] of its 4x4 LR window
// (one halo pixel on each side of its 2x2 LR pixels) and the RGB c[channel][i][j] of those 2x2
// pixels: the basis projections of each pixel and the 3x3 luma stencils centred on it.
__device__ __forceinline__ void luma_features(const float (&lw)[4][4], const float (&c)[3][2][2], const Analysis& an,
                                              float (&f)[8][4]) {
#pragma unroll
  for (int ph = 0; ph < 4; ++ph) {
    const int i = ph >> 1, j = ph & 1;
    const float3 v = make_float3(c[0][i][j], c[1][i][j], c[2][i][j]);   // this phase's pixel
    f[0][ph] = dot3_unfused(v, an.basis[0], an.basis[1], an.basis[2]);
    f[1][ph] = dot3_unfused(v, an.basis[3], an.basis[4], an.basis[5]);
    f[2][ph] = dot3_unfused(v, an.basis[6], an.basis[7], an.basis[8]);
    const float ul = lw[i][j], uc = lw[i][j + 1], ur = lw[i][j + 2];
    const float cl = lw[i + 1][j], cc = lw[i + 1][j + 1], cr = lw[i + 1][j + 2];
    const float dl = lw[i + 2][j], dc = lw[i + 2][j + 1], dr = lw[i + 2][j + 2];
    const float hmid = sub_rn(cr, cl), vmid = sub_rn(dc, uc);
    f[3][ph] = cc;
    f[4][ph] = comb3(sub_rn(ur, ul), an.dx[0], hmid, an.dx[1], sub_rn(dr, dl), an.dx[2]);
    f[5][ph] = comb3(sub_rn(dl, ul), an.dy[0], vmid, an.dy[1], sub_rn(dr, ur), an.dy[2]);
    f[6][ph] = comb3(sub_rn(dr, ul), an.d45[0], vmid, an.d45[1], hmid, an.d45[2]);
    f[7][ph] = d135_unfused(ur, dl, vmid, hmid, an.d135[0], an.d135[1], an.d135[2]);
  }
}

// The same from the 4x4 LR window w[channel][row][col] itself.
__device__ __forceinline__ void window_features(const float (&w)[3][4][4], const Analysis& an, float (&f)[8][4]) {
  float lw[4][4], c[3][2][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) lw[a][b] = luma(w[0][a][b], w[1][a][b], w[2][a][b], an);
#pragma unroll
  for (int ch = 0; ch < 3; ++ch)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) c[ch][i][j] = w[ch][i + 1][j + 1];
  luma_features(lw, c, an, f);
}

// The same from LDS: channel c of window pixel (a, b) is p[c * plane + a * rs + b].
__device__ __forceinline__ void packed_features(const float* p, int plane, int rs, const Analysis& an,
                                                float (&f)[8][4]) {
  float w[3][4][4];
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) w[c][a][b] = p[c * plane + a * rs + b];
  window_features(w, an, f);
}

// The 32 features as four MFMA operand slices (slice q = features 2q, 2q+1 at the four
// phases: the K slots 8q..8q+7 of the project weights), rounded to FP16; `lo` receives the
// FP16 residuals x - hi for the FP32-accurate hi/lo product.
template <bool WITH_LO>
__device__ __forceinline__ void feature_slices(const float (&f)[8][4], h8 (&hi)[4], h8 (&lo)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = f[2 * q + (e >> 2)][e & 3];
      hi[q][e] = (_Float16)x;
      if constexpr (WITH_LO) lo[q][e] = (_Float16)(x - (float)hi[q][e]);
    }
}

}  // namespace aeisu
