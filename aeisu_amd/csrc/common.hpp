// Shared device helpers for the gfx950 (CDNA4) AEISU kernels.
//
// Conventions used by every kernel in this directory:
//  * Activations live in HBM as NHWC tiles: skip/work = FP16 [B][Hq][Wq][32],
//    low = FP16/E4M3/INT8 [B][Hl][Wl][64], meta = FP16 [B][Hq][Wq][64].
//  * MFMA 16x16 tiles: operand lane l holds row/column (l & 15) and the
//    K-slots 8*(l>>4)..+7 (f16 / fp8 K=32) or 16*(l>>4)..+15 (i8 K=64);
//    the accumulator lane l holds column (l & 15), rows 4*(l>>4)+r, r=0..3.
//    Weight matrices are pre-permuted on the host so that each lane's
//    K-slots map to contiguous activation channels.
//  * Kernels are persistent over tiles: blocks walk tiles with a stride of
//    gridDim.x, so weights are staged into registers once per wave.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <type_traits>

namespace aeisu {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i8v __attribute__((ext_vector_type(8)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));

constexpr float kE4M3Max = 448.0f;
// Word 3 of a raw (untyped, stride 0) buffer resource: DATA_FORMAT = 32 bit (bits 18:15 = 4), the
// only field untyped loads and stores need non-zero; offsets at or past num_records are dropped
// on stores and read as zero on loads.
constexpr int kRawBufferWord3 = 0x00020000;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// A copy of a per-lane index that the compiler cannot see through, so addresses derived from
// it are recomputed where they are used instead of being hoisted out of a loop or across
// phases.  Hoisted addresses in a kernel near its register limit are spilled, and each
// scratch reload then waits for every memory load issued before it (the memory counter
// retires in order), which serialises prefetches.
__device__ __forceinline__ int fresh(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ f4 mfma_f16(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_f16_k16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_fp8(long a, long b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i4 mfma_i8(i4 a, i4 b, i4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Cross-row lane exchanges of CDNA4 (v_permlane32_swap: lanes 32-63 of x <-> lanes 0-31 of y;
// v_permlane16_swap: odd 16-lane rows of x <-> even rows of y).  Both registers are written.
// Written as inline asm on purpose: with the ROCm 7.2 compiler the
// __builtin_amdgcn_permlane{16,32}_swap builtin is treated as writing only its first result
// (adding the two results is compiled into r[0] + r[0]).  Inline asm is opaque to the hazard
// recognizer, so the asm carries the wait states itself: two before the swap (a VALU write of
// either operand must settle; without them the swap reads partially updated operands) and,
// in the *_mfma variants whose results feed an MFMA operand, five after it (the MFMA reads
// its operands through a path that does not interlock with the swap's writes).
#define AEISU_SWAP_ASM(op) asm volatile("s_nop 1\n\t" op " %0, %1" : "+v"(x), "+v"(y))
#define AEISU_SWAP_ASM_MFMA(op) asm volatile("s_nop 1\n\t" op " %0, %1\n\ts_nop 4" : "+v"(x), "+v"(y))
__device__ __forceinline__ void permlane32_swap(float& x, float& y) { AEISU_SWAP_ASM("v_permlane32_swap_b32"); }
__device__ __forceinline__ void permlane16_swap(float& x, float& y) { AEISU_SWAP_ASM("v_permlane16_swap_b32"); }
__device__ __forceinline__ void permlane32_swap_u(unsigned& x, unsigned& y) { AEISU_SWAP_ASM("v_permlane32_swap_b32"); }
__device__ __forceinline__ void permlane16_swap_u(unsigned& x, unsigned& y) { AEISU_SWAP_ASM("v_permlane16_swap_b32"); }
__device__ __forceinline__ void permlane32_swap_mfma(unsigned& x, unsigned& y) {
  AEISU_SWAP_ASM_MFMA("v_permlane32_swap_b32");
}
__device__ __forceinline__ void permlane16_swap_mfma(unsigned& x, unsigned& y) {
  AEISU_SWAP_ASM_MFMA("v_permlane16_swap_b32");
}
#undef AEISU_SWAP_ASM
#undef AEISU_SWAP_ASM_MFMA

// LeakyReLU as written by the reference epilogues: negative inputs scaled by the slope
// (v < 0 ? v * slope : v).  For 0 <= slope <= 1 that is max(v, v * slope) bit for bit: a
// negative v gives v * slope >= v (the rounded product cannot exceed |v| in magnitude), a
// non-negative v gives v >= v * slope, and -0 * slope = -0; two VALU ops instead of three.
__device__ __forceinline__ float leaky(float v, float slope) { return __builtin_fmaxf(v, v * slope); }

// Workgroup barrier for data handed over through LDS: waits for this wave's LDS operations
// only.  __syncthreads() also waits for every outstanding global load and store (on gfx9
// vmcnt counts both), which would drain prefetches issued just before it and stall each
// tile on the write acknowledgements of its output.  The memory clobber keeps the compiler
// from moving LDS accesses across the barrier.  Global data that feeds LDS stores is waited
// for at those stores (register dependency), before the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Next work item of a phase for this wave: the first items are dealt statically (one per wave),
// the rest are claimed from a counter in LDS.  A SIMD issues its older waves first, so with a
// static split the youngest waves finish last and run alone at the end of the phase; claimed
// items let the waves that are issued more often take more, and all waves leave together.
__device__ __forceinline__ int claim_group(int* counter, int lane) {
  int v = 0;
  if (lane == 0) v = atomicAdd(counter, 1);
  return __builtin_amdgcn_readfirstlane(v);
}

// float -> OCP E4M3 with round-to-nearest-even and saturation to +-448.
// The hardware convert rounds to nearest even but yields NaN above the
// saturation threshold, so the value is clamped first.
__device__ __forceinline__ unsigned pack_e4m3x2(float a, float b) {
  a = __builtin_amdgcn_fmed3f(a, -kE4M3Max, kE4M3Max);
  b = __builtin_amdgcn_fmed3f(b, -kE4M3Max, kE4M3Max);
  return (unsigned)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}
__device__ __forceinline__ unsigned pack_e4m3x4(float a, float b, float c, float d) {
  a = __builtin_amdgcn_fmed3f(a, -kE4M3Max, kE4M3Max);
  b = __builtin_amdgcn_fmed3f(b, -kE4M3Max, kE4M3Max);
  c = __builtin_amdgcn_fmed3f(c, -kE4M3Max, kE4M3Max);
  d = __builtin_amdgcn_fmed3f(d, -kE4M3Max, kE4M3Max);
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);     // bytes 0, 1
  return (unsigned)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);  // bytes 2, 3; keeps 0, 1
}
// E4M3 byte SEL of word w -> float (exact).
template <int SEL>
__device__ __forceinline__ float e4m3_to_f32(unsigned w) {
  return __builtin_amdgcn_cvt_f32_fp8((int)w, SEL);
}

// Eight E4M3 codes (bytes of w[0], w[1]) -> eight FP16 values.  Every E4M3 value is exactly
// representable in FP16 (3-bit mantissa, exponents 2^-9 .. 2^8), so the conversion is exact.
// v_cvt_scalef32_pk_f16_fp8 with scale 1.0 converts two codes per instruction (byte 2s of the
// word -> low half, byte 2s+1 -> high half); it agrees bit for bit with the two-step
// E4M3 -> FP32 -> FP16 conversion on all 65536 code pairs (checked on gfx950).
__device__ __forceinline__ h8 e4m3x8_to_h8(unsigned w0, unsigned w1) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  const h2v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, false);
  const h2v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, true);
  const h2v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, false);
  const h2v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, true);
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Symmetric INT8: clamp(rint(v * inv), -127, 127)  (rint = round half to even).
__device__ __forceinline__ int quant_s8(float v, float inv) {
  float q = __builtin_rintf(v * inv);
  q = __builtin_amdgcn_fmed3f(q, -127.0f, 127.0f);
  return (int)q;
}
__device__ __forceinline__ unsigned pack_s8x4(int a, int b, int c, int d) {
  return (unsigned)(a & 255) | ((unsigned)(b & 255) << 8) | ((unsigned)(c & 255) << 16) |
         ((unsigned)(d & 255) << 24);
}
// quant_s8 of a product x = fl32(v * inv) in the low byte of the returned word: x is clamped to
// [-127, 127] and 1.5 * 2^23 added.  The sum lies in [2^23, 2^24), where the unit in the last place
// is 1, so the addition rounds x to the nearest integer, ties to even (rint), and leaves that integer
// in the low mantissa bits in two's complement: the word is 0x4B400000 + q.  Clamping before
// rounding gives the same code as after it, the bounds being integers.  Two instructions instead of
// rint, clamp and a float -> int conversion.
__device__ __forceinline__ unsigned s8_code_word(float x) {
  return __builtin_bit_cast(unsigned, __builtin_amdgcn_fmed3f(x, -127.0f, 127.0f) + 12582912.0f);
}
// Low bytes of four words, a in byte 0 .. d in byte 3 (two v_perm_b32 and an or).
__device__ __forceinline__ unsigned pack_low_bytes4(unsigned a, unsigned b, unsigned c, unsigned d) {
  return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | __builtin_amdgcn_perm(d, c, 0x04000c0cu);
}
// Four INT8 codes (quant_s8 of the products a..d), packed as pack_s8x4 packs them.
__device__ __forceinline__ unsigned quant_s8x4(float a, float b, float c, float d) {
  return pack_low_bytes4(s8_code_word(a), s8_code_word(b), s8_code_word(c), s8_code_word(d));
}

__device__ __forceinline__ unsigned short f2h_bits(float v) {
  _Float16 h = (_Float16)v;
  return __builtin_bit_cast(unsigned short, h);
}
// Two FP32 values -> FP16 pair with one v_cvt_pk_f16_f32 (round to nearest even; identical
// to two scalar conversions for all 2^32 inputs, checked exhaustively on gfx950).
__device__ __forceinline__ unsigned pack_h2(float a, float b) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(unsigned, __builtin_convertvector((f2v){a, b}, h2v));
}
// pack_h2(clamp01(a), clamp01(b)) in one instruction: the clamp output modifier of the packed
// convert equals fmed3(x, 0, 1) before the conversion for all 2^32 inputs, NaN -> 0 included
// (checked exhaustively on gfx950).
__device__ __forceinline__ unsigned pack_h2_clamp01(float a, float b) {
  unsigned r;
  asm("v_cvt_pk_f16_f32 %0, %1, %2 clamp" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// gfx950's v_pk_minimum3_f16: per half, the IEEE 754-2019 minimum of three FP16 values (a NaN
// operand gives a quiet NaN, unlike v_pk_min_f16, which returns the other operand).
__device__ __forceinline__ unsigned pk_minimum3_h16(unsigned a, unsigned b, unsigned c) {
  unsigned r;
  asm("v_pk_minimum3_f16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Two FP16 coefficients (one dword) -> (u, w) with TransferCoefficient(v) = u + 0.05 w
// (reference: |v| <= 2 ? v : sign(v) min(2.5, 2 + 0.05 (|v| - 2))), both exact in FP16:
// u = sign(v) min(|v|, 2), w = sign(v) min(max(|v| - 2, 0), 10); a NaN v gives NaN u and w.
// u is a NaN-propagating minimum, w an integer min on the magnitude bits (unsigned order is
// value order for non-negative FP16) and one exact FP16 subtraction.  On gfx950 every code of both
// halves gives the same u and w as the integer-min form with a saturating NaN fix-up that this
// replaced (all 65,536 codes, NaN codes to NaN with their sign).
__device__ __forceinline__ void coef_clamp_split(unsigned v, unsigned& u, unsigned& w) {
  typedef unsigned short us2v __attribute__((ext_vector_type(2)));
  const unsigned mb = v & 0x7FFF7FFFu;
  const unsigned um = pk_minimum3_h16(mb, 0x40004000u, 0x40004000u);             // min(|v|, 2)
  const us2v mc = __builtin_elementwise_min(__builtin_bit_cast(us2v, mb), (us2v){0x4A00, 0x4A00});  // min(|v|, 12)
  const h2 wm = __builtin_bit_cast(h2, mc) - __builtin_bit_cast(h2, um);         // exact
  u = (um & 0x7FFF7FFFu) | (v & 0x80008000u);
  w = (__builtin_bit_cast(unsigned, wm) & 0x7FFF7FFFu) | (v & 0x80008000u);
}
// Two FP16 coefficients (one dword) -> the clamped coefficients rounded to FP16, for the head of
// the quantized policies (one FP16 B operand per coefficient instead of the exact u / w pair):
//   c = v                                              for |v| <= 2
//   c = sign(v) min(rne16((|v| - 2) h + 2), 2.5)       otherwise, h = fp16(0.05) = 0.0499877...,
// one fused rounding (|v| - 2 is exact in FP16 for |v| >= 1); c(+-inf) = +-2.5, a NaN v gives a
// quiet NaN.  The select is a minimum: rne16((m - 2) h + 2) >= m for m <= 2 and < m above, so
// c = min(m, t, 2.5) on the magnitude m, one NaN-propagating three-way minimum.  Differs from the
// FP32 clamp by at most half an FP16 ulp of c plus (0.05 - h)(|v| - 2) <= 1.2e-4, only where
// |v| > 2.  On gfx950 every code gives the result of the integer-min form with a saturating NaN
// fix-up that this replaced (all 65,536 codes in both halves).
__device__ __forceinline__ unsigned coef_clamp_h16(unsigned v) {
  const unsigned mb = v & 0x7FFF7FFFu;
  const h2 m = __builtin_bit_cast(h2, mb);
  const h2 two = {(_Float16)2.0f, (_Float16)2.0f};
  const h2 h05 = {(_Float16)0.05f, (_Float16)0.05f};
  const h2 t = __builtin_elementwise_fma(m - two, h05, two);
  const unsigned c = pk_minimum3_h16(mb, __builtin_bit_cast(unsigned, t), 0x41004100u);   // min(m, t, 2.5)
  return (c & 0x7FFF7FFFu) | (v & 0x80008000u);
}
__device__ __forceinline__ float h2f_lo(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
}
__device__ __forceinline__ float h2f_hi(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}
// fl32(float(half) * s) for the FP16 half of w as one v_fma_mix_f32 with a -0 addend: the FP16
// operand widens exactly and x + -0 = x for every x (+0 included), so the result is the rounded
// product bit for bit; the compiler turns fma(x, s, -0) into a separate conversion and multiply.
__device__ __forceinline__ float h2f_lo_mul(unsigned w, float s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(s));
  return r;
}
__device__ __forceinline__ float h2f_hi_mul(unsigned w, float s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(s));
  return r;
}
// fmaf(a, b, float(h)) for the FP16 half h of w (HI: the high half) as one v_fma_mix_f32: the addend
// widens exactly, so the single rounding is fmaf's.
template <bool HI>
__device__ __forceinline__ float fma_h16_addend(float a, float b, unsigned w) {
  float r;
  if constexpr (HI) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r) : "v"(a), "v"(b), "v"(w));
  else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,0,1]" : "=v"(r) : "v"(a), "v"(b), "v"(w));
  return r;
}
// fl32(float(x) + float(y)) for FP16 halves x of u and y of w (HX, HY: the high halves), as
// x * 1 + y in one v_fma_mix_f32 (both widen exactly; one rounding).
template <bool HX, bool HY>
__device__ __forceinline__ float add_h16_h16(unsigned u, unsigned w) {
  float r;
  if constexpr (HX && HY) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(u), "v"(w));
  else if constexpr (HX) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(u), "v"(w));
  else if constexpr (HY) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(u), "v"(w));
  else asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(u), "v"(w));
  return r;
}

// Tile scheduler: the i-th tile handled by this block.  Blocks are spread
// round-robin over the 8 XCDs; tiles are assigned so that consecutive tiles
// (which share halos) run on the same XCD and hit the same L2.
__device__ __forceinline__ int tile_of(int iter, int num_tiles) {
  const int grid = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  if (grid % 8 != 0) return b + iter * grid;
  const int per_xcd = grid / 8;
  const int xcd = b % 8, local = b / 8;
  const int band = (num_tiles + 7) / 8;              // tiles owned by one XCD
  const int t = xcd * band + local + iter * per_xcd;
  return (t < (xcd + 1) * band) ? t : num_tiles;      // past the band -> no tile
}
__device__ __forceinline__ int tile_iters(int num_tiles) {
  const int grid = (int)gridDim.x;
  if (grid % 8 != 0) return (num_tiles + grid - 1) / grid;
  const int band = (num_tiles + 7) / 8;
  return (band + grid / 8 - 1) / (grid / 8);
}

}  // namespace aeisu
