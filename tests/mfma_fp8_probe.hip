// Accumulation of the gfx950 E4M3 MFMA (v_mfma_f32_16x16x32_fp8_fp8) against the FP16 MFMA
// (v_mfma_f32_16x16x32_f16) on the same E4M3 values, which every FP16 number holds exactly.
// Built by aeisu_amd/build.py; tests/test_gpu_mfma_fp8.py runs it and checks the JSON it prints.
//
// Operand layout (16x16x32, one wave): A[i][k] in lane i + 16 (k / 8), byte / half k % 8;
// B[k][j] in lane j + 16 (k / 8); D[i][j] in lane j + 16 (i / 4), register i % 4.  Each case
// is one MFMA with C = 0; the host sums the 32 products exactly (double: an E4M3 product has at
// most 8 significant bits between 2^-18 and 2^18) and compares.
//
// Cases:
//  * window: one product 2^6 at k = 0 and one 2^-(a+b) at k = 1 (same group of 8 K slots),
//    a = row % 10, b = column % 10: does the small product survive at 6 + a + b bits below?
//  * cancel_same: +2^16 at k = 0, -2^16 at k = 8, 1.0 at k = 3 (in the group of the +2^16).
//  * cancel_cross: +2^16 at k = 0, -2^16 at k = 1, 2^-(a+b) at k = 10 (another group).
//  * random: 2048 MFMAs on weight-like (2^-4 .. 2^0) x activation-like (normal E4M3) operands.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)

__global__ void mfma_fp8(const long* a, const long* b, f4* d, int n) {
  const int c = blockIdx.x, l = threadIdx.x;
  if (c < n && l < 64)
    d[c * 64 + l] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a[c * 64 + l], b[c * 64 + l], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}
__global__ void mfma_f16(const h8* a, const h8* b, f4* d, int n) {
  const int c = blockIdx.x, l = threadIdx.x;
  if (c < n && l < 64)
    d[c * 64 + l] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c * 64 + l], b[c * 64 + l], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}

static double e4m3_value(uint8_t code) {
  const int e = (code >> 3) & 15, m = code & 7;
  const double v = e == 0 ? std::ldexp((double)m, -9) : std::ldexp(8.0 + m, e - 10);
  return (code & 0x80) ? -v : v;
}
// E4M3 code of an exactly representable value
static uint8_t e4m3_code(double v) {
  for (int c = 0; c < 256; ++c)
    if ((c & 0x7F) != 0x7F && e4m3_value((uint8_t)c) == v) return (uint8_t)c;
  std::printf("value %g is not an E4M3 value\n", v);
  std::exit(2);
}

struct Case {
  uint8_t A[16][32], B[32][16];   // E4M3 codes, A[i][k], B[k][j]
};

// D[case][i][j] of both MFMAs
static void run(const std::vector<Case>& cases, std::vector<float>& d8, std::vector<float>& d16) {
  const int n = (int)cases.size();
  std::vector<uint8_t> a8((size_t)n * 512), b8((size_t)n * 512);
  std::vector<_Float16> a16((size_t)n * 512), b16((size_t)n * 512);
  for (int c = 0; c < n; ++c)
    for (int l = 0; l < 64; ++l)
      for (int e = 0; e < 8; ++e) {
        const int k = 8 * (l >> 4) + e;
        const size_t o = ((size_t)c * 64 + l) * 8 + e;
        a8[o] = cases[c].A[l & 15][k];
        b8[o] = cases[c].B[k][l & 15];
        a16[o] = (_Float16)e4m3_value(a8[o]);
        b16[o] = (_Float16)e4m3_value(b8[o]);
      }
  void *da8, *db8, *da16, *db16, *dd;
  CHECK(hipMalloc(&da8, a8.size()));
  CHECK(hipMalloc(&db8, b8.size()));
  CHECK(hipMalloc(&da16, a16.size() * 2));
  CHECK(hipMalloc(&db16, b16.size() * 2));
  CHECK(hipMalloc(&dd, (size_t)n * 256 * 4));
  CHECK(hipMemcpy(da8, a8.data(), a8.size(), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(db8, b8.data(), b8.size(), hipMemcpyHostToDevice));
  CHECK(hipMemcpy(da16, a16.data(), a16.size() * 2, hipMemcpyHostToDevice));
  CHECK(hipMemcpy(db16, b16.data(), b16.size() * 2, hipMemcpyHostToDevice));
  std::vector<float> raw((size_t)n * 256);
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 0) mfma_fp8<<<n, 64>>>((const long*)da8, (const long*)db8, (f4*)dd, n);
    else mfma_f16<<<n, 64>>>((const h8*)da16, (const h8*)db16, (f4*)dd, n);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(raw.data(), dd, raw.size() * 4, hipMemcpyDeviceToHost));
    std::vector<float>& d = pass == 0 ? d8 : d16;
    d.assign((size_t)n * 256, 0.f);
    for (int c = 0; c < n; ++c)
      for (int l = 0; l < 64; ++l)
        for (int r = 0; r < 4; ++r) d[(size_t)c * 256 + (4 * (l >> 4) + r) * 16 + (l & 15)] = raw[((size_t)c * 64 + l) * 4 + r];
  }
  CHECK(hipFree(da8));
  CHECK(hipFree(db8));
  CHECK(hipFree(da16));
  CHECK(hipFree(db16));
  CHECK(hipFree(dd));
}

static double exact_sum(const Case& c, int i, int j, double* maxprod) {
  double s = 0, m = 0;
  for (int k = 0; k < 32; ++k) {
    const double p = e4m3_value(c.A[i][k]) * e4m3_value(c.B[k][j]);
    s += p;
    m = std::fmax(m, std::fabs(p));
  }
  if (maxprod) *maxprod = m;
  return s;
}

static Case zero_case() {
  Case c;
  for (int i = 0; i < 16; ++i)
    for (int k = 0; k < 32; ++k) c.A[i][k] = 0, c.B[k][i] = 0;
  return c;
}

int main() {
  int count = 0;
  CHECK(hipGetDeviceCount(&count));
  if (count < 1) {
    std::printf("no HIP device\n");
    return 2;
  }
  std::vector<Case> cases;
  // window
  {
    Case c = zero_case();
    for (int i = 0; i < 16; ++i) {
      c.A[i][0] = e4m3_code(8.0);
      c.A[i][1] = e4m3_code(std::ldexp(1.0, -(i % 10)));
    }
    for (int j = 0; j < 16; ++j) {
      c.B[0][j] = e4m3_code(8.0);
      c.B[1][j] = e4m3_code(std::ldexp(1.0, -(j % 10)));
    }
    cases.push_back(c);
  }
  // cancel_same
  {
    Case c = zero_case();
    for (int i = 0; i < 16; ++i) c.A[i][0] = e4m3_code(256.0), c.A[i][8] = e4m3_code(-256.0), c.A[i][3] = e4m3_code(1.0);
    for (int j = 0; j < 16; ++j) c.B[0][j] = c.B[8][j] = e4m3_code(256.0), c.B[3][j] = e4m3_code(1.0);
    cases.push_back(c);
  }
  // cancel_cross
  {
    Case c = zero_case();
    for (int i = 0; i < 16; ++i) {
      c.A[i][0] = e4m3_code(256.0), c.A[i][1] = e4m3_code(-256.0);
      c.A[i][10] = e4m3_code(std::ldexp(1.0, -(i % 10)));
    }
    for (int j = 0; j < 16; ++j) {
      c.B[0][j] = c.B[1][j] = e4m3_code(256.0);
      c.B[10][j] = e4m3_code(std::ldexp(1.0, -(j % 10)));
    }
    cases.push_back(c);
  }
  // random
  std::mt19937 rng(20261202);
  auto draw = [&](int lo, int hi) {
    for (;;) {
      const uint8_t b = (uint8_t)(rng() & 0xFF);
      const int e = (b >> 3) & 15;
      if ((b & 0x7F) != 0x7F && e >= lo && e <= hi) return b;
    }
  };
  const int nrand = 2048;
  for (int r = 0; r < nrand; ++r) {
    Case c;
    for (int i = 0; i < 16; ++i)
      for (int k = 0; k < 32; ++k) c.A[i][k] = draw(3, 7), c.B[k][i] = draw(1, 15);
    cases.push_back(c);
  }

  std::vector<float> d8, d16;
  run(cases, d8, d16);
  auto D = [&](const std::vector<float>& d, int c, int i, int j) { return (double)d[(size_t)c * 256 + i * 16 + j]; };

  std::printf("{");
  // window: bits below the largest product at which the small product is still in the result
  for (int pass = 0; pass < 2; ++pass) {
    std::printf("%s\"window_%s\": [", pass ? ", " : "", pass ? "f16" : "fp8");
    bool first = true;
    for (int i = 0; i < 10; ++i)
      for (int j = 0; j < 10; j += 9) {
        const int bits = 6 + i + j;
        if (bits > 23) continue;                           // beyond FP32 precision of 2^6 + small
        const double got = D(pass ? d16 : d8, 0, i, j) - 64.0;
        std::printf("%s[%d, %d]", first ? "" : ", ", bits, got == std::ldexp(1.0, -(i + j)) ? 1 : 0);
        first = false;
      }
    std::printf("]");
  }
  // cancellations
  for (int pass = 0; pass < 2; ++pass) {
    const std::vector<float>& d = pass ? d16 : d8;
    std::printf(", \"cancel_same_%s\": %.9g", pass ? "f16" : "fp8", D(d, 1, 0, 0));
    std::printf(", \"cancel_cross_%s\": [", pass ? "f16" : "fp8");
    for (int i = 0; i < 10; ++i)
      for (int j = 0; j < 10; j += 9) {
        if (j == 9 && i == 0) continue;                  // e = 9 once
        const double want = std::ldexp(1.0, -(i + j));
        std::printf("%s[%d, %d]", i + j ? ", " : "", i + j, D(d, 2, i, j) == want ? 1 : 0);
      }
    std::printf("]");
  }
  // random: results equal to fl32(exact sum), median and max |D - exact| / max|product| (log2)
  for (int pass = 0; pass < 2; ++pass) {
    const std::vector<float>& d = pass ? d16 : d8;
    std::vector<double> rel;
    long equal = 0;
    for (int c = 3; c < (int)cases.size(); ++c)
      for (int i = 0; i < 16; ++i)
        for (int j = 0; j < 16; ++j) {
          double m = 0;
          const double ex = exact_sum(cases[c], i, j, &m);
          const double got = D(d, c, i, j);
          if (got == (double)(float)ex) ++equal;
          rel.push_back(std::fabs(got - ex) / m);
        }
    std::vector<double> s = rel;
    std::nth_element(s.begin(), s.begin() + s.size() / 2, s.end());
    const double med = s[s.size() / 2];
    double mx = 0;
    for (double v : rel) mx = std::fmax(mx, v);
    std::printf(", \"random_%s\": {\"equal_fl32_exact\": %.6f, \"median_log2_rel\": %.3f, \"max_log2_rel\": %.3f}",
                pass ? "f16" : "fp8", (double)equal / rel.size(), med > 0 ? std::log2(med) : -99.0,
                mx > 0 ? std::log2(mx) : -99.0);
  }
  std::printf("}\n");
  return 0;
}
