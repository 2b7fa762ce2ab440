// C++ host program against the public C ABI (include/aeisu_amd.h), as a native caller of the
// reference's CudaRuntime would use it (SrcPyrCudaRuntime.h:29-96).  Built by aeisu_amd/build.py
// into tests/abi_smoke; tests/test_gpu_abi.py runs it on the GPU.
//
//   abi_smoke <SPYR8F8 Mixed artifact> <expected sha256 prefix>
//
// create -> configure -> upscale -> read back (FP32 frames); a sibling sharing the weights
// with a second geometry; a precision change at configure (FP16 weights uploaded on first use); the
// startup report; a non-finite input; and the documented error codes.  Prints "abi_smoke: OK".
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "aeisu_amd.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL: %s (last error: %s)\n", what, aeisu_last_error());
    ++g_failures;
  }
}

void require(int rc, const char* what) {
  if (rc != AEISU_OK) {
    std::printf("FATAL: %s returned %d: %s\n", what, rc, aeisu_last_error());
    std::exit(2);
  }
}

void hip_require(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::printf("FATAL: %s: %s\n", what, hipGetErrorString(e));
    std::exit(2);
  }
}

// deterministic frame in [0, 1]: gradients plus a checker pattern, planar [B][3][H][W]
std::vector<float> make_frame(int b, int h, int w) {
  std::vector<float> v(size_t(b) * 3 * h * w);
  for (int n = 0; n < b; ++n)
    for (int c = 0; c < 3; ++c)
      for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) {
          const float g = 0.2f + 0.5f * float(x) / float(w) + 0.2f * float(y) / float(h) + 0.05f * float(c + n);
          const float chk = ((x / 6 + y / 5) % 2) ? 0.15f : -0.1f;
          v[((size_t(n) * 3 + c) * h + y) * w + x] = std::fmin(1.f, std::fmax(0.f, g + chk));
        }
  return v;
}

struct Device {
  void* p = nullptr;
  explicit Device(size_t n) { hip_require(hipMalloc(&p, n), "hipMalloc"); }
  ~Device() { (void)hipFree(p); }
};

// one batch through a configured runtime with FP32 frames in and out
std::vector<float> run_f32(aeisu_runtime* rt, const std::vector<float>& in, int b, int h, int w, int* rc) {
  Device din(in.size() * 4), dout(size_t(b) * 3 * 4 * h * w * 4);
  hip_require(hipMemcpy(din.p, in.data(), in.size() * 4, hipMemcpyHostToDevice), "hipMemcpy in");
  *rc = aeisu_upscale(rt, din.p, dout.p, nullptr);
  std::vector<float> out(size_t(b) * 3 * 4 * h * w);
  hip_require(hipMemcpy(out.data(), dout.p, out.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy out");
  return out;
}

bool in_unit_range(const std::vector<float>& v) {
  for (float x : v)
    if (!(x >= 0.f && x <= 1.f)) return false;
  return true;
}

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
  float m = 0.f;
  for (size_t i = 0; i < a.size(); ++i) m = std::fmax(m, std::fabs(a[i] - b[i]));
  return m;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) {
    std::printf("usage: %s <SPYR8F8 Mixed artifact> <sha256 prefix>\n", argv[0]);
    return 2;
  }
  std::printf("abi_smoke: %s\n", aeisu_version());

  // --- create and configure (Mixed), FP32 frames
  aeisu_runtime* rt = nullptr;
  require(aeisu_create_from_file(argv[1], AEISU_PRECISION_MIXED, &rt), "aeisu_create_from_file");
  char sha[65];
  require(aeisu_artifact_checksum(rt, sha), "aeisu_artifact_checksum");
  expect(std::strncmp(sha, argv[2], std::strlen(argv[2])) == 0, "artifact checksum");
  expect(aeisu_startup_report(rt, nullptr, 0) == 0, "no report before configure");
  const int H = 72, W = 104;
  require(aeisu_configure(rt, 1, H, W, AEISU_LAYOUT_NCHW_F32, AEISU_LAYOUT_NCHW_F32, 0, 0), "aeisu_configure");
  const std::vector<float> frame = make_frame(1, H, W);
  int rc = 0;
  const std::vector<float> mixed = run_f32(rt, frame, 1, H, W, &rc);
  expect(rc == AEISU_OK, "aeisu_upscale (Mixed)");
  expect(in_unit_range(mixed), "Mixed output finite and in [0, 1]");

  std::vector<char> report(aeisu_startup_report(rt, nullptr, 0));
  expect(report.size() > 1, "startup report size");
  aeisu_startup_report(rt, report.data(), report.size());
  const std::string rep(report.data());
  std::printf("abi_smoke: report: %s\n", rep.c_str());
  expect(rep.find(std::string("sha256=") + sha) != std::string::npos, "report names the artifact hash");
  expect(rep.find("precision=FP8/FP16-Mixed") != std::string::npos, "report names the policy");
  expect(rep.find("source=104x72") != std::string::npos, "report names the geometry");

  // --- a sibling: shared weights, own geometry (a batch of 2 frames)
  aeisu_runtime* sib = nullptr;
  require(aeisu_create_sibling(rt, &sib), "aeisu_create_sibling");
  expect(aeisu_shares_weights(rt, sib) == 1, "sibling shares weights");
  int dummy[6];
  expect(aeisu_geometry(sib, dummy) == AEISU_ERR_STATE, "unconfigured sibling reports a state error");
  expect(aeisu_upscale_async(sib, frame.data(), nullptr, nullptr) == AEISU_ERR_STATE, "upscale before configure");
  require(aeisu_configure(sib, 2, H, W, AEISU_LAYOUT_NCHW_F32, AEISU_LAYOUT_NCHW_F32, 0, 0), "configure sibling");
  std::vector<float> two = make_frame(1, H, W);
  const std::vector<float> second = make_frame(2, H, W);
  two.insert(two.end(), second.begin() + size_t(3) * H * W, second.end());   // frames 0 and 1 of make_frame(2)
  const std::vector<float> pair = run_f32(sib, two, 2, H, W, &rc);
  expect(rc == AEISU_OK, "sibling upscale");
  const std::vector<float> first(pair.begin(), pair.begin() + mixed.size());
  expect(max_abs_diff(first, mixed) == 0.f, "sibling's frame 0 equals the first runtime's result");
  aeisu_runtime* bare = nullptr;
  require(aeisu_create_sibling(rt, &bare), "bare sibling");
  const size_t shared = aeisu_persistent_bytes(bare);
  expect(shared > 0 && aeisu_persistent_bytes(rt) > shared && aeisu_persistent_bytes(sib) > shared,
         "persistent bytes = shared weights + own scratch");
  aeisu_destroy(bare);

  // --- precision chosen at configure: the FP16 weights of the same artifact, uploaded on first use
  require(aeisu_configure(rt, 1, H, W, AEISU_LAYOUT_NCHW_F32, AEISU_LAYOUT_NCHW_F32, AEISU_PRECISION_FP16, 0),
          "configure FP16");
  const std::vector<float> fp16 = run_f32(rt, frame, 1, H, W, &rc);
  expect(rc == AEISU_OK, "aeisu_upscale (FP16)");
  const float d = max_abs_diff(fp16, mixed);
  std::printf("abi_smoke: max |FP16 - Mixed| = %.5f\n", d);
  expect(d > 0.f && d < 0.05f, "FP16 and Mixed policies agree to the Mixed quantization error");
  aeisu_startup_report(rt, report.data(), report.size());
  expect(std::string(report.data()).find("precision=FP16") != std::string::npos, "report follows the policy");
  expect(aeisu_shares_weights(rt, sib) == 1, "still sharing after a precision change");

  // --- errors
  expect(aeisu_configure(rt, 1, 0, W, 0, 0, 0, 0) == AEISU_ERR_INVALID_ARGUMENT, "zero height rejected");
  expect(aeisu_configure(rt, 1, 9000, W, 0, 0, 0, 0) == AEISU_ERR_INVALID_ARGUMENT, "height > 8192 rejected");
  expect(aeisu_configure(rt, 1, H, W, 0, 0, 99, 0) == AEISU_ERR_INVALID_ARGUMENT, "unknown precision rejected");
  expect(aeisu_configure(rt, 1, H, W, 0, 0, AEISU_PRECISION_INT8, 0) == AEISU_ERR_ARTIFACT,
         "a policy without tensors in the artifact is rejected");
  expect(std::strstr(aeisu_last_error(), "weight_i8") != nullptr, "error names the missing tensor");
  aeisu_runtime* none = nullptr;
  expect(aeisu_create_from_file("/nonexistent.bin", AEISU_PRECISION_MIXED, &none) == AEISU_ERR_ARTIFACT && !none,
         "missing file rejected");

  // --- non-finite input
  require(aeisu_configure(rt, 1, H, W, AEISU_LAYOUT_NCHW_F32, AEISU_LAYOUT_NCHW_F32, AEISU_PRECISION_MIXED, 0),
          "reconfigure Mixed");
  std::vector<float> bad = frame;
  bad[size_t(1) * H * W + 5 * W + 7] = NAN;
  (void)run_f32(rt, bad, 1, H, W, &rc);
  expect(rc == AEISU_ERR_NONFINITE, "NaN input reports AEISU_ERR_NONFINITE");
  const std::vector<float> again = run_f32(rt, frame, 1, H, W, &rc);
  expect(rc == AEISU_OK && max_abs_diff(again, mixed) == 0.f, "flag cleared; result reproducible");

  aeisu_destroy(sib);
  aeisu_destroy(rt);
  if (g_failures) {
    std::printf("abi_smoke: %d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("abi_smoke: OK\n");
  return 0;
}
