// AEISU runtime engine for MI355X: artifact validation, weight-fragment packing,
// scratch allocation, the per-frame launch sequence, HIP graphs and stage timing.
//
// Reference counterparts: ModelArtifact::Load (optimized/native/src/neural/srcpyr/
// SrcPyrModel.cpp:243-470), SharedExecutionEngine::UploadModel / AttachConfiguration /
// EnqueueGraphBody (SrcPyrCudaRuntime.cu:2924-3170, 3310-3806, 4131-4873).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "aeisu_amd.h"
#include "kernels.hpp"
#include "sha256.hpp"

namespace aeisu {

// ------------------------------------------------------------------------------------------------
// errors
// ------------------------------------------------------------------------------------------------
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] static void fail(int code, const std::string& msg) { throw Error(code, msg); }
static void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(AEISU_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Diagnostic, off by default (the reference's AESS_NEURAL_EAGER_VALIDATE, SrcPyrCudaRuntime.cu:5349-5354):
// with AEISU_EAGER_VALIDATE=1 in the environment every kernel launch outside graph capture is followed
// by a synchronisation of its stream, so that an asynchronous failure is reported with the launch
// that caused it instead of at a later call.
static bool eager_validate() {
  static const bool on = [] {
    const char* v = std::getenv("AEISU_EAGER_VALIDATE");
    return v && v[0] == '1';
  }();
  return on;
}
static void check_launch(hipError_t e, const char* what, hipStream_t s) {
  check_hip(e, what);
  if (!eager_validate()) return;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  check_hip(hipStreamIsCapturing(s, &cs), what);
  if (cs != hipStreamCaptureStatusNone) return;
  check_hip(hipStreamSynchronize(s), what);
}

// ------------------------------------------------------------------------------------------------
// SPYR8F8 artifact (layout: SrcPyrModel.cpp:37-81)
// ------------------------------------------------------------------------------------------------
constexpr size_t kHeaderSize = 512, kDescSize = 80, kChecksumOffset = 184, kAlign = 64;
constexpr const char* kArchitecture = "aif16x5_learnedrgb4dir8_s32_parallel32x4_learnedbase_oc25_v1";
enum DType : uint32_t { kE4M3 = 1, kF16 = 2, kF32 = 3, kI8 = 6 };

struct TensorView {
  uint32_t dtype = 0, layout = 0, rank = 0, shape[4] = {0, 0, 0, 0};
  const uint8_t* data = nullptr;
  uint64_t bytes = 0;
  uint64_t count() const {
    uint64_t n = 1;
    for (uint32_t d = 0; d < rank; ++d) n *= shape[d];
    return n;
  }
  const float* f32() const { return reinterpret_cast<const float*>(data); }
  const uint16_t* f16() const { return reinterpret_cast<const uint16_t*>(data); }
};

template <typename T>
static T rd(const uint8_t* p, size_t off) {
  T v;
  std::memcpy(&v, p + off, sizeof(T));
  return v;
}
static std::string fixed_string(const uint8_t* p, size_t n, const char* what) {
  size_t len = 0;
  while (len < n && p[len]) ++len;
  if (len == n) fail(AEISU_ERR_ARTIFACT, std::string("unterminated SPYR8 ") + what);
  for (size_t i = len; i < n; ++i)
    if (p[i]) fail(AEISU_ERR_ARTIFACT, std::string("nonzero padding after SPYR8 ") + what);
  return std::string(reinterpret_cast<const char*>(p), len);
}
static size_t elem_size(uint32_t dt) {
  switch (dt) {
    case kE4M3: return 1;
    case kF16: return 2;
    case kF32: return 4;
    case kI8: return 1;
    default: return 0;
  }
}

struct Artifact {
  std::vector<uint8_t> storage;
  std::string checksum_hex;
  std::unordered_map<std::string, TensorView> tensors;

  bool has(const std::string& name) const { return tensors.count(name) != 0; }
  const TensorView& need(const std::string& name, uint32_t dtype, std::initializer_list<uint32_t> shape) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) fail(AEISU_ERR_ARTIFACT, "missing SPYR8 tensor: " + name);
    const TensorView& t = it->second;
    bool ok = t.dtype == dtype && t.rank == shape.size();
    uint32_t d = 0;
    for (uint32_t s : shape) ok = ok && t.shape[d++] == s;
    if (!ok) fail(AEISU_ERR_ARTIFACT, "SPYR8 tensor has wrong type or shape: " + name);
    return t;
  }
};

static Artifact parse_artifact(const uint8_t* data, size_t size) {
  Artifact a;
  if (size < kHeaderSize) fail(AEISU_ERR_ARTIFACT, "SPYR8 artifact is smaller than its header");
  a.storage.assign(data, data + size);
  const uint8_t* p = a.storage.data();
  static const char magic[8] = {'S', 'P', 'Y', 'R', '8', 'F', '8', '\0'};
  if (std::memcmp(p, magic, 8) != 0 || rd<uint32_t>(p, 8) != 1 || rd<uint32_t>(p, 12) != kHeaderSize ||
      rd<uint32_t>(p, 16) != 0x01020304u || rd<uint32_t>(p, 20) != 0)
    fail(AEISU_ERR_ARTIFACT, "unsupported SPYR8 magic/version/endian/flags");
  const std::string arch = fixed_string(p + 24, 64, "architecture");
  if (arch != kArchitecture) fail(AEISU_ERR_ARTIFACT, "unsupported SPYR8 architecture: " + arch);
  const uint32_t expect[14] = {8, 32, 32, 64, 4, 64, 2, 1, 1, 2, 1, 0, 64, 80};
  for (int i = 0; i < 14; ++i) {
    if (i == 11) continue;  // tensor count
    if (rd<uint32_t>(p, 88 + 4 * i) != expect[i]) fail(AEISU_ERR_ARTIFACT, "unsupported or inconsistent SPYR8 header");
  }
  const uint32_t count = rd<uint32_t>(p, 132);
  const float shift = rd<float>(p, 144), gain = rd<float>(p, 148);
  const uint64_t file_size = rd<uint64_t>(p, 152), toc_off = rd<uint64_t>(p, 160), toc_bytes = rd<uint64_t>(p, 168),
                 payload = rd<uint64_t>(p, 176);
  const uint64_t toc_end = toc_off + toc_bytes;
  if (file_size != size || toc_off != kHeaderSize || toc_bytes != uint64_t(count) * kDescSize ||
      payload < ((toc_end + kAlign - 1) / kAlign) * kAlign || payload > file_size)
    fail(AEISU_ERR_ARTIFACT, "unsupported or inconsistent SPYR8 header");
  for (size_t i = 216; i < kHeaderSize; ++i)
    if (p[i]) fail(AEISU_ERR_ARTIFACT, "nonzero SPYR8 v1 header extension bytes");
  if (!std::isfinite(shift) || shift < 0 || !std::isfinite(gain) || gain < 0)
    fail(AEISU_ERR_ARTIFACT, "invalid SPYR8 edge-phase parameters");
  {
    Sha256 h;
    h.update(p, kChecksumOffset);
    const uint8_t zeros[32] = {};
    h.update(zeros, 32);
    h.update(p + kChecksumOffset + 32, size - kChecksumOffset - 32);
    const auto digest = h.finish();
    char hex[65];
    for (int i = 0; i < 32; ++i) std::snprintf(hex + 2 * i, 3, "%02x", digest[i]);
    if (std::memcmp(digest.data(), p + kChecksumOffset, 32) != 0) {
      char stored[65];
      for (int i = 0; i < 32; ++i) std::snprintf(stored + 2 * i, 3, "%02x", p[kChecksumOffset + i]);
      fail(AEISU_ERR_ARTIFACT, std::string("SPYR8 artifact checksum mismatch: expected ") + stored + ", observed " + hex);
    }
    a.checksum_hex = hex;
  }
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (uint32_t i = 0; i < count; ++i) {
    const uint8_t* d = p + toc_off + uint64_t(i) * kDescSize;
    const std::string name = fixed_string(d, 32, "tensor name");
    TensorView t;
    t.dtype = rd<uint32_t>(d, 32);
    t.layout = rd<uint32_t>(d, 36);
    t.rank = rd<uint32_t>(d, 40);
    if (name.empty() || a.tensors.count(name) || t.rank == 0 || t.rank > 4)
      fail(AEISU_ERR_ARTIFACT, "invalid or duplicate SPYR8 tensor descriptor");
    uint64_t elements = 1;
    for (int k = 0; k < 4; ++k) {
      t.shape[k] = rd<uint32_t>(d, 44 + 4 * k);
      if ((uint32_t)k < t.rank) {
        if (t.shape[k] == 0 || elements > (uint64_t(1) << 40) / t.shape[k])
          fail(AEISU_ERR_ARTIFACT, "invalid SPYR8 tensor dimensions: " + name);
        elements *= t.shape[k];
      } else if (t.shape[k] != 0) {
        fail(AEISU_ERR_ARTIFACT, "nonzero unused SPYR8 dimension: " + name);
      }
    }
    const size_t es = elem_size(t.dtype);
    if (es == 0) fail(AEISU_ERR_ARTIFACT, "unsupported SPYR8 tensor data type: " + name);
    const uint64_t off = rd<uint64_t>(d, 60), bytes = rd<uint64_t>(d, 68);
    if (off % kAlign || off < payload || bytes == 0 || off > file_size || bytes > file_size - off ||
        bytes != elements * es || rd<uint32_t>(d, 76) != 0)
      fail(AEISU_ERR_ARTIFACT, "SPYR8 tensor bounds or byte count mismatch: " + name);
    t.data = p + off;
    t.bytes = bytes;
    a.tensors.emplace(name, t);
    ranges.emplace_back(off, off + bytes);
  }
  std::sort(ranges.begin(), ranges.end());
  for (size_t i = 1; i < ranges.size(); ++i)
    if (ranges[i - 1].second > ranges[i].first) fail(AEISU_ERR_ARTIFACT, "overlapping SPYR8 tensor payloads");
  return a;
}

// ------------------------------------------------------------------------------------------------
// fragment packing (operand register images; layout described in common.hpp)
// ------------------------------------------------------------------------------------------------
static uint16_t f32_to_f16_bits(float v) {
  _Float16 h = (_Float16)v;
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}
static float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  std::memcpy(&h, &b, 2);
  return (float)h;
}

// Value of an OCP E4M3 code (bias 7, 3 mantissa bits, subnormals below 2^-6; 0x7F/0xFF are NaN).
static float e4m3_value(uint8_t code) {
  const int e = (code >> 3) & 15, m = code & 7;
  if (e == 15 && m == 7) return NAN;
  const float v = e == 0 ? std::ldexp(float(m), -9) : std::ldexp(1.0f + m / 8.0f, e - 7);
  return (code & 0x80) ? -v : v;
}

// out[(f*64 + lane)*E + i] = fn(f, m = lane & 15, slot = (lane >> 4)*E + i)
template <typename T, typename Fn>
static std::vector<T> pack_frags(int nfrag, int E, Fn fn) {
  std::vector<T> out(size_t(nfrag) * 64 * E);
  for (int f = 0; f < nfrag; ++f)
    for (int lane = 0; lane < 64; ++lane)
      for (int i = 0; i < E; ++i) out[(size_t(f) * 64 + lane) * E + i] = fn(f, lane & 15, (lane >> 4) * E + i);
  return out;
}

struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  std::vector<uint8_t> staged;  // host image waiting for commit()
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { release(); }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  void alloc(size_t n) {
    release();
    if (n == 0) return;
    check_hip(hipMalloc(&ptr, n), "hipMalloc");
    bytes = n;
  }
  // Stage a host image; the device copy is made by commit() once every
  // tensor of the artifact has been validated (no HIP call before that).
  template <typename T>
  void upload(const std::vector<T>& v) {
    staged.resize(v.size() * sizeof(T));
    std::memcpy(staged.data(), v.data(), staged.size());
  }
  void commit() {
    if (staged.empty()) return;
    alloc(staged.size());
    check_hip(hipMemcpy(ptr, staged.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy(weights)");
    staged.clear();
    staged.shrink_to_fit();
  }
  template <typename T>
  T* as() const { return reinterpret_cast<T*>(ptr); }
};

struct LayerDev {
  DeviceBuffer frag, bias, scale;
};

// ------------------------------------------------------------------------------------------------
// engine
// ------------------------------------------------------------------------------------------------
constexpr int kStageEvents = AEISU_STAGE_COUNT;  // 7 boundaries per frame (start + 6 stage ends)
constexpr int kMaxTimedFrames = 4096;
constexpr int kModes = 5;
constexpr int kModeFp32 = 4;

// Kernel mode of a precision: 0 FP16, 1 E4M3 on the FP8 MFMA, 2 INT8, 3 E4M3 values on the FP16 MFMA,
// 4 FP32 (per-layer FP32 kernels, k_fp32.hip).
static int mode_of(int precision) {
  switch (precision) {
    case AEISU_PRECISION_FP16: return 0;
    case AEISU_PRECISION_MIXED_FP8MMA: return 1;
    case AEISU_PRECISION_INT8: return 2;
    case AEISU_PRECISION_MIXED: return 3;
    case AEISU_PRECISION_FP32: return kModeFp32;
    default: fail(AEISU_ERR_INVALID_ARGUMENT, "unknown precision");
  }
}
static const char* precision_name(int mode) {
  static const char* names[kModes] = {"FP16", "FP8-E4M3 on the FP8 MFMA", "INT8/FP16", "FP8/FP16-Mixed", "FP32"};
  return names[mode];
}

// Weights of one arithmetic policy, packed into MFMA fragments and resident on the device.
struct ModeWeights {
  int mode = 0;
  bool project_precise = false;
  float analysis[24];
  float act[10] = {};
  LayerDev project, compress, grouped[4], expand, refine_tail, head;
  DeviceBuffer compress_rgb;       // INT8 compress weights in the frame-input fused body's K order
  DeviceBuffer tail_bias;
  DeviceBuffer body_consts;        // epilogue constants of the fused body (kBodyConsts floats)
  DeviceBuffer fp32;               // FP32 policy: the whole weight image (kernels.hpp kF32*)

  // every device buffer, for commit() and byte accounting
  template <typename Fn>
  void each_buffer(Fn fn) {
    for (LayerDev* l : {&project, &compress, &grouped[0], &grouped[1], &grouped[2], &grouped[3], &expand,
                        &refine_tail, &head}) {
      fn(l->frag);
      fn(l->bias);
      fn(l->scale);
    }
    fn(compress_rgb);
    fn(tail_bias);
    fn(body_consts);
    fn(fp32);
  }
  size_t bytes() const {
    size_t n = 0;
    const_cast<ModeWeights*>(this)->each_buffer([&](DeviceBuffer& b) { n += b.bytes; });
    return n;
  }
};

// The loaded artifact and its uploaded weights: shared by a runtime and its siblings (the reference's
// shared execution engine, SrcPyrCudaRuntime.cu:5392-5396).  A policy's weights are packed and uploaded
// the first time a runtime is configured for it.
struct Model {
  Artifact art;
  int device = 0, cu_count = 0;
  std::string gpu_name, gcn_arch;
  int hip_runtime_version = 0;
  std::mutex mu;
  std::unique_ptr<ModeWeights> modes[kModes];

  const ModeWeights& weights(int mode);
  size_t bytes() {
    std::lock_guard<std::mutex> lock(mu);
    size_t n = 0;
    for (const auto& m : modes)
      if (m) n += m->bytes();
    return n;
  }
};

// Frame geometry and launch shapes of one configuration: a pure function of the policy, the device's
// CU count and the configure arguments (computed without allocating).
struct Geometry {
  int batch = 0, H = 0, W = 0, Hp = 0, Wp = 0, py = 0, px = 0, Hq = 0, Wq = 0, Hl = 0, Wl = 0;
  int in_fp32 = 0, out_fp32 = 0;
  int act_bytes = 2;               // bytes per skip / work / coefficient element (FP32 policy: 4)
  int low_bytes = 2;               // bytes per low-resolution activation (FP16 2, byte policies 1, FP32 4)
  int qclamp = 0;                  // head of the quantized policies: clamped coefficients in FP16
  unsigned flags = 0;
  bool fused = false;              // fused body kernel, and refine + tail + head in one kernel
                                   // (body activations and coefficients stay on chip)
  bool fused_rgb = false;          // the fused body takes the frames (project recomputed on chip,
                                   // no skip tensor); the quantized policies
  int nlow = 0;                    // body activations in device memory (per-layer path)
  int body_split = 0;              // frame-input body: leading frames on 24x24 tiles, the rest on 16x16
  int body_cols24 = 0;             // frame-input body: > 0: low columns [0, body_cols24) on 24x24 tiles, the rest on 16x16
  int body_rows16 = 0;             // FP16 policy body: low rows on 16x16 tiles, the rest on 8x8
  int body_xc_tile = 0;            // frame-input body with the compress exchange: its tile code (0: off)
  int body_xc_frames = 0;          // ... in launches of this many whole frames
  int cus = 0;                     // compute units of the device
  struct Grids { int project, compress, grouped, expand, refine, head, fused; } grid{};

  size_t packed() const { return size_t(batch) * Hq * Wq; }
  size_t lowpx() const { return size_t(batch) * Hl * Wl; }
  // device scratch of the configuration (bytes): skip, work, meta, low activations
  size_t skip_bytes() const { return fused_rgb ? 0 : packed() * 32 * act_bytes; }
  size_t work_bytes() const { return packed() * 32 * act_bytes; }
  size_t meta_bytes() const { return fused ? 0 : packed() * 64 * act_bytes; }
  size_t low_layer_bytes() const { return lowpx() * 64 * low_bytes; }
  // compress exchange: the cores' compress codes (64 bytes per low pixel) and one counter per tile
  size_t xbuf_bytes() const { return body_xc_tile ? lowpx() * 64 : 0; }
  size_t xflag_bytes() const {
    return body_xc_tile ? size_t(body_fused_num_tiles(2, batch, Hl, Wl, body_xc_tile)) * sizeof(unsigned) : 0;
  }
};

// Device pointers the kernels of one frame use beyond the inputs, outputs and weights.
struct Scratch {
  void* skip = nullptr;
  void* work = nullptr;
  void* meta = nullptr;
  void* low[5] = {};
  unsigned* nonfinite = nullptr;
  void* xbuf = nullptr;
  unsigned* xflags = nullptr;
};

struct Runtime {
  std::shared_ptr<Model> model;
  int precision = 0, mode = 0;
  const ModeWeights* w = nullptr;  // the policy this runtime runs
  bool configured = false;
  Geometry g;
  DeviceBuffer skip, work, meta, nonfinite, xbuf, xflags;
  DeviceBuffer low[5];
  std::string report;              // startup report of the configuration
  // captured frame graphs, one per (input, output) buffer pair
  struct Graph {
    const void* in;
    void* out;
    hipGraph_t graph;
    hipGraphExec_t exec;
  };
  static constexpr size_t kMaxGraphs = 16;
  std::vector<Graph> graphs;
  hipStream_t capture_stream = nullptr;
  // timing
  std::vector<hipEvent_t> events;  // kStageEvents per recorded frame
  int timed_frames = 0;

  ~Runtime() {
    if (model) (void)hipSetDevice(model->device);
    // frames of this runtime may still be running on the caller's stream: their scratch, events and
    // graphs are released only once the device has finished
    if (configured || !graphs.empty()) (void)hipDeviceSynchronize();
    drop_graph();
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
  }
  // An executable graph may still be running on the caller's stream (aeisu_upscale_graph returns
  // once it is launched), and HIP does not promise to keep an executable graph's resources (its
  // kernel-argument memory) alive past hipGraphExecDestroy, so the device is drained first.  This
  // runs on reconfiguration, on destruction and when the graph cache is full: never per frame.
  void drop_graph() {
    if (!graphs.empty()) (void)hipDeviceSynchronize();
    for (Graph& gr : graphs) {
      (void)hipGraphExecDestroy(gr.exec);
      (void)hipGraphDestroy(gr.graph);
    }
    graphs.clear();
  }
  Scratch scratch() {
    Scratch sc;
    sc.skip = skip.ptr;
    sc.work = work.ptr;
    sc.meta = meta.ptr;
    for (int i = 0; i < 5; ++i) sc.low[i] = low[i].ptr;
    sc.nonfinite = nonfinite.as<unsigned>();
    sc.xbuf = xbuf.ptr;
    sc.xflags = xflags.as<unsigned>();
    return sc;
  }
  size_t scratch_bytes() const {
    size_t n = skip.bytes + work.bytes + meta.bytes + nonfinite.bytes + xbuf.bytes + xflags.bytes;
    for (const auto& l : low) n += l.bytes;
    return n;
  }
};

static void require_prelu(const Artifact& a, const std::string& layer, uint32_t cout, float value) {
  const TensorView& t = a.need(layer + ".prelu", kF32, {cout});
  for (uint32_t i = 0; i < cout; ++i)
    if (t.f32()[i] != value)
      fail(AEISU_ERR_ARTIFACT, "unsupported per-channel slope in " + layer + ".prelu (kernels implement " +
                                   std::to_string(value) + ")");
}

static std::vector<float> as_f32_vector(const TensorView& t) { return std::vector<float>(t.f32(), t.f32() + t.count()); }

// FP32 policy: every layer's FP32 weights (<layer>.weight_fp32, written by the folded-checkpoint
// converter) re-laid [tap][ci][co] into one image (kernels.hpp kF32*).
static void pack_fp32(ModeWeights& rt, const Artifact& a, const float* base, const float* basis) {
  std::vector<float> img(kF32Floats, 0.f);
  auto w32 = [&](const std::string& l, uint32_t cout, uint32_t cin, uint32_t ks) {
    if (!a.has(l + ".weight_fp32"))
      fail(AEISU_ERR_ARTIFACT, "the FP32 policy needs " + l + ".weight_fp32 (convert a folded FP32 checkpoint)");
    return a.need(l + ".weight_fp32", kF32, {cout, cin, ks, ks}).f32();
  };
  auto layer = [&](const std::string& l, uint32_t cout, uint32_t cin, uint32_t ks, int off, float slope) {
    const float* w = w32(l, cout, cin, ks);
    require_prelu(a, l, cout, slope);
    const float* b = a.need(l + ".bias", kF32, {cout}).f32();
    for (uint32_t o = 0; o < cout; ++o) {
      for (uint32_t i = 0; i < cin; ++i)
        for (uint32_t t = 0; t < ks * ks; ++t) {
          const float v = w[(size_t(o) * cin + i) * ks * ks + t];
          if (!std::isfinite(v)) fail(AEISU_ERR_ARTIFACT, "nonfinite weight in " + l);
          img[off + (size_t(t) * cin + i) * cout + o] = v;         // [tap][ci][co]
        }
      img[off + size_t(ks * ks) * cin * cout + o] = b[o];
    }
  };
  layer("project", 32, 32, 1, kF32Project, 0.1f);
  layer("compress", 64, 128, 1, kF32Compress, 0.1f);
  for (int l = 0; l < 4; ++l) layer("bottleneck" + std::to_string(l), 64, 32, 3, kF32Grouped + l * kF32GroupedStride, 0.1f);
  layer("expand", 128, 64, 1, kF32Expand, 0.1f);
  layer("refine", 64, 32, 3, kF32Refine, 0.1f);
  layer("tail", 64, 64, 1, kF32Tail, 1.0f);
  for (int i = 0; i < 100; ++i) img[kF32Base + i] = base[i];
  for (int i = 0; i < 1600; ++i) img[kF32Basis + i] = basis[i];
  for (int i = 0; i < 24; ++i) img[kF32Analysis + i] = rt.analysis[i];
  rt.fp32.upload(img);
}

static void pack_weights(ModeWeights& rt, const Artifact& a) {
  // --- shared tensors and contracts (SrcPyrModel.cpp:355-422)
  const TensorView& stencil = a.need("analysis_stencil", kF32, {24});
  for (int i = 0; i < 24; ++i) {
    rt.analysis[i] = stencil.f32()[i];
    if (!std::isfinite(rt.analysis[i])) fail(AEISU_ERR_ARTIFACT, "Nonfinite learned analysis 4-dir parameters");
  }
  const TensorView& base = a.need("adaptive_base", kF32, {25, 4});
  const TensorView& basis = a.need("adaptive_basis", kF32, {25, 16, 4});
  for (int i = 0; i < 100; ++i)
    if (!std::isfinite(base.f32()[i])) fail(AEISU_ERR_ARTIFACT, "Nonfinite adaptive learned base");
  for (int kp = 0; kp < 64; ++kp) {
    float dc = 0, l1 = 0;
    for (int tap = 0; tap < 25; ++tap) {
      const float v = basis.f32()[tap * 64 + kp];
      if (!std::isfinite(v)) fail(AEISU_ERR_ARTIFACT, "Nonfinite adaptive basis");
      dc += v;
      l1 += std::fabs(v);
    }
    if (std::fabs(dc) > 1e-5f || l1 > 0.5001f) fail(AEISU_ERR_ARTIFACT, "Adaptive basis violates zero-DC/L1 contract");
  }
  const TensorView& guards = a.need("precision_guards", kF32, {2});
  for (int i = 0; i < 2; ++i)
    if (guards.f32()[i] != 0.f && guards.f32()[i] != 1.f) fail(AEISU_ERR_ARTIFACT, "Invalid adaptive precision policy");
  if (rt.mode != 0 && rt.mode != kModeFp32) {
    const TensorView& s = a.need("activation_scales", kF32, {10});
    for (int i = 0; i < 10; ++i) {
      rt.act[i] = s.f32()[i];
      if (!std::isfinite(rt.act[i]) || rt.act[i] <= 0) fail(AEISU_ERR_ARTIFACT, "invalid activation scale");
    }
  }

  if (rt.mode == kModeFp32) {
    pack_fp32(rt, a, base.f32(), basis.f32());
    return;
  }

  // --- FP16 layers used by every policy: project, refine, tail
  auto w16 = [&](const std::string& l, std::initializer_list<uint32_t> shape) {
    return a.need(l + ".weight_fp16", kF16, shape).f16();
  };
  auto bias = [&](const std::string& l, uint32_t cout) { return as_f32_vector(a.need(l + ".bias", kF32, {cout})); };
  {
    // FP16 policy: hi/lo split operands (fragments hi T0, hi T1, lo T0, lo T1); the FP32
    // weights come from project.weight_fp32 when the artifact carries them.  Mixed / INT8:
    // FP16 weights as in the reference deployment (SrcPyrCudaRuntime.cu:2536-2566).
    const uint16_t* w = w16("project", {32, 32, 1, 1});
    require_prelu(a, "project", 32, 0.1f);
    rt.project_precise = rt.mode == 0;
    const float* w32 = nullptr;
    if (rt.project_precise && a.has("project.weight_fp32")) w32 = a.need("project.weight_fp32", kF32, {32, 32, 1, 1}).f32();
    rt.project.frag.upload(pack_frags<uint16_t>(rt.project_precise ? 4 : 2, 8, [&](int f, int m, int s) -> uint16_t {
      const int idx = (16 * (f & 1) + m) * 32 + s;
      if (!w32) return f < 2 ? w[idx] : (uint16_t)0;
      const uint16_t hi = f32_to_f16_bits(w32[idx]);
      return f < 2 ? hi : f32_to_f16_bits(w32[idx] - f16_bits_to_f32(hi));
    }));
    rt.project.bias.upload(bias("project", 32));
  }
  {
    const uint16_t* wr = w16("refine", {64, 32, 3, 3});
    const uint16_t* wt = w16("tail", {64, 64, 1, 1});
    require_prelu(a, "refine", 64, 0.1f);
    require_prelu(a, "tail", 64, 1.0f);
    auto img = pack_frags<uint16_t>(36, 8, [&](int f, int m, int s) {
      const int T = f / 9, tap = f % 9;
      return wr[((16 * T + m) * 32 + s) * 9 + tap];
    });
    auto tail = pack_frags<uint16_t>(8, 8, [&](int f, int m, int s) {
      const int T = f / 2, k = f % 2, g = s / 8, i = s % 8;
      return wt[(16 * T + m) * 64 + 16 * (2 * k + i / 4) + 4 * g + (i % 4)];
    });
    img.insert(img.end(), tail.begin(), tail.end());
    rt.refine_tail.frag.upload(img);
    rt.refine_tail.bias.upload(bias("refine", 64));
    std::vector<float> tb = bias("tail", 64);
    for (float& v : tb) v = f16_bits_to_f32(f32_to_f16_bits(v));  // FP16-rounded tail bias (SrcPyrNativeFp16Refine.cuh:494-495)
    rt.tail_bias.upload(tb);
  }

  // --- low-resolution body
  static const char* bodies[6] = {"compress", "bottleneck0", "bottleneck1", "bottleneck2", "bottleneck3", "expand"};
  for (int li = 0; li < 6; ++li) {
    const std::string l = bodies[li];
    const bool grp = li >= 1 && li <= 4;
    const uint32_t cout = li == 0 ? 64 : (li == 5 ? 128 : 64);
    const uint32_t cin = li == 0 ? 128 : (li == 5 ? 64 : 32);
    const uint32_t ks = grp ? 3 : 1;
    LayerDev& dst = li == 0 ? rt.compress : (li == 5 ? rt.expand : rt.grouped[li - 1]);
    require_prelu(a, l, cout, 0.1f);
    // generic element fetch W[o][i][tap] from whichever storage the policy uses
    if (rt.mode != 2) {
      const bool fp8 = rt.mode == 1 || rt.mode == 3;
      const uint8_t* codes = fp8 ? a.need(l + ".weight_fp8", kE4M3, {cout, cin, ks, ks}).data : nullptr;
      const uint16_t* half = fp8 ? nullptr : a.need(l + ".weight_fp16", kF16, {cout, cin, ks, ks}).f16();
      auto W = [&](int o, int i, int tap) -> uint32_t {
        const size_t idx = (size_t(o) * cin + i) * ks * ks + tap;
        return fp8 ? codes[idx] : half[idx];
      };
      std::function<uint32_t(int, int, int)> fn;
      int nfrag = 0;
      if (li == 0 && (rt.mode == 1 || rt.mode == 3)) {
        // E4M3 policies: slot s = 8g + j of phase chunk kappa takes skip channel pc(g, j) = 4g + j (j < 4) or
        // 16 + 4g + j - 4, the project accumulator order in which the frame-input fused body holds its
        // compress operands; every E4M3 compress kernel reads in this order, so each MFMA sums its 32
        // products in one order on every path (the MFMA's FP32 sum depends on that order)
        nfrag = 16;
        fn = [&](int f, int m, int s) {
          const int g = s / 8, j = s % 8, c = j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
          return W(16 * (f / 4) + m, c * 4 + (f % 4), 0);
        };
      } else if (li == 0) {
        nfrag = 16;  // f = T*4 + kappa(phase); slot s = skip channel c
        fn = [&](int f, int m, int s) { return W(16 * (f / 4) + m, s * 4 + (f % 4), 0); };
      } else if (li == 5) {
        nfrag = 16;  // f = T*2 + kappa; row m of tile T = channel c of phase T&3
        fn = [&](int f, int m, int s) {
          const int T = f / 2, k = f % 2, o = (16 * (T >> 2) + m) * 4 + (T & 3);
          return W(o, 32 * k + s, 0);
        };
      } else {
        nfrag = 36;  // f = (group*2 + T)*9 + tap
        fn = [&](int f, int m, int s) {
          const int gt = f / 9, tap = f % 9;
          return W(32 * (gt / 2) + 16 * (gt % 2) + m, s, tap);
        };
      }
      if (rt.mode == 1)
        dst.frag.upload(pack_frags<uint8_t>(nfrag, 8, [&](int f, int m, int s) { return (uint8_t)fn(f, m, s); }));
      else if (rt.mode == 3)  // E4M3 values widened exactly to FP16 for the FP16 MFMA
        dst.frag.upload(pack_frags<uint16_t>(nfrag, 8, [&](int f, int m, int s) {
          return f32_to_f16_bits(e4m3_value((uint8_t)fn(f, m, s)));
        }));
      else
        dst.frag.upload(pack_frags<uint16_t>(nfrag, 8, [&](int f, int m, int s) { return (uint16_t)fn(f, m, s); }));
      if (fp8) {
        const int s_in = li == 0 ? 1 : li + 1;  // compress s1, bottleneck i s(i+2), expand s6
        const TensorView& ws = a.need(l + ".weight_scale", kF32, {cout});
        std::vector<float> sc(cout);
        for (uint32_t c = 0; c < cout; ++c) sc[c] = rt.act[s_in] * ws.f32()[c];
        dst.scale.upload(sc);
        dst.bias.upload(as_f32_vector(a.need(l + ".bias_fp8", kF32, {cout})));
      } else {
        dst.bias.upload(bias(l, cout));
      }
    } else {
      const int8_t* q = reinterpret_cast<const int8_t*>(a.need(l + ".weight_i8", kI8, {cout, cin, ks, ks}).data);
      auto W = [&](int o, int i, int tap) -> int8_t { return q[(size_t(o) * cin + i) * ks * ks + tap]; };
      std::vector<int8_t> img;
      if (li == 0) {
        img = pack_frags<int8_t>(8, 16, [&](int f, int m, int s) {  // f = T*2 + k
          const int T = f / 2, k = f % 2, g = s / 16, i = s % 16;
          const int ph = 2 * k + (g >> 1), c = 16 * (g & 1) + i;
          return W(16 * T + m, c * 4 + ph, 0);
        });
        // frame-input fused body: slots 16g + i take phase 2k + (i >= 8), project accumulator
        // channel pc(g, i & 7)
        rt.compress_rgb.upload(pack_frags<int8_t>(8, 16, [&](int f, int m, int s) {
          const int T = f / 2, k = f % 2, g = s / 16, i = s % 16, j = i & 7;
          const int ph = 2 * k + (i >> 3), c = j < 4 ? 4 * g + j : 16 + 4 * g + j - 4;
          return W(16 * T + m, c * 4 + ph, 0);
        }));
      } else if (li == 5) {
        img = pack_frags<int8_t>(8, 16, [&](int T, int m, int s) {
          return W((16 * (T >> 2) + m) * 4 + (T & 3), s, 0);
        });
      } else {
        img = pack_frags<int8_t>(20, 16, [&](int f, int m, int s) {  // f = (group*2 + T)*5 + k
          const int gt = f / 5, k = f % 5, g = s / 16, i = s % 16;
          const int tap = 2 * k + (g >> 1), c = 16 * (g & 1) + i;
          return tap > 8 ? (int8_t)0 : W(32 * (gt / 2) + 16 * (gt % 2) + m, c, tap);
        });
      }
      dst.frag.upload(img);
      dst.scale.upload(as_f32_vector(a.need(l + ".int8_factor", kF32, {cout})));
      dst.bias.upload(bias(l, cout));
    }
  }

  // --- fused-body epilogue constants (layout: kBodyConsts in kernels.hpp), from the staged images
  {
    auto staged_f32 = [](const DeviceBuffer& d, size_t i) {
      float v = 0.f;
      if (!d.staged.empty()) std::memcpy(&v, d.staged.data() + 4 * i, 4);
      return v;
    };
    std::vector<float> cst(kBodyConsts, 0.f);
    const LayerDev* body[5] = {&rt.compress, &rt.grouped[0], &rt.grouped[1], &rt.grouped[2], &rt.grouped[3]};
    for (int l = 0; l < 5; ++l)
      for (int c = 0; c < 64; ++c) {
        cst[128 * l + c] = staged_f32(body[l]->bias, c);
        cst[128 * l + 64 + c] = rt.mode ? staged_f32(body[l]->scale, c) : 0.f;
      }
    for (int j = 0; j < 128; ++j) {
      const int T = j >> 4, mm = j & 15, o = (16 * (T >> 2) + mm) * 4 + (T & 3);
      cst[640 + j] = staged_f32(rt.expand.bias, o);
      cst[768 + j] = rt.mode ? staged_f32(rt.expand.scale, o) : 0.f;
    }
    for (int c = 0; c < 32; ++c) cst[896 + c] = staged_f32(rt.project.bias, c);
    rt.body_consts.upload(cst);
  }

  // --- head bank: two K=32 fragment sets of 7 row tiles each, FP32 accumulation in the kernel:
  //   A1  = [K_hi | K_lo]                         against [u ; u]
  //   A23 = slots 8g..8g+3: (0.05 K)_hi of coefficients 4g..4g+3, slots 4, 5: base_hi, base_lo
  //                                               against the lane's own w and [1, 1] (group 0)
  // (clamp(a) = u + 0.05 w in the kernel).  Row m = 4g + i of tile t is (phase g, tap 4t + i);
  // taps 25..27 (tile 6, i > 0) are zero rows.  The accumulator lane (n, g) thus holds all 25
  // taps of phase g for pixel n.  After the fragments (kHeadBankFrags of them): the FP32 base
  // of those rows, float4 [g][t] = base[tap 4t + i][phase g], i = 0..3, the accumulator input
  // of the quantized policies' head (A1 against [c ; c], c the clamped coefficient in FP16).
  {
    const float* K = basis.f32();  // [25][16][4]
    const float* B = base.f32();   // [25][4]
    auto row_of = [](int t, int m, int& tap, int& ph) {
      const int g = m / 4, i = m % 4;
      tap = 4 * t + i;
      ph = g;
      if (tap > 24) tap = -1;
    };
    auto hi = [](double v) { return f32_to_f16_bits((float)v); };
    auto lo = [](double v) {
      return f32_to_f16_bits((float)(v - (double)f16_bits_to_f32(f32_to_f16_bits((float)v))));
    };
    std::vector<uint16_t> img = pack_frags<uint16_t>(kHeadBankFrags, 8, [&](int f, int m, int s) -> uint16_t {
      int tap, ph;
      row_of(f % 7, m, tap, ph);
      if (tap < 0) return 0;
      if (f < 7) {
        const double k = K[(tap * 16 + (s & 15)) * 4 + ph];
        return s < 16 ? hi(k) : lo(k);
      }
      const int gs = s / 8, i = s % 8;
      if (i < 4) return hi(0.05 * (double)K[(tap * 16 + 4 * gs + i) * 4 + ph]);
      if (s == 4) return hi(B[tap * 4 + ph]);
      if (s == 5) return lo(B[tap * 4 + ph]);
      return 0;
    });
    std::vector<float> basec(4 * 7 * 4, 0.f);
    for (int g = 0; g < 4; ++g)
      for (int t = 0; t < 7; ++t)
        for (int i = 0; i < 4; ++i)
          if (4 * t + i < 25) basec[(g * 7 + t) * 4 + i] = B[(4 * t + i) * 4 + g];
    const size_t frag_halves = img.size();
    img.resize(frag_halves + basec.size() * 2);
    std::memcpy(img.data() + frag_halves, basec.data(), basec.size() * sizeof(float));
    rt.head.frag.upload(img);
  }
}

static void commit_weights(ModeWeights& w) {
  w.each_buffer([](DeviceBuffer& b) { b.commit(); });
}

// Per-device set-up that every launch path needs: the fused kernels' LDS limits, and the address of
// the library's static scratch array (defined with the allocation-free entry point in noalloc.hip).
static std::mutex g_prepare_mu;
static bool g_prepared[64];
static void prepare_device(int device) {
  std::lock_guard<std::mutex> lock(g_prepare_mu);
  if (device < 0 || device >= 64) fail(AEISU_ERR_HIP, "device ordinal out of range");
  if (g_prepared[device]) return;
  check_hip(fused_prepare(), "hipFuncSetAttribute(fused LDS)");
  check_hip(body_fused_prepare(), "hipFuncSetAttribute(fused body LDS)");
  check_hip(noalloc_scratch_init(device), "hipGetSymbolAddress(scratch)");
  g_prepared[device] = true;
}

const ModeWeights& Model::weights(int mode) {
  std::lock_guard<std::mutex> lock(mu);
  if (!modes[mode]) {
    auto w = std::make_unique<ModeWeights>();
    w->mode = mode;
    pack_weights(*w, art);          // host-only: validates every tensor the policy needs
    check_hip(hipSetDevice(device), "hipSetDevice");
    commit_weights(*w);
    modes[mode] = std::move(w);
  }
  return *modes[mode];
}

static int clamp_grid(int tiles, int per_cu, int cus) {
  int g = std::min(tiles, std::max(1, per_cu) * cus);
  if (g >= 8) g -= g % 8;
  return std::max(g, 1);
}

static Geometry make_geometry(int mode, bool project_precise, int cus, int batch, int height, int width, int in_layout,
                              int out_layout, unsigned flags) {
  if (batch <= 0 || height <= 0 || width <= 0) fail(AEISU_ERR_INVALID_ARGUMENT, "batch, height and width must be positive");
  if (height > 8192 || width > 8192 || batch > 1024) fail(AEISU_ERR_INVALID_ARGUMENT, "frame dimensions exceed 8192 (or batch > 1024)");
  if ((in_layout != AEISU_LAYOUT_NCHW_F16 && in_layout != AEISU_LAYOUT_NCHW_F32) ||
      (out_layout != AEISU_LAYOUT_NCHW_F16 && out_layout != AEISU_LAYOUT_NCHW_F32))
    fail(AEISU_ERR_INVALID_ARGUMENT, "unsupported frame layout");
  if (flags & ~(AEISU_FLAG_KEEP_INTERMEDIATES | AEISU_FLAG_STAGE_TIMING | AEISU_FLAG_NO_PAD | AEISU_FLAG_UNFUSED |
                AEISU_FLAG_BODY_TILE24 | AEISU_FLAG_BODY_NO_EXCHANGE | AEISU_FLAG_BODY_EXCHANGE_FALLBACK))
    fail(AEISU_ERR_INVALID_ARGUMENT, "unknown configure flag");
  const bool no_pad = flags & AEISU_FLAG_NO_PAD;
  if (no_pad && (height % 4 || width % 4))
    fail(AEISU_ERR_INVALID_ARGUMENT, "Source H/W must be divisible by 4");
  Geometry g;
  g.batch = batch;
  g.H = height;
  g.W = width;
  if (no_pad) {
    // The caller passes a frame that is already on the padded grid (aeisu/model.py:473-479).
    g.py = g.px = 0;
    g.Hp = height;
    g.Wp = width;
  } else {
    // align32 + halo16 replicate padding (aeisu/runtime.py:82-84), realised by clamped reads.
    const int ey = (32 - height % 32) % 32, ex = (32 - width % 32) % 32;
    g.py = 16 + ey / 2;
    g.px = 16 + ex / 2;
    g.Hp = height + 32 + ey;
    g.Wp = width + 32 + ex;
  }
  g.Hq = g.Hp / 2;
  g.Wq = g.Wp / 2;
  g.Hl = g.Hp / 4;
  g.Wl = g.Wp / 4;
  g.in_fp32 = in_layout == AEISU_LAYOUT_NCHW_F32;
  g.out_fp32 = out_layout == AEISU_LAYOUT_NCHW_F32;
  g.flags = flags;
  g.cus = cus;
  if (mode == kModeFp32) {
    // per-layer FP32 kernels, one thread per pixel (no persistent grids, no fused variants)
    g.act_bytes = g.low_bytes = 4;
    g.nlow = (flags & AEISU_FLAG_KEEP_INTERMEDIATES) ? 5 : 2;
    return g;
  }
  g.low_bytes = mode == 0 ? 2 : 1;
  g.fused = !(flags & (AEISU_FLAG_KEEP_INTERMEDIATES | AEISU_FLAG_UNFUSED));
  // the skip tensor only exists in device memory where the project kernel runs
  g.fused_rgb = g.fused && mode != 0;
  g.qclamp = mode != 0;
  // low-resolution activations only reach device memory on the per-layer path
  g.nlow = (flags & AEISU_FLAG_KEEP_INTERMEDIATES) ? 5 : (g.fused ? 0 : 2);
  const int low_groups = batch * g.Hl * ((g.Wl + 15) / 16);
  g.grid.project = clamp_grid(project_num_tiles(batch, g.Hq, g.Wq), project_blocks_per_cu(g.in_fp32, project_precise), cus);
  g.grid.compress = clamp_grid((low_groups + 3) / 4, body_blocks_per_cu(0, mode), cus);
  g.grid.grouped = clamp_grid(grouped_num_tiles(batch, g.Hl, g.Wl), body_blocks_per_cu(1, mode), cus);
  g.grid.expand = clamp_grid((low_groups + 3) / 4, body_blocks_per_cu(2, mode), cus);
  g.grid.refine = clamp_grid(refine_num_tiles(batch, g.Hq, g.Wq), refine_blocks_per_cu(), cus);
  g.grid.head = clamp_grid(head_num_tiles(batch, height, width), head_blocks_per_cu(g.in_fp32, g.out_fp32, g.qclamp), cus);
  const BodyPlan plan = (flags & AEISU_FLAG_BODY_TILE24) ? BodyPlan{batch, 0} : body_fused_plan(mode, batch, g.Hl, g.Wl, cus);
  g.body_split = plan.frames24;
  g.body_cols24 = plan.cols24;
  g.body_rows16 = (flags & AEISU_FLAG_BODY_TILE24) ? g.Hl : body_fused_row_split(mode, batch, g.Hl, g.Wl, cus);
  g.cus = cus;
  // compress exchange: a whole-batch launch of one tile side whose tiles all fit on the device at
  // once (one block per CU), else launches of whole frames where they beat the plan without it
  if (g.fused_rgb && !(flags & AEISU_FLAG_BODY_NO_EXCHANGE)) {
    if (plan.cols24 == 0 && (plan.frames24 == batch || plan.frames24 == 0)) {
      const int tile = plan.frames24 == batch ? 24 : 16;
      if (body_fused_num_tiles(mode, batch, g.Hl, g.Wl, tile) <= cus) {
        g.body_xc_tile = tile;
        g.body_xc_frames = batch;
      }
    }
    if (!g.body_xc_tile && batch > 1) {
      const BodyXcPlan xp = body_fused_xc_plan(mode, batch, g.Hl, g.Wl, cus, flags & AEISU_FLAG_BODY_TILE24);
      g.body_xc_tile = xp.tile;
      g.body_xc_frames = xp.frames;
    }
  }
  g.grid.fused = clamp_grid(fused_num_tiles(g.in_fp32, batch, height, width, g.Hq, g.Wq, g.py, g.px), 1, cus);
  return g;
}

static float inv(float s) { return 1.0f / s; }

// Compress exchange: polls of a neighbour's counter before a tile computes its halo ring itself.  A
// poll is one device-scope load (about a microsecond); neighbours normally publish within a few.
constexpr int kExchangePolls = 128;

// Low-buffer slot written by body layer li (0 compress, 1..4 bottlenecks).
static int low_slot(const Geometry& g, int li) { return g.nlow == 5 ? li : (li % 2); }

// project .. expand (the controller up to the FP16 work tensor); events 0..4
static void enqueue_body(const ModeWeights& w, const Geometry& g, const Scratch& sc, const void* d_in, hipStream_t s,
                         hipEvent_t* ev) {
  const int m = w.mode;
  if (ev) check_hip(hipEventRecord(ev[0], s), "hipEventRecord");
  if (g.fused_rgb) {
    // analysis + project + compress .. expand in one kernel from the frames, timed as the
    // bottleneck stage (events 0 -> 3; project, compress and expand report zero)
    BodyFusedArgs P{};
    P.frames = d_in;
    P.work = static_cast<_Float16*>(sc.work);
    P.consts = w.body_consts.as<float>();
    const LayerDev* layers[6] = {&w.compress, &w.grouped[0], &w.grouped[1], &w.grouped[2], &w.grouped[3], &w.expand};
    for (int l = 0; l < 6; ++l) {
      P.frag[l] = layers[l]->frag.ptr;
      P.inv_out[l] = inv(w.act[l + 2]);
    }
    if (m == 2) P.frag[0] = w.compress_rgb.ptr;     // INT8: its own frame-input K order
    P.pfrag = w.project.frag.ptr;
    P.inv_in = inv(w.act[1]);
    P.s_out = w.act[7];
    for (int i = 0; i < 24; ++i) P.analysis[i] = w.analysis[i];
    P.Hl = g.Hl;
    P.Wl = g.Wl;
    P.H = g.H;
    P.W = g.W;
    P.py = g.py;
    P.px = g.px;
    const BodySrc src = g.in_fp32 ? BodySrc::Frames32 : BodySrc::Frames16;
    const int k = g.body_split;
    if (g.body_xc_tile) {                          // compress exchange between neighbouring tiles
      P.xspins = (g.flags & AEISU_FLAG_BODY_EXCHANGE_FALLBACK) ? 0 : kExchangePolls;
      // launches of whole frames, each with its own part of the exchange tensor and counters
      const int per_frame = body_fused_num_tiles(m, 1, g.Hl, g.Wl, g.body_xc_tile);
      const size_t in_frame = size_t(3) * g.H * g.W * (g.in_fp32 ? 4 : 2);
      for (int f0 = 0; f0 < g.batch; f0 += g.body_xc_frames) {
        BodyFusedArgs Q = P;
        Q.frames = static_cast<const char*>(P.frames) + size_t(f0) * in_frame;
        Q.work = P.work + size_t(f0) * g.Hq * g.Wq * 32;
        Q.xbuf = static_cast<unsigned char*>(sc.xbuf) + size_t(f0) * g.Hl * g.Wl * 64;
        Q.xflags = sc.xflags + size_t(f0) * per_frame;
        check_launch(launch_body_fused_xc(m, src, Q, std::min(g.body_xc_frames, g.batch - f0), g.body_xc_tile, g.cus, s),
                     "fused body launch", s);
      }
    } else if (g.body_cols24 > 0) {                       // right-hand columns on 16x16 tiles
      BodyFusedArgs Q = P;
      P.col0 = 0;
      P.cols = g.body_cols24;
      Q.col0 = g.body_cols24;
      Q.cols = g.Wl - g.body_cols24;
      check_launch(launch_body_fused_pair(m, src, P, g.batch, 24, Q, g.batch, 16, s), "fused body launch", s);
    } else if (k == g.batch) {
      check_launch(launch_body_fused(m, src, P, k, 24, s), "fused body launch", s);
    } else {                                       // trailing frames on 16x16 tiles
      BodyFusedArgs Q = P;
      Q.frames = static_cast<const char*>(P.frames) + size_t(k) * 3 * g.H * g.W * (g.in_fp32 ? 4 : 2);
      Q.work = P.work + size_t(k) * g.Hq * g.Wq * 32;
      if (k == 0) check_launch(launch_body_fused(m, src, Q, g.batch, 16, s), "fused body launch", s);
      else check_launch(launch_body_fused_pair(m, src, P, k, 24, Q, g.batch - k, 16, s), "fused body launch", s);
    }
    if (ev) check_hip(hipEventRecord(ev[3], s), "hipEventRecord");
    return;
  }
  check_launch(launch_project(g.in_fp32, w.project_precise, d_in, w.project.frag.ptr, w.project.bias.as<float>(), sc.skip,
                              w.analysis, g.H, g.W, g.Hq, g.Wq, g.py, g.px, g.batch, g.grid.project, s), "project launch", s);
  if (ev) check_hip(hipEventRecord(ev[1], s), "hipEventRecord");
  const float* A = w.act;
  if (g.fused) {
    // one kernel for compress .. expand, timed as the bottleneck stage (events 1 -> 3;
    // aeisu_stage_timings reports compress and expand as zero on this path)
    BodyFusedArgs P{};
    P.skip = static_cast<const _Float16*>(sc.skip);
    P.work = static_cast<_Float16*>(sc.work);
    P.consts = w.body_consts.as<float>();
    const LayerDev* layers[6] = {&w.compress, &w.grouped[0], &w.grouped[1], &w.grouped[2], &w.grouped[3], &w.expand};
    for (int l = 0; l < 6; ++l) {
      P.frag[l] = layers[l]->frag.ptr;
      P.inv_out[l] = m ? inv(A[l + 2]) : 0.f;   // compress s2, bottleneck i s(i+3), expand s7
    }
    P.inv_in = m ? inv(A[1]) : 0.f;
    P.s_out = m ? A[7] : 0.f;
    P.Hl = g.Hl;
    P.Wl = g.Wl;
    if (m != 0 || g.body_rows16 >= g.Hl) {
      check_launch(launch_body_fused(m, BodySrc::Skip, P, g.batch, 0, s), "fused body launch", s);
    } else {                                       // FP16 policy: bottom rows on 8x8 tiles
      BodyFusedArgs Q = P;
      Q.row0 = g.body_rows16;
      Q.rows = g.Hl - g.body_rows16;
      if (g.body_rows16 == 0) {
        check_launch(launch_body_fused(m, BodySrc::Skip, Q, g.batch, 8, s), "fused body launch", s);
      } else {
        P.row0 = 0;
        P.rows = g.body_rows16;
        check_launch(launch_body_fused_pair(m, BodySrc::Skip, P, g.batch, 16, Q, g.batch, 8, s), "fused body launch", s);
      }
    }
    if (ev) check_hip(hipEventRecord(ev[3], s), "hipEventRecord");
    return;
  }
  check_launch(launch_compress(m, sc.skip, w.compress.frag.ptr, w.compress.bias.as<float>(), w.compress.scale.as<float>(),
                               sc.low[low_slot(g, 0)], m ? inv(A[1]) : 0.f, m ? inv(A[2]) : 0.f, g.Hl, g.Wl, g.batch,
                               g.grid.compress, s), "compress launch", s);
  if (ev) check_hip(hipEventRecord(ev[2], s), "hipEventRecord");
  for (int i = 0; i < 4; ++i) {
    check_launch(launch_grouped(m, sc.low[low_slot(g, i)], w.grouped[i].frag.ptr, w.grouped[i].bias.as<float>(),
                                w.grouped[i].scale.as<float>(), sc.low[low_slot(g, i + 1)], m ? inv(A[i + 3]) : 0.f,
                                g.Hl, g.Wl, g.batch, g.grid.grouped, s), "bottleneck launch", s);
  }
  if (ev) check_hip(hipEventRecord(ev[3], s), "hipEventRecord");
  check_launch(launch_expand(m, sc.low[low_slot(g, 4)], sc.skip, w.expand.frag.ptr, w.expand.bias.as<float>(),
                             w.expand.scale.as<float>(), sc.work, m ? inv(A[7]) : 0.f, m ? A[7] : 0.f, g.Hl, g.Wl,
                             g.batch, g.grid.expand, s), "expand launch", s);
  if (ev) check_hip(hipEventRecord(ev[4], s), "hipEventRecord");
}

static void enqueue_controller(const ModeWeights& w, const Geometry& g, const Scratch& sc, const void* d_in,
                               void* d_meta, hipStream_t s, hipEvent_t* ev) {
  enqueue_body(w, g, sc, d_in, s, ev);
  check_launch(launch_refine_tail(sc.work, w.refine_tail.frag.ptr, w.refine_tail.bias.as<float>(),
                                  w.tail_bias.as<float>(), d_meta, g.Hq, g.Wq, g.batch, g.grid.refine, s),
               "refine/tail launch", s);
  if (ev) check_hip(hipEventRecord(ev[5], s), "hipEventRecord");
}

static void enqueue_head(const ModeWeights& w, const Geometry& g, const Scratch& sc, const void* d_in,
                         const void* d_meta, void* d_out, hipStream_t s) {
  check_launch(launch_head(g.in_fp32, g.out_fp32, g.qclamp, d_in, d_meta, w.head.frag.ptr, d_out, g.H, g.W, g.Hq, g.Wq,
                           g.py, g.px, g.batch, sc.nonfinite, g.grid.head, s), "head launch", s);
}

// FP32 policy: project, compress, 4 grouped, expand, refine + tail, head; events 0..6 as the per-layer path
static void enqueue_fp32(const ModeWeights& w, const Geometry& g, const Scratch& sc, const void* d_in, void* d_out,
                         hipStream_t s, hipEvent_t* ev) {
  if (ev) check_hip(hipEventRecord(ev[0], s), "hipEventRecord");
  float* lows[5];
  for (int i = 0; i < 5; ++i) lows[i] = static_cast<float*>(sc.low[i]);
  check_launch(launch_f32_controller(g.in_fp32, d_in, w.fp32.as<float>(), static_cast<float*>(sc.skip), lows[0], lows[1],
                                     g.nlow == 5 ? lows : nullptr, static_cast<float*>(sc.work), static_cast<float*>(sc.meta),
                                     g.H, g.W, g.Hq, g.Wq, g.py, g.px, g.batch, s, ev),
               "FP32 controller launch", s);
  check_launch(launch_f32_head(g.in_fp32, g.out_fp32, d_in, static_cast<const float*>(sc.meta), w.fp32.as<float>(), d_out,
                               g.H, g.W, g.Hq, g.Wq, g.py, g.px, g.batch, sc.nonfinite, s),
               "FP32 head launch", s);
  if (ev) check_hip(hipEventRecord(ev[6], s), "hipEventRecord");
}

static void enqueue_frame(const ModeWeights& w, const Geometry& g, const Scratch& sc, const void* d_in, void* d_out,
                          hipStream_t s, hipEvent_t* ev) {
  if (w.mode == kModeFp32) {
    enqueue_fp32(w, g, sc, d_in, d_out, s, ev);
    return;
  }
  if (!g.fused) {
    enqueue_controller(w, g, sc, d_in, sc.meta, s, ev);
    enqueue_head(w, g, sc, d_in, sc.meta, d_out, s);
    if (ev) check_hip(hipEventRecord(ev[6], s), "hipEventRecord");
    return;
  }
  // fused path: events 0, (1,) 3, 6 only; the head stage times refine + tail + head (3 -> 6)
  enqueue_body(w, g, sc, d_in, s, ev);
  check_launch(launch_fused_tail_head(g.in_fp32, g.out_fp32, g.qclamp, sc.work, d_in, w.refine_tail.frag.ptr,
                                      w.refine_tail.bias.as<float>(), w.tail_bias.as<float>(), w.head.frag.ptr, d_out,
                                      g.H, g.W, g.Hq, g.Wq, g.py, g.px, g.batch, sc.nonfinite, g.grid.fused, s),
               "fused refine/tail/head launch", s);
  if (ev) check_hip(hipEventRecord(ev[6], s), "hipEventRecord");
}

static std::string startup_report(const Runtime& rt) {
  const Model& md = *rt.model;
  const Geometry& g = rt.g;
  std::ostringstream r;
  r << "aeisu_amd architecture=" << kArchitecture << " sha256=" << md.art.checksum_hex << " GPU=\"" << md.gpu_name
    << "\" arch=" << md.gcn_arch << " CUs=" << md.cu_count << " HIP=" << md.hip_runtime_version
    << " precision=" << precision_name(rt.mode)
    << " body=" << (g.fused ? (g.fused_rgb ? "fused-analysis-project-compress-4x-grouped-expand"
                                           : "project+fused-compress-4x-grouped-expand")
                            : "per-layer-kernels")
    << " body_mfma=" << (rt.mode == 0 ? "f16" : rt.mode == 1 ? "fp8" : rt.mode == 2 ? "i8" : rt.mode == 3 ? "f16-on-e4m3-values" : "none-fp32-fma")
    << " head=" << (g.fused ? "fused-refine-tail-reconstruction" : "refine-tail+reconstruction")
    << " source=" << g.W << 'x' << g.H << " batch=" << g.batch << " padded=" << g.Wp << 'x' << g.Hp
    << " packed=" << g.Wq << 'x' << g.Hq << " low=" << g.Wl << 'x' << g.Hl << " source_pad=" << g.px << ','
    << g.py << " io=" << (g.in_fp32 ? "f32" : "f16") << '/' << (g.out_fp32 ? "f32" : "f16")
    << " body_tiles24_frames=" << g.body_split << " body_tiles24_cols=" << g.body_cols24
    << " body_exchange_tile=" << g.body_xc_tile << " body_exchange_frames=" << g.body_xc_frames
    << " weights_bytes=" << rt.w->bytes()
    << " scratch_bytes=" << rt.scratch_bytes() << " static_scratch_bytes=" << kNoAllocScratchBytes
    << " shared_model_users=" << rt.model.use_count();
  return r.str();
}

static void configure(Runtime& rt, int batch, int height, int width, int in_layout, int out_layout, int precision,
                      unsigned flags) {
  const int mode = precision ? mode_of(precision) : rt.mode;
  const ModeWeights& w = rt.model->weights(mode);
  Geometry g = make_geometry(mode, w.project_precise, rt.model->cu_count, batch, height, width, in_layout, out_layout,
                             flags);
  if (rt.configured) (void)hipDeviceSynchronize();   // earlier frames may still use the scratch freed below
  rt.drop_graph();
  rt.configured = false;
  rt.timed_frames = 0;                 // recorded stage events belong to the previous layout
  rt.skip.alloc(g.skip_bytes());
  rt.work.alloc(g.work_bytes());
  rt.meta.alloc(g.meta_bytes());
  for (int i = 0; i < 5; ++i) rt.low[i].alloc(i < g.nlow ? g.low_layer_bytes() : 0);
  rt.nonfinite.alloc(4);
  check_hip(hipMemset(rt.nonfinite.ptr, 0, 4), "hipMemset(flag)");
  rt.xbuf.alloc(g.xbuf_bytes());
  rt.xflags.alloc(g.xflag_bytes());
  if (rt.xflags.ptr) check_hip(hipMemset(rt.xflags.ptr, 0, rt.xflags.bytes), "hipMemset(exchange counters)");
  if (precision) rt.precision = precision;
  rt.mode = mode;
  rt.w = &w;
  rt.g = g;
  rt.configured = true;
  rt.report = startup_report(rt);
}

static hipEvent_t* next_events(Runtime& rt) {
  if (!(rt.g.flags & AEISU_FLAG_STAGE_TIMING) || rt.timed_frames >= kMaxTimedFrames) return nullptr;
  const size_t need = size_t(rt.timed_frames + 1) * kStageEvents;
  while (rt.events.size() < need) {
    hipEvent_t e;
    check_hip(hipEventCreate(&e), "hipEventCreate");
    rt.events.push_back(e);
  }
  return &rt.events[size_t(rt.timed_frames++) * kStageEvents];
}

static void require_configured(const Runtime& rt) {
  if (!rt.configured) fail(AEISU_ERR_STATE, "runtime is not configured");
}

// The default (fused) path on the static scratch array: geometry on the stack, no allocation.
// Scratch layout: [0, 256) non-finite flag, then the skip tensor (FP16 policy) and the work tensor,
// each 256-byte aligned.
static void enqueue_noalloc(const Runtime& rt, int batch, int height, int width, int in_layout, int out_layout,
                            const void* d_in, void* d_out, hipStream_t s) {
  if (rt.mode == kModeFp32)
    fail(AEISU_ERR_STATE, "the allocation-free entry point runs the fused path; the FP32 policy runs per-layer "
                          "kernels on FP32 activations (use aeisu_upscale_async)");
  Geometry g = make_geometry(rt.mode, rt.w->project_precise, rt.model->cu_count, batch, height, width, in_layout,
                             out_layout, 0);
  g.body_xc_tile = g.body_xc_frames = 0;           // the exchange needs its own zeroed counters
  auto up = [](size_t n) { return (n + 255) & ~size_t(255); };
  const size_t need = 256 + up(g.skip_bytes()) + up(g.work_bytes());
  if (need > kNoAllocScratchBytes)
    fail(AEISU_ERR_INVALID_ARGUMENT, "frame needs " + std::to_string(need) + " bytes of scratch; the allocation-free "
                                     "entry point has " + std::to_string(kNoAllocScratchBytes));
  char* base = static_cast<char*>(noalloc_scratch(rt.model->device));
  if (!base) fail(AEISU_ERR_STATE, "static scratch was not set up on this device");
  Scratch sc;
  sc.nonfinite = reinterpret_cast<unsigned*>(base);
  sc.skip = g.skip_bytes() ? base + 256 : nullptr;
  sc.work = base + 256 + up(g.skip_bytes());
  enqueue_frame(*rt.w, g, sc, d_in, d_out, s, nullptr);
}

}  // namespace aeisu

// ================================================================================================
// C ABI
// ================================================================================================
using aeisu::Error;
using aeisu::Runtime;

struct aeisu_runtime {
  std::unique_ptr<Runtime> impl;
};

static thread_local std::string g_last_error;

template <typename Fn>
static int guarded(Fn fn) {
  try {
    fn();
    g_last_error.clear();
    return AEISU_OK;
  } catch (const Error& e) {
    g_last_error = e.what();
    return e.code;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return AEISU_ERR_HIP;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return AEISU_ERR_HIP;
  }
}

static Runtime& runtime_of(aeisu_runtime* rt) {
  if (!rt || !rt->impl) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null runtime handle");
  aeisu::check_hip(hipSetDevice(rt->impl->model->device), "hipSetDevice");
  return *rt->impl;
}

static int create_impl(const uint8_t* data, size_t size, int precision, aeisu_runtime** out) {
  return guarded([&] {
    if (!out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!data || size == 0) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "empty artifact");
    const int mode = aeisu::mode_of(precision);
    auto model = std::make_shared<aeisu::Model>();
    model->art = aeisu::parse_artifact(data, size);   // host-only validation before any HIP call
    {
      // pack (and so validate) the requested policy's tensors on the host first
      aeisu::ModeWeights probe;
      probe.mode = mode;
      aeisu::pack_weights(probe, model->art);
    }
    aeisu::check_hip(hipGetDevice(&model->device), "hipGetDevice");
    hipDeviceProp_t prop;
    aeisu::check_hip(hipGetDeviceProperties(&prop, model->device), "hipGetDeviceProperties");
    model->cu_count = prop.multiProcessorCount;
    model->gpu_name = prop.name;
    model->gcn_arch = prop.gcnArchName;
    aeisu::check_hip(hipRuntimeGetVersion(&model->hip_runtime_version), "hipRuntimeGetVersion");
    aeisu::prepare_device(model->device);
    auto rt = std::make_unique<Runtime>();
    rt->model = model;
    rt->precision = precision;
    rt->mode = mode;
    rt->w = &model->weights(mode);
    auto* h = new aeisu_runtime;
    h->impl = std::move(rt);
    *out = h;
  });
}

extern "C" {

int aeisu_create_from_memory(const void* data, size_t size, int precision, aeisu_runtime** out) {
  return create_impl(static_cast<const uint8_t*>(data), size, precision, out);
}

int aeisu_create_from_file(const char* path, int precision, aeisu_runtime** out) {
  std::vector<uint8_t> bytes;
  const int rc = guarded([&] {
    if (!path) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null path");
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) aeisu::fail(AEISU_ERR_ARTIFACT, std::string("could not open SPYR8 model: ") + path);
    const std::streamsize n = f.tellg();
    f.seekg(0);
    bytes.resize(size_t(std::max<std::streamsize>(n, 0)));
    if (n <= 0 || !f.read(reinterpret_cast<char*>(bytes.data()), n))
      aeisu::fail(AEISU_ERR_ARTIFACT, "failed to read complete SPYR8 artifact");
  });
  if (rc != AEISU_OK) {
    if (out) *out = nullptr;
    return rc;
  }
  return create_impl(bytes.data(), bytes.size(), precision, out);
}

int aeisu_create_sibling(const aeisu_runtime* src, aeisu_runtime** out) {
  return guarded([&] {
    if (!out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (!src || !src->impl) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null runtime handle");
    const Runtime& s = *src->impl;
    auto rt = std::make_unique<Runtime>();
    rt->model = s.model;
    rt->precision = s.precision;
    rt->mode = s.mode;
    rt->w = s.w;
    auto* h = new aeisu_runtime;
    h->impl = std::move(rt);
    *out = h;
  });
}

int aeisu_shares_weights(const aeisu_runtime* a, const aeisu_runtime* b) {
  return a && b && a->impl && b->impl && a->impl->model == b->impl->model;
}

int aeisu_configure(aeisu_runtime* h, int batch, int height, int width, int in_layout, int out_layout, int precision,
                    unsigned flags) {
  return guarded([&] {
    aeisu::configure(runtime_of(h), batch, height, width, in_layout, out_layout, precision, flags);
  });
}

int aeisu_upscale_async(aeisu_runtime* h, const void* d_in, void* d_out, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    if (!d_in || !d_out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null frame buffer");
    aeisu::enqueue_frame(*rt.w, rt.g, rt.scratch(), d_in, d_out, (hipStream_t)stream, aeisu::next_events(rt));
  });
}

int aeisu_upscale_noalloc(aeisu_runtime* h, int batch, int height, int width, int in_layout, int out_layout,
                          const void* d_in, void* d_out, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    if (!d_in || !d_out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null frame buffer");
    aeisu::enqueue_noalloc(rt, batch, height, width, in_layout, out_layout, d_in, d_out, (hipStream_t)stream);
  });
}

int aeisu_check_finite(aeisu_runtime* h, void* stream) {
  int status = AEISU_OK;
  const int rc = guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    unsigned flag = 0;
    aeisu::check_hip(hipMemcpyAsync(&flag, rt.nonfinite.ptr, 4, hipMemcpyDeviceToHost, (hipStream_t)stream), "flag readback");
    aeisu::check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    if (flag) {
      aeisu::check_hip(hipMemsetAsync(rt.nonfinite.ptr, 0, 4, (hipStream_t)stream), "flag reset");
      aeisu::check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
      status = AEISU_ERR_NONFINITE;
    }
  });
  if (rc != AEISU_OK) return rc;
  if (status != AEISU_OK) g_last_error = "Non-finite model reconstruction";
  return status;
}

int aeisu_upscale(aeisu_runtime* h, const void* d_in, void* d_out, void* stream) {
  const int rc = aeisu_upscale_async(h, d_in, d_out, stream);
  if (rc != AEISU_OK) return rc;
  return aeisu_check_finite(h, stream);
}

int aeisu_upscale_graph(aeisu_runtime* h, const void* d_in, void* d_out, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    if (!d_in || !d_out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null frame buffer");
    hipGraphExec_t exec = nullptr;
    for (const auto& g : rt.graphs)
      if (g.in == d_in && g.out == d_out) exec = g.exec;
    if (!exec) {
      if (rt.graphs.size() >= Runtime::kMaxGraphs) rt.drop_graph();
      if (!rt.capture_stream)
        aeisu::check_hip(hipStreamCreateWithFlags(&rt.capture_stream, hipStreamNonBlocking), "hipStreamCreate");
      aeisu::check_hip(hipStreamBeginCapture(rt.capture_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      hipGraph_t graph = nullptr;
      try {
        aeisu::enqueue_frame(*rt.w, rt.g, rt.scratch(), d_in, d_out, rt.capture_stream, nullptr);
      } catch (...) {
        (void)hipStreamEndCapture(rt.capture_stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
      }
      aeisu::check_hip(hipStreamEndCapture(rt.capture_stream, &graph), "hipStreamEndCapture");
      // Topology check (as the reference checks its captured graph, SrcPyrCudaRuntime.cu:4914-4941): a
      // frame is kernel launches only.  A memset or copy node would also be replayed with every frame,
      // and memset nodes are not trusted to replay correctly here, so none may have been captured.
      {
        size_t n = 0;
        hipError_t ge = hipGraphGetNodes(graph, nullptr, &n);
        std::vector<hipGraphNode_t> nodes(n);
        if (ge == hipSuccess && n) ge = hipGraphGetNodes(graph, nodes.data(), &n);
        size_t kernels = 0;
        for (size_t i = 0; ge == hipSuccess && i < n; ++i) {
          hipGraphNodeType type;
          ge = hipGraphNodeGetType(nodes[i], &type);
          kernels += ge == hipSuccess && type == hipGraphNodeTypeKernel;
        }
        if (ge != hipSuccess || n == 0 || kernels != n) {
          (void)hipGraphDestroy(graph);
          aeisu::fail(AEISU_ERR_HIP, ge != hipSuccess ? std::string("reading the captured frame graph: ") + hipGetErrorString(ge)
                                                      : "captured frame graph holds " + std::to_string(n - kernels) +
                                                            " non-kernel node(s) among " + std::to_string(n));
        }
      }
      const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        aeisu::check_hip(e, "hipGraphInstantiate");
      }
      rt.graphs.push_back({d_in, d_out, graph, exec});
    }
    aeisu::check_hip(hipGraphLaunch(exec, (hipStream_t)stream), "hipGraphLaunch");
  });
}

int aeisu_controller_async(aeisu_runtime* h, const void* d_in, void* d_meta, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    if (!d_in || !d_meta) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null buffer");
    if (rt.mode == aeisu::kModeFp32)
      aeisu::fail(AEISU_ERR_STATE, "the FP32 policy has no FP16 coefficient stage; run the whole frame "
                                   "(aeisu_upscale*) or configure an FP16 or quantized policy");
    aeisu::enqueue_controller(*rt.w, rt.g, rt.scratch(), d_in, d_meta, (hipStream_t)stream, nullptr);
  });
}

int aeisu_head_async(aeisu_runtime* h, const void* d_in, const void* d_meta, void* d_out, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    if (!d_in || !d_meta || !d_out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null buffer");
    if (rt.mode == aeisu::kModeFp32)
      aeisu::fail(AEISU_ERR_STATE, "the FP32 policy has no FP16 coefficient stage; run the whole frame "
                                   "(aeisu_upscale*) or configure an FP16 or quantized policy");
    aeisu::enqueue_head(*rt.w, rt.g, rt.scratch(), d_in, d_meta, d_out, (hipStream_t)stream);
  });
}

size_t aeisu_intermediate_bytes(const aeisu_runtime* h, int which) {
  if (!h || !h->impl || !h->impl->configured) return 0;
  const Runtime& rt = *h->impl;
  const size_t packed = rt.g.packed(), lowpx = rt.g.lowpx();
  if (which == AEISU_BUF_SKIP || which == AEISU_BUF_WORK) return packed * 32 * rt.g.act_bytes;
  if (which == AEISU_BUF_META) return packed * 64 * rt.g.act_bytes;
  if (which >= AEISU_BUF_LOW0 && which <= AEISU_BUF_LOW4) return lowpx * 64 * rt.g.low_bytes;
  return 0;
}

int aeisu_copy_intermediate(aeisu_runtime* h, int which, void* d_dst, size_t bytes, void* stream) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    aeisu::require_configured(rt);
    const size_t need = aeisu_intermediate_bytes(h, which);
    if (need == 0 || bytes != need || !d_dst) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "bad intermediate id, size or pointer");
    const void* src = nullptr;
    if (which == AEISU_BUF_SKIP) {
      if (!rt.skip.ptr)
        aeisu::fail(AEISU_ERR_STATE, "the fused body recomputes the skip tensor on chip for this policy; configure "
                                     "with AEISU_FLAG_UNFUSED or AEISU_FLAG_KEEP_INTERMEDIATES to read it");
      src = rt.skip.ptr;
    }
    else if (which == AEISU_BUF_WORK) src = rt.work.ptr;
    else if (which == AEISU_BUF_META) {
      if (!rt.meta.ptr)
        aeisu::fail(AEISU_ERR_STATE, "the fused path keeps coefficients on chip; configure with "
                                     "AEISU_FLAG_UNFUSED or AEISU_FLAG_KEEP_INTERMEDIATES to read them");
      src = rt.meta.ptr;
    } else {
      const int li = which - AEISU_BUF_LOW0;
      if (rt.g.nlow == 0)
        aeisu::fail(AEISU_ERR_STATE, "the fused body keeps activations on chip; configure with "
                                     "AEISU_FLAG_UNFUSED or AEISU_FLAG_KEEP_INTERMEDIATES to read them");
      if (rt.g.nlow != 5 && li != 4) aeisu::fail(AEISU_ERR_STATE, "configure with AEISU_FLAG_KEEP_INTERMEDIATES to read this layer");
      src = rt.low[aeisu::low_slot(rt.g, li)].ptr;
    }
    aeisu::check_hip(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync");
  });
}

int aeisu_geometry(const aeisu_runtime* h, int out[6]) {
  return guarded([&] {
    if (!h || !h->impl || !out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null argument");
    const Runtime& rt = *h->impl;
    aeisu::require_configured(rt);
    const aeisu::Geometry& g = rt.g;
    out[0] = g.Hp; out[1] = g.Wp; out[2] = g.py; out[3] = g.px; out[4] = g.Hq; out[5] = g.Wq;
  });
}

int aeisu_stage_timings(aeisu_runtime* h, float ms[AEISU_STAGE_COUNT], int* frames) {
  return guarded([&] {
    Runtime& rt = runtime_of(h);
    if (!ms) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null output");
    double acc[AEISU_STAGE_COUNT] = {};
    // stage s spans events from[s] -> to[s]; on the fused path (one body kernel, one
    // refine + tail + head kernel) only events 0, 1, 3 and 6 are recorded, and 0, 3, 6 when the
    // fused body also computes the project from the frames
    static const int per_layer_from[6] = {0, 1, 2, 3, 4, 5}, per_layer_to[6] = {1, 2, 3, 4, 5, 6};
    static const int fused_from[6] = {0, -1, 1, -1, -1, 3}, fused_to[6] = {1, -1, 3, -1, -1, 6};
    static const int rgb_from[6] = {-1, -1, 0, -1, -1, 3}, rgb_to[6] = {-1, -1, 3, -1, -1, 6};
    const int* from = rt.g.fused_rgb ? rgb_from : rt.g.fused ? fused_from : per_layer_from;
    const int* to = rt.g.fused_rgb ? rgb_to : rt.g.fused ? fused_to : per_layer_to;
    for (int f = 0; f < rt.timed_frames; ++f) {
      hipEvent_t* e = &rt.events[size_t(f) * aeisu::kStageEvents];
      aeisu::check_hip(hipEventSynchronize(e[6]), "hipEventSynchronize");
      for (int s = 0; s < 6; ++s) {
        if (from[s] < 0) continue;
        float t = 0;
        aeisu::check_hip(hipEventElapsedTime(&t, e[from[s]], e[to[s]]), "hipEventElapsedTime");
        acc[s] += t;
      }
      float total = 0;
      aeisu::check_hip(hipEventElapsedTime(&total, e[0], e[6]), "hipEventElapsedTime");
      acc[AEISU_STAGE_TOTAL] += total;
    }
    for (int s = 0; s < AEISU_STAGE_COUNT; ++s) ms[s] = rt.timed_frames ? float(acc[s] / rt.timed_frames) : 0.f;
    if (frames) *frames = rt.timed_frames;
  });
}

int aeisu_reset_timings(aeisu_runtime* h) {
  return guarded([&] { runtime_of(h).timed_frames = 0; });
}

size_t aeisu_persistent_bytes(const aeisu_runtime* h) {
  if (!h || !h->impl) return 0;
  const Runtime& rt = *h->impl;
  return rt.model->bytes() + rt.scratch_bytes();
}

size_t aeisu_startup_report(const aeisu_runtime* h, char* out, size_t capacity) {
  if (!h || !h->impl || !h->impl->configured) return 0;
  const std::string& r = h->impl->report;
  if (out && capacity) {
    const size_t n = std::min(capacity - 1, r.size());
    std::memcpy(out, r.data(), n);
    out[n] = '\0';
  }
  return r.size() + 1;
}

int aeisu_artifact_checksum(const aeisu_runtime* h, char out[65]) {
  return guarded([&] {
    if (!h || !h->impl || !out) aeisu::fail(AEISU_ERR_INVALID_ARGUMENT, "null argument");
    std::snprintf(out, 65, "%s", h->impl->model->art.checksum_hex.c_str());
  });
}

void aeisu_destroy(aeisu_runtime* h) { delete h; }

const char* aeisu_last_error(void) { return g_last_error.c_str(); }

const char* aeisu_version(void) { return "aeisu_amd 0.2.0 (gfx950)"; }

}  // extern "C"
