// Mutation fuzzing of the SPYR8F8 parser and weight packer through aeisu_create_from_memory.
// Built by tests/test_fuzz_cpu.py with the library's host code under AddressSanitizer and
// UndefinedBehaviorSanitizer; on a machine without a GPU a mutant that passes every check stops at
// the first HIP call (AEISU_ERR_HIP), so only the host-side validation runs.  Mutants: bit flips
// (mostly in the header and tensor table), boundary values written into 4- and 8-byte fields,
// truncation, extension, and NaN/Inf/extreme values written into the payload; four in five get a
// recomputed SHA-256 (offset 184, computed with its own 32 bytes zeroed, SrcPyrModel.cpp:37-81) so
// that they reach the checks behind the checksum.
// Usage: fuzz_artifact FILE PRECISION ITERATIONS SEED
#include "aeisu_amd.h"
#include "sha256.hpp"
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <random>
#include <string>
#include <vector>

static std::vector<uint8_t> read_file(const char* p) {
  std::ifstream f(p, std::ios::binary);
  return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}
static void fix_sha(std::vector<uint8_t>& b) {
  if (b.size() < 216) return;
  std::memset(b.data() + 184, 0, 32);
  aeisu::Sha256 h;
  h.update(b.data(), b.size());
  auto d = h.finish();
  std::memcpy(b.data() + 184, d.data(), 32);
}
int main(int argc, char** argv) {
  if (argc < 5) { std::fprintf(stderr, "fuzz_artifact FILE PRECISION ITERATIONS SEED\n"); return 2; }
  const auto base = read_file(argv[1]);
  const int precision = std::atoi(argv[2]);
  const long iters = std::atol(argv[3]);
  std::mt19937_64 rng(std::strtoull(argv[4], nullptr, 10));
  std::map<int, long> hist;
  std::map<std::string, long> msgs;
  {
    aeisu_runtime* rt = nullptr;
    const int rc = aeisu_create_from_memory(base.data(), base.size(), precision, &rt);
    std::printf("unmutated: rc %d (%s)\n", rc, aeisu_last_error());
    if (rt) aeisu_destroy(rt);
  }
  for (long it = 0; it < iters; ++it) {
    auto b = base;
    const int kind = int(rng() % 7);
    const size_t hot = std::min<size_t>(b.size(), 512 + 80 * 64);   // header + TOC region
    if (kind <= 2) {                         // bit flips, mostly in the header/TOC
      const int nflip = 1 + int(rng() % 8);
      for (int k = 0; k < nflip; ++k) {
        const size_t pos = (rng() % 4 != 0) ? rng() % hot : rng() % b.size();
        b[pos] ^= uint8_t(1u << (rng() % 8));
      }
    } else if (kind == 3) {                  // boundary values into a 4- or 8-byte field
      static const uint64_t vals[] = {0, 1, 0xFFFFFFFFull, 0x7FFFFFFFull, 0x80000000ull, 0xFFFFFFFFFFFFFFFFull,
                                      0x7FFFFFFFFFFFFFFFull, 64, 512, 4096};
      const uint64_t v = (rng() % 3 == 0) ? uint64_t(b.size() + (rng() % 3) - 1) : vals[rng() % 10];
      const size_t pos = (rng() % hot) & ~size_t(3);
      const size_t w = (rng() % 2) ? 4 : 8;
      if (pos + w <= b.size()) std::memcpy(b.data() + pos, &v, w);
    } else if (kind == 4) {                  // truncation
      b.resize(rng() % b.size());
    } else if (kind == 5) {                  // extension
      const size_t add = 1 + rng() % 4096;
      for (size_t k = 0; k < add; ++k) b.push_back(uint8_t(rng()));
    } else {                                 // random float garbage into the payload (NaN/Inf/huge)
      static const uint32_t fv[] = {0x7FC00000u, 0x7F800000u, 0xFF800000u, 0x7F7FFFFFu, 0x00000001u, 0x80000000u};
      const int n = 1 + int(rng() % 16);
      for (int k = 0; k < n && b.size() > hot + 4; ++k) {
        const size_t pos = hot + ((rng() % (b.size() - hot - 4)) & ~size_t(1));
        const uint32_t v = fv[rng() % 6];
        if (rng() % 2) std::memcpy(b.data() + pos, &v, 4);
        else { const uint16_t h = uint16_t(rng() % 2 ? 0x7E00 : 0x7C00); std::memcpy(b.data() + pos, &h, 2); }
      }
    }
    if (rng() % 5 != 0) fix_sha(b);          // most mutants get a valid checksum, to reach deeper checks
    aeisu_runtime* rt = nullptr;
    const int rc = aeisu_create_from_memory(b.data(), b.size(), precision, &rt);
    if (rt) aeisu_destroy(rt);
    hist[rc]++;
    std::string m = aeisu_last_error();
    if (m.size() > 60) m.resize(60);
    msgs[m]++;
  }
  for (auto& [rc, n] : hist) std::printf("rc %d: %ld\n", rc, n);
  int shown = 0;
  for (auto& [m, n] : msgs) if (shown++ < 60) std::printf("  %6ld  %s\n", n, m.c_str());
  return 0;
}
