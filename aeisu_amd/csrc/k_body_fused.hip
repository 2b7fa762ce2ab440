// Fused body, host side: tile plans, LDS attributes and launches of the frame-input kernels
// (Mixed, FP8-MFMA, INT8 policies).  The kernels are in body_fused.hpp; the FP16 policy's
// skip-input kernels are instantiated in k_body_fused_fp16.hip.
#include "body_fused.hpp"

namespace aeisu {

// ------------------------------------------------------------------------------------------------
int body_fused_num_tiles(int mode, int batch, int Hl, int Wl, int tile) {
  const int T = tile ? tile : (mode == 0 ? BodyFusedCfg<0>::T : BodyFusedCfg<3>::T);
  return batch * ((Hl + T - 1) / T) * ((Wl + T - 1) / T);
}

// Time to run n1 blocks of cost c1 and then n2 blocks of cost c2 in one launch: the hardware hands
// block g to XCD g % 8, and each XCD starts its next block on its first free CU (cus / 8 each).
static double pair_makespan(long n1, double c1, long n2, double c2, int cus) {
  const int per = cus / 8 > 0 ? cus / 8 : 1;
  std::vector<double> busy(per);
  double worst = 0.0;
  for (int x = 0; x < 8; ++x) {
    std::fill(busy.begin(), busy.end(), 0.0);
    for (long g = x; g < n1 + n2; g += 8) *std::min_element(busy.begin(), busy.end()) += g < n1 ? c1 : c2;
    worst = std::max(worst, *std::max_element(busy.begin(), busy.end()));
  }
  return worst;
}

// Frame-input tiles: a block computes one tile, and a 16x16 tile costs about 0.6 of a 24x24 one
// (its compress region is 24^2 against 32^2 pixels, the bottleneck and expand regions shrink
// alike).  Two tile sides run in one launch (body_fused_pair_kernel), and the plan with the
// shortest simulated schedule is taken (ties, within 1 %, keep more 24x24 tiles):
//  * frames: the leading frames on 24x24 tiles, the rest on 16x16 tiles.  Small frames at batch 1
//    take 16x16 tiles, 1080p and larger 24x24 ones.
//  * columns: every frame's low columns [0, C) on 24x24 tiles (C a multiple of 24), the rest on
//    16x16 tiles.  Where a frame's last 24-wide tile column is mostly past the frame (540p: 248
//    low columns, 8 in the eleventh tile column), 16x16 tiles cover it for less, and a batch that
//    needed a third round of 24x24 tiles (540p x 8: 528 tiles on 256 CUs) fits in about two.
static BodyPlan plan_with_cost(int mode, int batch, int Hl, int Wl, int cus, double& best) {
  BodyPlan best_plan{batch, 0};
  best = pair_makespan(body_fused_num_tiles(mode, batch, Hl, Wl, 24), 1.0, 0, 0.0, cus);
  if (mode == 0 || cus <= 0) return best_plan;
  const long t24 = body_fused_num_tiles(mode, 1, Hl, Wl, 24), t16 = body_fused_num_tiles(mode, 1, Hl, Wl, 16);
  best = -1.0;
  for (int k = batch; k >= 0; --k) {
    const double cost = pair_makespan(t24 * k, 1.0, t16 * (batch - k), 0.6, cus);
    if (best < 0.0 || cost < 0.99 * best) {
      best = cost;
      best_plan = BodyPlan{k, 0};
    }
  }
  for (int c = (Wl - 1) / 24 * 24; c >= 24; c -= 24) {
    const long n24 = (long)batch * body_fused_num_tiles(mode, 1, Hl, c, 24);
    const long n16 = (long)batch * body_fused_num_tiles(mode, 1, Hl, Wl - c, 16);
    const double cost = pair_makespan(n24, 1.0, n16, 0.6, cus);
    if (cost < 0.99 * best) {
      best = cost;
      best_plan = BodyPlan{batch, c};
    }
  }
  return best_plan;
}
BodyPlan body_fused_plan(int mode, int batch, int Hl, int Wl, int cus) {
  double cost;
  return plan_with_cost(mode, batch, Hl, Wl, cus, cost);
}

// Compress exchange in launches of whole frames on 24x24 tiles, for batches whose tiles outnumber
// the CUs: each launch's tiles all fit on the device at once, so a launch takes about one tile's
// time, and a tile with the exchange takes kGain of one without it (measured, bench events: Mixed
// 1080p 65.8 -> 61.6 us; INT8 none left once its compress got cheaper, 1080p x 2 104.0 against
// 105.8 us with the exchange).  Taken where the launches beat body_fused_plan's simulated schedule
// without the exchange (in 24x24 tile units), or with tile24_only, the single 24x24 launch.
BodyXcPlan body_fused_xc_plan(int mode, int batch, int Hl, int Wl, int cus, bool tile24_only) {
  const double kGain = mode == 3 ? 0.94 : 1.0;
  BodyXcPlan none{0, 0};
  if (mode == 0 || cus <= 0) return none;
  double base;
  if (tile24_only) base = pair_makespan(body_fused_num_tiles(mode, batch, Hl, Wl, 24), 1.0, 0, 0.0, cus);
  else plan_with_cost(mode, batch, Hl, Wl, cus, base);
  const int frames = std::min(batch, cus / body_fused_num_tiles(mode, 1, Hl, Wl, 24));
  if (frames < 1) return none;
  const int launches = (batch + frames - 1) / frames;
  return launches * kGain < 0.99 * base ? BodyXcPlan{24, frames} : none;
}

// FP16 policy: the same trade between 16x16 tiles and 8x8 tiles (compress region 16^2 against
// 24^2 pixels plus the fixed per-tile prologue: about half the cost), split by low rows since the
// batch is usually one frame: rows [0, R) on 16x16 tiles, the rest on 8x8 tiles, in one launch.
int body_fused_row_split(int mode, int batch, int Hl, int Wl, int cus) {
  if (mode != 0 || cus <= 0) return Hl;
  const int top = (Hl + 15) / 16 * 16;
  double best = -1.0;
  int best_r = top;
  for (int r = top; r >= 0; r -= 16) {            // ties (within 1 %) keep more rows on 16x16 tiles
    const long t16 = (long)batch * ((std::min(r, Hl) + 15) / 16) * ((Wl + 15) / 16);
    const long t8 = r >= Hl ? 0 : (long)batch * ((Hl - r + 7) / 8) * ((Wl + 7) / 8);
    const double cost = pair_makespan(t16, 1.0, t8, 0.5, cus);
    if (best < 0.0 || cost < 0.99 * best) {
      best = cost;
      best_r = r;
    }
  }
  return best_r >= Hl ? Hl : best_r;
}


hipError_t body_fused_prepare() {
  struct K {
    const void* fn;
    int lds;
  };
  const K k[] = {
      {body_kernel_ptr<1, 1, 24>(), BodyFusedCfg<1, 24>::LdsRgb}, {body_kernel_ptr<1, 2, 24>(), BodyFusedCfg<1, 24>::LdsRgb},
      {body_kernel_ptr<2, 1, 24>(), BodyFusedCfg<2, 24>::LdsRgb}, {body_kernel_ptr<2, 2, 24>(), BodyFusedCfg<2, 24>::LdsRgb},
      {body_kernel_ptr<3, 1, 24>(), BodyFusedCfg<3, 24>::LdsRgb}, {body_kernel_ptr<3, 2, 24>(), BodyFusedCfg<3, 24>::LdsRgb},
      {body_kernel_ptr<1, 1, 16>(), BodyFusedCfg<1, 16>::LdsRgb}, {body_kernel_ptr<1, 2, 16>(), BodyFusedCfg<1, 16>::LdsRgb},
      {body_kernel_ptr<2, 1, 16>(), BodyFusedCfg<2, 16>::LdsRgb}, {body_kernel_ptr<2, 2, 16>(), BodyFusedCfg<2, 16>::LdsRgb},
      {body_kernel_ptr<3, 1, 16>(), BodyFusedCfg<3, 16>::LdsRgb}, {body_kernel_ptr<3, 2, 16>(), BodyFusedCfg<3, 16>::LdsRgb},
      {body_pair_ptr<1, 1, 24, 16>(), body_pair_lds<1, 1, 24, 16>()}, {body_pair_ptr<1, 2, 24, 16>(), body_pair_lds<1, 2, 24, 16>()},
      {body_pair_ptr<2, 1, 24, 16>(), body_pair_lds<2, 1, 24, 16>()}, {body_pair_ptr<2, 2, 24, 16>(), body_pair_lds<2, 2, 24, 16>()},
      {body_pair_ptr<3, 1, 24, 16>(), body_pair_lds<3, 1, 24, 16>()}, {body_pair_ptr<3, 2, 24, 16>(), body_pair_lds<3, 2, 24, 16>()},
      {body_xc_ptr<1, 1, 24>(), BodyFusedCfg<1, 24>::LdsRgb}, {body_xc_ptr<1, 2, 24>(), BodyFusedCfg<1, 24>::LdsRgb},
      {body_xc_ptr<2, 1, 24>(), BodyFusedCfg<2, 24>::LdsRgb}, {body_xc_ptr<2, 2, 24>(), BodyFusedCfg<2, 24>::LdsRgb},
      {body_xc_ptr<3, 1, 24>(), BodyFusedCfg<3, 24>::LdsRgb}, {body_xc_ptr<3, 2, 24>(), BodyFusedCfg<3, 24>::LdsRgb},
      {body_xc_ptr<1, 1, 16>(), BodyFusedCfg<1, 16>::LdsRgb}, {body_xc_ptr<1, 2, 16>(), BodyFusedCfg<1, 16>::LdsRgb},
      {body_xc_ptr<2, 1, 16>(), BodyFusedCfg<2, 16>::LdsRgb}, {body_xc_ptr<2, 2, 16>(), BodyFusedCfg<2, 16>::LdsRgb},
      {body_xc_ptr<3, 1, 16>(), BodyFusedCfg<3, 16>::LdsRgb}, {body_xc_ptr<3, 2, 16>(), BodyFusedCfg<3, 16>::LdsRgb}};
  for (const K& e : k) {
    const hipError_t r = hipFuncSetAttribute(e.fn, hipFuncAttributeMaxDynamicSharedMemorySize, e.lds);
    if (r != hipSuccess) return r;
  }
  return body_fused_prepare_fp16();
}

template <int MODE>
static void launch_body_m(BodySrc src, const BodyFusedArgs& args, int tile, int tiles, hipStream_t stream) {
  switch (src) {
    case BodySrc::Frames16:
      if (tile == 16) launch_body_t<MODE, 1, 16>(args, tiles, stream);
      else launch_body_t<MODE, 1, 24>(args, tiles, stream);
      break;
    default:
      if (tile == 16) launch_body_t<MODE, 2, 16>(args, tiles, stream);
      else launch_body_t<MODE, 2, 24>(args, tiles, stream);
      break;
  }
}

hipError_t launch_body_fused(int mode, BodySrc src, const BodyFusedArgs& args, int batch, int tile,
                             hipStream_t stream) {
  const int rows = args.rows ? args.rows : args.Hl, cols = args.cols ? args.cols : args.Wl;
  if (args.row0 < 0 || rows < 1 || args.row0 + rows > args.Hl) return hipErrorInvalidValue;
  if (args.col0 < 0 || cols < 1 || args.col0 + cols > args.Wl) return hipErrorInvalidValue;
  if (mode == 0) {
    // FP16 policy: skip input only (its FP16 hi/lo project operands need twice the feature slice)
    if (tile == 0) tile = 16;
    if (src != BodySrc::Skip || (tile != 16 && tile != 8)) return hipErrorInvalidValue;
    launch_body_fused_fp16(args, tile, body_fused_num_tiles(0, batch, rows, cols, tile), stream);
    return hipGetLastError();
  }
  // quantized policies: frame input only (the engine runs their skip-input layers per layer)
  if (tile == 0) tile = 24;
  if (src == BodySrc::Skip || (tile != 24 && tile != 16)) return hipErrorInvalidValue;
  const int tiles = body_fused_num_tiles(mode, batch, rows, cols, tile);
  switch (mode) {
    case 1: launch_body_m<1>(src, args, tile, tiles, stream); break;
    case 2: launch_body_m<2>(src, args, tile, tiles, stream); break;
    default: launch_body_m<3>(src, args, tile, tiles, stream); break;
  }
  return hipGetLastError();
}

template <int MODE, int SRC, int TT>
static void launch_xc_t(const BodyFusedArgs& args, int tiles, hipStream_t stream) {
  typedef BodyFusedCfg<MODE, TT> C;
  constexpr int lds = C::LdsRgb;
  hipLaunchKernelGGL((body_fused_xc_kernel<MODE, SRC, TT>), dim3(tiles), dim3(C::Threads), lds, stream, args);
}
template <int MODE>
static void launch_xc_m(BodySrc src, const BodyFusedArgs& args, int tile, int tiles, hipStream_t stream) {
  if (src == BodySrc::Frames16) {
    if (tile == 16) launch_xc_t<MODE, 1, 16>(args, tiles, stream);
    else launch_xc_t<MODE, 1, 24>(args, tiles, stream);
  } else {
    if (tile == 16) launch_xc_t<MODE, 2, 16>(args, tiles, stream);
    else launch_xc_t<MODE, 2, 24>(args, tiles, stream);
  }
}

hipError_t launch_body_fused_xc(int mode, BodySrc src, const BodyFusedArgs& args, int batch, int tile, int cus,
                                hipStream_t stream) {
  // whole frames only, every tile resident at once (the LDS admits one block per CU)
  if (mode == 0 || src == BodySrc::Skip || (tile != 24 && tile != 16)) return hipErrorInvalidValue;
  if (args.row0 || args.rows || args.col0 || args.cols || !args.xbuf || !args.xflags)
    return hipErrorInvalidValue;
  const int tiles = body_fused_num_tiles(mode, batch, args.Hl, args.Wl, tile);
  if (tiles > cus) return hipErrorInvalidValue;
  switch (mode) {
    case 1: launch_xc_m<1>(src, args, tile, tiles, stream); break;
    case 2: launch_xc_m<2>(src, args, tile, tiles, stream); break;
    default: launch_xc_m<3>(src, args, tile, tiles, stream); break;
  }
  return hipGetLastError();
}

template <int MODE>
static void launch_pair_m(BodySrc src, const BodyFusedArgs& a1, int n1, const BodyFusedArgs& a2, int n2,
                          hipStream_t stream) {
  if (src == BodySrc::Frames16) launch_pair_t<MODE, 1, 24, 16>(a1, n1, a2, n2, stream);
  else launch_pair_t<MODE, 2, 24, 16>(a1, n1, a2, n2, stream);
}

hipError_t launch_body_fused_pair(int mode, BodySrc src, const BodyFusedArgs& a1, int batch1, int tile1,
                                  const BodyFusedArgs& a2, int batch2, int tile2, hipStream_t stream) {
  for (const BodyFusedArgs* a : {&a1, &a2}) {
    const int rows = a->rows ? a->rows : a->Hl, cols = a->cols ? a->cols : a->Wl;
    if (a->row0 < 0 || rows < 1 || a->row0 + rows > a->Hl) return hipErrorInvalidValue;
    if (a->col0 < 0 || cols < 1 || a->col0 + cols > a->Wl) return hipErrorInvalidValue;
  }
  auto rows_of = [](const BodyFusedArgs& a) { return a.rows ? a.rows : a.Hl; };
  auto cols_of = [](const BodyFusedArgs& a) { return a.cols ? a.cols : a.Wl; };
  if (batch1 < 1 || batch2 < 1) return hipErrorInvalidValue;
  if (mode == 0) {
    if (src != BodySrc::Skip || tile1 != 16 || tile2 != 8) return hipErrorInvalidValue;
    const int n1 = body_fused_num_tiles(0, batch1, rows_of(a1), cols_of(a1), 16);
    const int n2 = body_fused_num_tiles(0, batch2, rows_of(a2), cols_of(a2), 8);
    launch_body_fused_pair_fp16(a1, n1, a2, n2, stream);
    return hipGetLastError();
  }
  if (src == BodySrc::Skip || tile1 != 24 || tile2 != 16) return hipErrorInvalidValue;
  const int n1 = body_fused_num_tiles(mode, batch1, rows_of(a1), cols_of(a1), 24);
  const int n2 = body_fused_num_tiles(mode, batch2, rows_of(a2), cols_of(a2), 16);
  switch (mode) {
    case 1: launch_pair_m<1>(src, a1, n1, a2, n2, stream); break;
    case 2: launch_pair_m<2>(src, a1, n1, a2, n2, stream); break;
    default: launch_pair_m<3>(src, a1, n1, a2, n2, stream); break;
  }
  return hipGetLastError();
}

}  // namespace aeisu
