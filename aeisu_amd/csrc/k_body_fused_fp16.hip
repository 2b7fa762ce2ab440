// Fused body of the FP16 policy (skip input, FP16 activations in LDS): its kernel instantiations,
// kept apart from the frame-input ones so that each translation unit gets its own instruction
// scheduler (the default here; LLVM's iterative ILP scheduler made this body 2 us slower at 1080p
// and the frame-input body 2 us faster).
#include "body_fused.hpp"

namespace aeisu {

hipError_t body_fused_prepare_fp16() {
  const void* fn[] = {body_kernel_ptr<0, 0, 16>(), body_kernel_ptr<0, 0, 8>(), body_pair_ptr<0, 0, 16, 8>()};
  const int lds[] = {BodyFusedCfg<0>::Lds, BodyFusedCfg<0, 8>::Lds, body_pair_lds<0, 0, 16, 8>()};
  for (int i = 0; i < 3; ++i) {
    const hipError_t r = hipFuncSetAttribute(fn[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds[i]);
    if (r != hipSuccess) return r;
  }
  return hipSuccess;
}

void launch_body_fused_fp16(const BodyFusedArgs& args, int tile, int tiles, hipStream_t stream) {
  if (tile == 16) launch_body_t<0, 0, 16>(args, tiles, stream);
  else launch_body_t<0, 0, 8>(args, tiles, stream);
}

void launch_body_fused_pair_fp16(const BodyFusedArgs& a1, int n1, const BodyFusedArgs& a2, int n2, hipStream_t stream) {
  launch_pair_t<0, 0, 16, 8>(a1, n1, a2, n2, stream);
}

}  // namespace aeisu
