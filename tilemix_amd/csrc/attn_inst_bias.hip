// Instantiations of the attention kernels: additive score bias (reference HAS_BIAS).
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_bias(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<false, true, false>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
