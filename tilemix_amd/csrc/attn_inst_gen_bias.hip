// Instantiations of the attention kernels, GEN variants: the same with an additive score bias.
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_gen_bias(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<false, true, true>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
