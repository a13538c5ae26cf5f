// Instantiations of the attention kernels, GEN variants: block_n 128/256 or K/V scale blocks not a multiple of 64.
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_gen_main(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<false, false, true>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
