// Instantiations of the attention kernels, GEN variants: the same with the score dump of tilemix_attn_fwd_debug.
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_gen_dump(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<true, false, true>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
