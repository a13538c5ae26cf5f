// Instantiations of the attention kernels: score dump of tilemix_attn_fwd_debug.
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_dump(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<true, false, false>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
