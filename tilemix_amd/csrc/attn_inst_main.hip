// Instantiations of the attention kernels: the production variants (no bias, no dump).
#include "attn_launch.h"

namespace tmx {

void dispatch_attn_main(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
  AttnLauncher<false, false, false>::run(a, kind, dp, mode, int8v, stream);
}

}  // namespace tmx
