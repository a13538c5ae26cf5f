// Instantiations of attn_fwd_kernel: additive score bias (reference HAS_BIAS).
#include "attn_kernel.h"

namespace tmx {

namespace {

template <int NW, int DP, int MODE, bool INT8V>
void launch_one(const AttnKArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<NW, DP, MODE, INT8V, false, true>), dim3(8 * a.per_xcd), dim3(NW * 64), 0,
                     stream, a);
}

template <int NW, int DP>
void by_mode(const AttnKArgs& a, int mode, bool int8v, hipStream_t stream) {
  if (mode == TILEMIX_ROUTING_FP16) {
    launch_one<NW, DP, TILEMIX_ROUTING_FP16, false>(a, stream);
  } else if (mode == TILEMIX_ROUTING_INT8) {
    if (int8v) launch_one<NW, DP, TILEMIX_ROUTING_INT8, true>(a, stream);
    else launch_one<NW, DP, TILEMIX_ROUTING_INT8, false>(a, stream);
  } else {
    if (int8v) launch_one<NW, DP, TILEMIX_ROUTING_MIXED, true>(a, stream);
    else launch_one<NW, DP, TILEMIX_ROUTING_MIXED, false>(a, stream);
  }
}

}  // namespace

void dispatch_attn_bias(const AttnKArgs& a, int nw, int dp, int mode, bool int8v, hipStream_t stream) {
  if (nw == 4) {
    if (dp == 128) by_mode<4, 128>(a, mode, int8v, stream);
    else by_mode<4, 64>(a, mode, int8v, stream);
  } else {
    if (dp == 128) by_mode<2, 128>(a, mode, int8v, stream);
    else by_mode<2, 64>(a, mode, int8v, stream);
  }
}

}  // namespace tmx
