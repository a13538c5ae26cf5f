// Kernel selection shared by the instantiation files (attn_inst_*.hip).
// Head dims up to 64 use the 64-wide tile layout, larger ones the 128-wide one.
#pragma once

#include "attn_kernel16.h"
#include "attn_kernel32.h"

namespace tmx {

template <bool DUMP, bool BIAS, bool GEN>
struct AttnLauncher {
  template <int DP, int MODE, bool INT8V>
  static void one(const AttnKArgs& a, int kind, hipStream_t stream) {
    const dim3 grid(8 * a.per_xcd), block(256);
    if constexpr (MODE == TILEMIX_ROUTING_MIXED && INT8V) {
      if (kind == kAttn16) {
        hipLaunchKernelGGL((attn16_kernel<4, DP, MODE, INT8V, DUMP, BIAS, GEN>), grid, block, 0, stream, a);
        return;
      }
    }
    if constexpr (MODE == TILEMIX_ROUTING_MIXED && !INT8V) {
      if (kind == kAttn32Split) {
        if constexpr (DP == 128 && !DUMP && !BIAS && !GEN) {
          if (a.pipe) {
            hipLaunchKernelGGL((attn32_kernel<4, DP, MODE, INT8V, DUMP, BIAS, true, GEN, true>), grid, block, 0,
                               stream, a);
            return;
          }
        }
        hipLaunchKernelGGL((attn32_kernel<4, DP, MODE, INT8V, DUMP, BIAS, true, GEN>), grid, block, 0, stream, a);
        return;
      }
    }
    if constexpr (DP == 128 && !INT8V && !DUMP && !BIAS && !GEN) {
      if (a.pipe) {
        hipLaunchKernelGGL((attn32_kernel<4, DP, MODE, INT8V, DUMP, BIAS, false, GEN, true>), grid, block, 0, stream,
                           a);
        return;
      }
    }
    hipLaunchKernelGGL((attn32_kernel<4, DP, MODE, INT8V, DUMP, BIAS, false, GEN>), grid, block, 0, stream, a);
  }

  template <int DP>
  static void by_mode(const AttnKArgs& a, int kind, int mode, bool int8v, hipStream_t stream) {
    // The debug dump has no int8-V variant (rejected on the host).
    constexpr bool kInt8V = !DUMP;
    if (mode == TILEMIX_ROUTING_FP16) {
      one<DP, TILEMIX_ROUTING_FP16, false>(a, kind, stream);
    } else if (mode == TILEMIX_ROUTING_INT8) {
      if (kInt8V && int8v) one<DP, TILEMIX_ROUTING_INT8, kInt8V>(a, kind, stream);
      else one<DP, TILEMIX_ROUTING_INT8, false>(a, kind, stream);
    } else {
      if (kInt8V && int8v) one<DP, TILEMIX_ROUTING_MIXED, kInt8V>(a, kind, stream);
      else one<DP, TILEMIX_ROUTING_MIXED, false>(a, kind, stream);
    }
  }

  static void run(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream) {
    if (dp == 128) by_mode<128>(a, kind, mode, int8v, stream);
    else by_mode<64>(a, kind, mode, int8v, stream);
  }
};

}  // namespace tmx
