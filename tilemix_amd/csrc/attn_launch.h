// Kernel selection shared by the instantiation files (attn_inst_*.hip):
// block_m = 128 runs the 32-row kernel (4 waves x 32 rows), block_m = 64 the
// 16-row kernel (4 waves x 16 rows); head dims up to 64 use the 64-wide tile
// layout, larger ones the 128-wide one.
#pragma once

#include "attn_kernel16.h"
#include "attn_kernel32.h"

namespace tmx {

template <bool DUMP, bool BIAS>
struct AttnLauncher {
  template <int DP, int MODE, bool INT8V>
  static void one(const AttnKArgs& a, int block_m, hipStream_t stream) {
    if (block_m == 128)
      hipLaunchKernelGGL((attn32_kernel<4, DP, MODE, INT8V, DUMP, BIAS>), dim3(8 * a.per_xcd), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn16_kernel<4, DP, MODE, INT8V, DUMP, BIAS>), dim3(8 * a.per_xcd), dim3(256), 0, stream, a);
  }

  template <int DP>
  static void by_mode(const AttnKArgs& a, int block_m, int mode, bool int8v, hipStream_t stream) {
    // The debug dump has no int8-V variant (rejected on the host).
    constexpr bool kInt8V = !DUMP;
    if (mode == TILEMIX_ROUTING_FP16) {
      one<DP, TILEMIX_ROUTING_FP16, false>(a, block_m, stream);
    } else if (mode == TILEMIX_ROUTING_INT8) {
      if (kInt8V && int8v) one<DP, TILEMIX_ROUTING_INT8, kInt8V>(a, block_m, stream);
      else one<DP, TILEMIX_ROUTING_INT8, false>(a, block_m, stream);
    } else {
      if (kInt8V && int8v) one<DP, TILEMIX_ROUTING_MIXED, kInt8V>(a, block_m, stream);
      else one<DP, TILEMIX_ROUTING_MIXED, false>(a, block_m, stream);
    }
  }

  static void run(const AttnKArgs& a, int block_m, int dp, int mode, bool int8v, hipStream_t stream) {
    if (dp == 128) by_mode<128>(a, block_m, mode, int8v, stream);
    else by_mode<64>(a, block_m, mode, int8v, stream);
  }
};

}  // namespace tmx
