// extern "C" entry points of libtilemix_hip.so (declared in include/tilemix_hip.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace tmx {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace tmx

extern "C" {

int tilemix_quant_per_block_int8(const tilemix_quant_params* p, void* stream) {
  if (p == nullptr) {
    tmx::set_error("tilemix_quant_per_block_int8: null params");
    return TILEMIX_E_INVALID;
  }
  return tmx::launch_quant(*p, static_cast<hipStream_t>(stream));
}

int tilemix_attn_fwd(const tilemix_attn_params* p, void* stream) {
  if (p == nullptr) {
    tmx::set_error("tilemix_attn_fwd: null params");
    return TILEMIX_E_INVALID;
  }
  return tmx::launch_attn(*p, nullptr, nullptr, 0, 0, static_cast<hipStream_t>(stream));
}

int tilemix_attn_fwd_debug(const tilemix_attn_params* p, int32_t* qk_i32, void* qk_f16,
                           int64_t dump_stride_token, int64_t dump_stride_head, void* stream) {
  if (p == nullptr) {
    tmx::set_error("tilemix_attn_fwd_debug: null params");
    return TILEMIX_E_INVALID;
  }
  if (qk_i32 == nullptr && qk_f16 == nullptr) {
    tmx::set_error("tilemix_attn_fwd_debug: both dump pointers are null");
    return TILEMIX_E_INVALID;
  }
  return tmx::launch_attn(*p, qk_i32, qk_f16, dump_stride_token, dump_stride_head,
                         static_cast<hipStream_t>(stream));
}

int tilemix_rms_norm_f16(const tilemix_rmsnorm_params* p, void* stream) {
  if (p == nullptr) {
    tmx::set_error("tilemix_rms_norm_f16: null params");
    return TILEMIX_E_INVALID;
  }
  return tmx::launch_rmsnorm(*p, static_cast<hipStream_t>(stream));
}

int tilemix_rotary_f16(const tilemix_rotary_params* p, void* stream) {
  if (p == nullptr) {
    tmx::set_error("tilemix_rotary_f16: null params");
    return TILEMIX_E_INVALID;
  }
  return tmx::launch_rotary(*p, static_cast<hipStream_t>(stream));
}

int tilemix_silu_mul_f16(const void* gate, const void* up, void* out, int64_t n, void* stream) {
  return tmx::launch_silu_mul(gate, up, out, n, static_cast<hipStream_t>(stream));
}

int tilemix_abi_version(void) { return TILEMIX_ABI_VERSION; }

int64_t tilemix_params_size(int which) {
  switch (which) {
    case 0:
      return (int64_t)sizeof(tilemix_quant_params);
    case 1:
      return (int64_t)sizeof(tilemix_attn_params);
    case 2:
      return (int64_t)sizeof(tilemix_rmsnorm_params);
    case 3:
      return (int64_t)sizeof(tilemix_rotary_params);
    default:
      return -1;
  }
}

const char* tilemix_last_error(void) { return tmx::g_last_error; }

}  // extern "C"
