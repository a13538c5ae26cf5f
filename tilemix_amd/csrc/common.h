// Shared device/host helpers of libtilemix_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tilemix_hip.h"

namespace tmx {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// log2(e) rounded to fp32, the constant the reference multiplies sm_scale by
// (attention/triton/tilemix.py:16,641).
constexpr float kLog2eF32 = 1.4426950408889634f;

// Record an error message for tilemix_last_error() (thread-local).
void set_error(const char* fmt, ...);

int launch_quant(const tilemix_quant_params& p, hipStream_t stream);
int launch_attn(const tilemix_attn_params& p, int32_t* dump_i32, void* dump_f16,
                int64_t dump_t, int64_t dump_h, hipStream_t stream);
int launch_rmsnorm(const tilemix_rmsnorm_params& p, hipStream_t stream);
int launch_rotary(const tilemix_rotary_params& p, hipStream_t stream);
int launch_silu_mul(const void* gate, const void* up, void* out, int64_t n, hipStream_t stream);

// Exchange a value between lane l and lane l^32 of a wave64 and combine:
// returns {value of this lane, value of the partner lane} as (lo, hi) pair
// such that op(lo, hi) is bitwise identical on both lanes for commutative op.
__device__ __forceinline__ float2 swap_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

}  // namespace tmx
