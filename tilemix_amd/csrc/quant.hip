// Per-block symmetric int8 quantisation (Q per BLKQ tokens, K per BLKK tokens).
//
// Follows quant_per_block_int8_kernel (attention/triton/quant_per_block_varlen.py:6-45):
//   x    = fp32(x) * sm_scale                      (:38-39)
//   s    = max|x| / 127.                           (:40, IEEE fp32 division)
//   t    = x / s ; t += 0.5 * (t >= 0 ? 1 : -1)    (:41-42)
//   code = int8(t)  (truncation)                   (:43)
// plus the host-side scale bookkeeping of per_block_int8_single (:55-63),
// done on the device so no device->host copy is needed to size the output.
//
// One workgroup owns one (block, head, sequence).  Blocks of up to
// kRegChunks * 256 eight-element chunks (BLK * D <= 16384: every Q/K block of
// the hot path) are read from HBM once and held in registers between the max
// pass and the code pass; larger blocks are streamed twice.
#include "attn_common.h"

namespace tmx {

namespace {

constexpr int kQuantThreads = 256;
constexpr int kRegChunks = 8;

struct QuantKArgs {
  const f16* in;
  int8_t* out;
  float* scale;
  f16* scale_half;
  const int32_t* cu;
  int32_t* cu_scale;
  int64_t si_t, si_h, so_t, so_h;
  int64_t capacity;
  float sm_scale;
  int heads, d, blk, batch;
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ void __launch_bounds__(kQuantThreads) quant_per_block_int8_kernel(const QuantKArgs a) {
  __shared__ float red_f[kQuantThreads / 64];
  __shared__ int red_i[kQuantThreads / 64];
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // Scale-row base of sequence b: sum over earlier sequences of ceil(L/blk).
  int part = 0;
  for (int bb = tid; bb < b; bb += kQuantThreads) {
    const int len = a.cu[bb + 1] - a.cu[bb];
    part += (len + a.blk - 1) / a.blk;
  }
  part = wave_sum_i(part);
  if (lane == 0) red_i[wave] = part;
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int w = 0; w < kQuantThreads / 64; ++w) base += red_i[w];

  const int start = a.cu[b];
  const int len = a.cu[b + 1] - start;
  if (blk == 0 && h == 0 && tid == 0 && a.cu_scale != nullptr) {
    a.cu_scale[b + 1] = base + (len + a.blk - 1) / a.blk;
    if (b == 0) a.cu_scale[0] = 0;
  }
  if (blk * a.blk >= len) return;

  const int rows = min(a.blk, len - blk * a.blk);
  const int cpr = a.d >> 3;  // 8-element chunks per row
  const int chunks = rows * cpr;
  const int64_t tok0 = (int64_t)start + (int64_t)blk * a.blk;
  const f16* in = a.in + tok0 * a.si_t + (int64_t)h * a.si_h;
  int8_t* out = a.out + tok0 * a.so_t + (int64_t)h * a.so_h;

  const float sm = a.sm_scale;
  // sm_scale == 1 (the hot path: quantize_q(k)_for_tilemix): the quotient is
  // taken from an IEEE reciprocal with one correction step, equal to the IEEE
  // division on the whole fp16 domain; other scales divide directly.
  const bool unit_scale = sm == 1.0f;
  auto encode = [&](const f16x8& x, float s, float rs, int r, int col) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = unit_scale ? div_by_recip((float)x[e], s, rs) : ((float)x[e] * sm) / s;
      t += (t >= 0.0f) ? 0.5f : -0.5f;
      // An all-zero block gives 0/0; its codes are defined as 0.
      const int code = (s == 0.0f) ? 0 : (int)t;
      const uint32_t byte = (uint32_t)(code & 0xff);
      if (e < 4) w0 |= byte << (8 * e);
      else w1 |= byte << (8 * (e - 4));
    }
    *reinterpret_cast<uint2*>(out + (int64_t)r * a.so_t + col) = make_uint2(w0, w1);
  };
  auto block_max = [&](float amax) {
    amax = wave_max(amax);
    if (lane == 0) red_f[wave] = amax;
    __syncthreads();
    amax = red_f[0];
#pragma unroll
    for (int w = 1; w < kQuantThreads / 64; ++w) amax = fmaxf(amax, red_f[w]);
    return amax;
  };

  float s;
  if (chunks <= kRegChunks * kQuantThreads) {
    f16x8 xs[kRegChunks];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kRegChunks; ++i) {
      const int c = tid + i * kQuantThreads;
      if (c < chunks) {
        const int r = c / cpr, col = (c - r * cpr) << 3;
        xs[i] = *reinterpret_cast<const f16x8*>(in + (int64_t)r * a.si_t + col);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)xs[i][e] * sm));
      }
    }
    s = block_max(amax) / 127.0f;  // IEEE division (no fast-math in this build)
    const float rs = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kRegChunks; ++i) {
      const int c = tid + i * kQuantThreads;
      if (c < chunks) {
        const int r = c / cpr, col = (c - r * cpr) << 3;
        encode(xs[i], s, rs, r, col);
      }
    }
  } else {
    float amax = 0.0f;
    for (int c = tid; c < chunks; c += kQuantThreads) {
      const int r = c / cpr, col = (c - r * cpr) << 3;
      const f16x8 x = *reinterpret_cast<const f16x8*>(in + (int64_t)r * a.si_t + col);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)x[e] * sm));
    }
    s = block_max(amax) / 127.0f;
    const float rs = 1.0f / s;
    for (int c = tid; c < chunks; c += kQuantThreads) {
      const int r = c / cpr, col = (c - r * cpr) << 3;
      encode(*reinterpret_cast<const f16x8*>(in + (int64_t)r * a.si_t + col), s, rs, r, col);
    }
  }
  if (tid == 0) {
    const int64_t row = (int64_t)base + blk;
    if (row < a.capacity) {
      a.scale[row * a.heads + h] = s;
      if (a.scale_half != nullptr) a.scale_half[row * a.heads + h] = (f16)s;
    }
  }
}

}  // namespace

int launch_quant(const tilemix_quant_params& p, hipStream_t stream) {
  if (!p.input || !p.output || !p.scale || !p.cu_seqlens) {
    set_error("tilemix_quant_per_block_int8: null tensor pointer");
    return TILEMIX_E_INVALID;
  }
  if (p.heads <= 0 || p.batch < 0 || p.blk_tokens <= 0 || p.max_seqlen < 0) {
    set_error("tilemix_quant_per_block_int8: invalid sizes (heads=%d batch=%d blk=%d max_seqlen=%d)",
              p.heads, p.batch, p.blk_tokens, p.max_seqlen);
    return TILEMIX_E_INVALID;
  }
  if (p.head_dim <= 0 || p.head_dim % 8 != 0 || p.head_dim > 256) {
    set_error("tilemix_quant_per_block_int8: head_dim must be a positive multiple of 8 <= 256, got %d",
              p.head_dim);
    return TILEMIX_E_INVALID;
  }
  if ((reinterpret_cast<uintptr_t>(p.input) & 15) || (p.stride_in_token & 7) || (p.stride_in_head & 7) ||
      (reinterpret_cast<uintptr_t>(p.output) & 7) || (p.stride_out_token & 7) || (p.stride_out_head & 7)) {
    set_error("tilemix_quant_per_block_int8: input must be 16-byte aligned with strides multiple of 8 "
              "elements; output 8-byte aligned with strides multiple of 8");
    return TILEMIX_E_INVALID;
  }
  if (p.batch == 0) return TILEMIX_OK;
  const int nblk = (p.max_seqlen + p.blk_tokens - 1) / p.blk_tokens;
  QuantKArgs a;
  a.in = static_cast<const f16*>(p.input);
  a.out = p.output;
  a.scale = p.scale;
  a.scale_half = static_cast<f16*>(p.scale_half);
  a.cu = p.cu_seqlens;
  a.cu_scale = p.cu_seqlens_scale;
  a.si_t = p.stride_in_token;
  a.si_h = p.stride_in_head;
  a.so_t = p.stride_out_token;
  a.so_h = p.stride_out_head;
  a.capacity = p.scale_rows_capacity;
  a.sm_scale = p.sm_scale;
  a.heads = p.heads;
  a.d = p.head_dim;
  a.blk = p.blk_tokens;
  a.batch = p.batch;
  // With no tokens, one block per sequence still publishes cu_seqlens_scale.
  dim3 grid(nblk > 0 ? nblk : 1, p.heads, p.batch);
  hipLaunchKernelGGL(quant_per_block_int8_kernel, grid, dim3(kQuantThreads), 0, stream, a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("tilemix_quant_per_block_int8: launch failed: %s", hipGetErrorString(err));
    return TILEMIX_E_LAUNCH;
  }
  return TILEMIX_OK;
}

}  // namespace tmx
