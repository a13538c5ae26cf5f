// Prefill helper kernels of the LLaMA glue: RMSNorm, token-major split-half
// rotary embedding of Q and K, SiLU(gate) * up.  All three are HBM-streaming
// kernels (one read of every input, one write of every output, 16-byte
// accesses); the formulas follow models/tilemix_llama.py:718-869.
#include "common.h"

#include <math.h>

namespace tmx {

namespace {

// Materialise an fp32 result before its conversion to fp16: the reference
// rounds to fp32 and then to fp16, which the compiler would otherwise fuse
// into one mixed-precision instruction (a single rounding).  Products of two
// fp16 values are exact in fp32 and need no barrier.
__device__ __forceinline__ float keep32(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// ---- RMSNorm (reference :718-797) ------------------------------------------
// The sum of squares adds separately rounded products (the reference's
// reduction is built without FMA contraction), in this kernel's own order.
// One wave per row; rows of up to kNormChunks * 64 eight-element chunks
// (cols <= 8192) stay in registers between the sum of squares and the output
// pass, longer rows are read twice.
constexpr int kNormWaves = 4;
constexpr int kNormChunks = 16;

struct NormArgs {
  const f16* x;
  const f16* w;
  f16* out;
  int64_t rows, sx, so;
  int cols;
  float inv_cols, eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ f16 norm_one(float x, float rs, f16 w) {
  const f16 hn = (f16)keep32(x * rs);        // fp16(fp32(x) * rsqrt(var + eps))
  return (f16)((float)w * (float)hn);        // fp16(fp32(w) * fp32(hn))
}

__global__ void __launch_bounds__(kNormWaves * 64) rmsnorm_kernel(const NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const f16* xr = a.x + row * a.sx;
  f16* orow = a.out + row * a.so;
  const int chunks = a.cols >> 3;          // full 8-element chunks
  const int tail0 = chunks << 3;           // first element of the ragged tail
  const bool vec = ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(orow) |
                     reinterpret_cast<uintptr_t>(a.w)) & 15) == 0;
  float ss = 0.0f;
  if (vec && chunks <= kNormChunks * 64) {
    f16x8 xv[kNormChunks];
#pragma unroll
    for (int i = 0; i < kNormChunks; ++i) {
      const int c = i * 64 + lane;
      if (c < chunks) {
        xv[i] = *reinterpret_cast<const f16x8*>(xr + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)xv[i][e] * (float)xv[i][e];
      }
    }
    for (int c = tail0 + lane; c < a.cols; c += 64) ss += (float)xr[c] * (float)xr[c];
    const float var = wave_sum(ss) * a.inv_cols;
    const float rs = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int i = 0; i < kNormChunks; ++i) {
      const int c = i * 64 + lane;
      if (c < chunks) {
        const f16x8 wv = *reinterpret_cast<const f16x8*>(a.w + c * 8);
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = norm_one((float)xv[i][e], rs, wv[e]);
        *reinterpret_cast<f16x8*>(orow + c * 8) = o;
      }
    }
    for (int c = tail0 + lane; c < a.cols; c += 64) orow[c] = norm_one((float)xr[c], rs, a.w[c]);
  } else {
    for (int c = lane; c < a.cols; c += 64) ss += (float)xr[c] * (float)xr[c];
    const float var = wave_sum(ss) * a.inv_cols;
    const float rs = 1.0f / sqrtf(var + a.eps);
    for (int c = lane; c < a.cols; c += 64) orow[c] = norm_one((float)xr[c], rs, a.w[c]);
  }
}

// ---- rotary (reference :808-847) -------------------------------------------
// One thread per 8-element chunk of one (b, t, h) row; the partner chunk at
// d' = (d + D/2) % D is loaded directly.  Output rows are token-major.
struct RotaryArgs {
  const f16* q;
  const f16* k;
  const f16* cs;
  const f16* sn;
  f16* oq;
  f16* ok;
  int64_t qz, qh, qt, kz, kh, kt, cz, ct, sz, st;
  int64_t rows;  // batch * tokens * (hq + hk)
  int t, hq, hk, d;
};

__device__ __forceinline__ f16 rope_one(float x, float xr, float c, float s, float sign) {
  const f16 a = (f16)(x * c);
  const f16 b = (f16)((xr * sign) * s);
  return (f16)keep32((float)a + (float)b);
}

__global__ void __launch_bounds__(256) rotary_kernel(const RotaryArgs a) {
  const int cpr = a.d >> 3;  // chunks per row (d % 16 == 0 on this path)
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= a.rows * cpr) return;
  const int ch = (int)(gid % cpr);
  int64_t r = gid / cpr;
  const int H = a.hq + a.hk;
  const int h = (int)(r % H);
  r /= H;
  const int t = (int)(r % a.t);
  const int64_t b = r / a.t;
  const int d0 = ch * 8;
  const int half = a.d >> 1;
  const int dr = d0 < half ? d0 + half : d0 - half;
  const float sign = d0 < half ? -1.0f : 1.0f;
  const f16* src;
  f16* dst;
  if (h < a.hq) {
    src = a.q + b * a.qz + (int64_t)h * a.qh + (int64_t)t * a.qt;
    dst = a.oq + ((b * a.t + t) * a.hq + h) * a.d;
  } else {
    src = a.k + b * a.kz + (int64_t)(h - a.hq) * a.kh + (int64_t)t * a.kt;
    dst = a.ok + ((b * a.t + t) * a.hk + (h - a.hq)) * a.d;
  }
  const f16x8 x = *reinterpret_cast<const f16x8*>(src + d0);
  const f16x8 xr = *reinterpret_cast<const f16x8*>(src + dr);
  const f16x8 c = *reinterpret_cast<const f16x8*>(a.cs + b * a.cz + (int64_t)t * a.ct + d0);
  const f16x8 s = *reinterpret_cast<const f16x8*>(a.sn + b * a.sz + (int64_t)t * a.st + d0);
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = rope_one((float)x[e], (float)xr[e], (float)c[e], (float)s[e], sign);
  *reinterpret_cast<f16x8*>(dst + d0) = o;
}

// Generic element-wise variant (any even head_dim, any alignment).
__global__ void __launch_bounds__(256) rotary_kernel_scalar(const RotaryArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= a.rows * a.d) return;
  const int d = (int)(gid % a.d);
  int64_t r = gid / a.d;
  const int H = a.hq + a.hk;
  const int h = (int)(r % H);
  r /= H;
  const int t = (int)(r % a.t);
  const int64_t b = r / a.t;
  const int half = a.d >> 1;
  const int dr = (d + half) % a.d;
  const float sign = d < half ? -1.0f : 1.0f;
  const f16* src;
  f16* dst;
  if (h < a.hq) {
    src = a.q + b * a.qz + (int64_t)h * a.qh + (int64_t)t * a.qt;
    dst = a.oq + ((b * a.t + t) * a.hq + h) * a.d;
  } else {
    src = a.k + b * a.kz + (int64_t)(h - a.hq) * a.kh + (int64_t)t * a.kt;
    dst = a.ok + ((b * a.t + t) * a.hk + (h - a.hq)) * a.d;
  }
  const float c = (float)a.cs[b * a.cz + (int64_t)t * a.ct + d];
  const float s = (float)a.sn[b * a.sz + (int64_t)t * a.st + d];
  dst[d] = rope_one((float)src[d], (float)src[dr], c, s, sign);
}

// ---- SiLU * up (reference :850-869) -----------------------------------------
__device__ __forceinline__ f16 silu_mul_one(f16 g16, f16 u16) {
  const float g = (float)g16;
  const f16 act = (f16)keep32(g / keep32(1.0f + expf(-g)));  // IEEE division
  return (f16)((float)act * (float)u16);
}

__global__ void __launch_bounds__(256) silu_mul_kernel(const f16* g, const f16* u, f16* o, int64_t n) {
  const int64_t i8 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i8 + 8 <= n) {
    const f16x8 gv = *reinterpret_cast<const f16x8*>(g + i8);
    const f16x8 uv = *reinterpret_cast<const f16x8*>(u + i8);
    f16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = silu_mul_one(gv[e], uv[e]);
    *reinterpret_cast<f16x8*>(o + i8) = ov;
  } else {
    for (int64_t i = i8; i < n; ++i) o[i] = silu_mul_one(g[i], u[i]);
  }
}

__global__ void __launch_bounds__(256) silu_mul_kernel_scalar(const f16* g, const f16* u, f16* o, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) o[i] = silu_mul_one(g[i], u[i]);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TILEMIX_E_LAUNCH;
  }
  return TILEMIX_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int launch_rmsnorm(const tilemix_rmsnorm_params& p, hipStream_t stream) {
  if (p.x == nullptr || p.weight == nullptr || p.out == nullptr) {
    set_error("tilemix_rms_norm_f16: null tensor pointer");
    return TILEMIX_E_INVALID;
  }
  if (p.rows < 0 || p.cols <= 0 || p.stride_x < p.cols || p.stride_out < p.cols || !(p.eps >= 0.0f)) {
    set_error("tilemix_rms_norm_f16: invalid shape (rows %lld, cols %d, strides %lld/%lld, eps %g)",
              (long long)p.rows, p.cols, (long long)p.stride_x, (long long)p.stride_out, (double)p.eps);
    return TILEMIX_E_INVALID;
  }
  if (p.rows == 0) return TILEMIX_OK;
  NormArgs a;
  a.x = static_cast<const f16*>(p.x);
  a.w = static_cast<const f16*>(p.weight);
  a.out = static_cast<f16*>(p.out);
  a.rows = p.rows;
  a.sx = p.stride_x;
  a.so = p.stride_out;
  a.cols = p.cols;
  a.inv_cols = 1.0f / (float)p.cols;  // the mean's factor, as fp32(1/N)
  a.eps = p.eps;
  // Rows whose start is not 16-byte aligned take the kernel's scalar branch.
  const int64_t blocks = (p.rows + kNormWaves - 1) / kNormWaves;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)blocks), dim3(kNormWaves * 64), 0, stream, a);
  return check_launch("tilemix_rms_norm_f16");
}

int launch_rotary(const tilemix_rotary_params& p, hipStream_t stream) {
  if (p.q == nullptr || p.k == nullptr || p.cos == nullptr || p.sin == nullptr || p.q_out == nullptr ||
      p.k_out == nullptr) {
    set_error("tilemix_rotary_f16: null tensor pointer");
    return TILEMIX_E_INVALID;
  }
  if (p.batch < 0 || p.tokens < 0 || p.heads_q <= 0 || p.heads_k <= 0 || p.head_dim <= 0 || (p.head_dim & 1)) {
    set_error("tilemix_rotary_f16: invalid shape (batch %d, tokens %d, heads %d/%d, head_dim %d)", p.batch,
              p.tokens, p.heads_q, p.heads_k, p.head_dim);
    return TILEMIX_E_INVALID;
  }
  RotaryArgs a;
  a.q = static_cast<const f16*>(p.q);
  a.k = static_cast<const f16*>(p.k);
  a.cs = static_cast<const f16*>(p.cos);
  a.sn = static_cast<const f16*>(p.sin);
  a.oq = static_cast<f16*>(p.q_out);
  a.ok = static_cast<f16*>(p.k_out);
  a.qz = p.stride_q_batch;
  a.qh = p.stride_q_head;
  a.qt = p.stride_q_token;
  a.kz = p.stride_k_batch;
  a.kh = p.stride_k_head;
  a.kt = p.stride_k_token;
  a.cz = p.stride_cos_batch;
  a.ct = p.stride_cos_token;
  a.sz = p.stride_sin_batch;
  a.st = p.stride_sin_token;
  a.t = p.tokens;
  a.hq = p.heads_q;
  a.hk = p.heads_k;
  a.d = p.head_dim;
  a.rows = (int64_t)p.batch * p.tokens * (p.heads_q + p.heads_k);
  if (a.rows == 0) return TILEMIX_OK;
  // 16-byte chunks need head_dim % 16 == 0 (so both halves are chunk aligned)
  // and every row start 16-byte aligned.
  const bool vec = (p.head_dim % 16) == 0 && aligned16(p.q) && aligned16(p.k) && aligned16(p.cos) &&
                   aligned16(p.sin) && aligned16(p.q_out) && aligned16(p.k_out) &&
                   ((a.qz | a.qh | a.qt | a.kz | a.kh | a.kt | a.cz | a.ct | a.sz | a.st) & 7) == 0;
  if (vec) {
    const int64_t threads = a.rows * (p.head_dim / 8);
    hipLaunchKernelGGL(rotary_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  } else {
    const int64_t threads = a.rows * p.head_dim;
    hipLaunchKernelGGL(rotary_kernel_scalar, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  }
  return check_launch("tilemix_rotary_f16");
}

int launch_silu_mul(const void* gate, const void* up, void* out, int64_t n, hipStream_t stream) {
  if (gate == nullptr || up == nullptr || out == nullptr || n < 0) {
    set_error("tilemix_silu_mul_f16: null tensor pointer or negative size");
    return TILEMIX_E_INVALID;
  }
  if (n == 0) return TILEMIX_OK;
  const f16* g = static_cast<const f16*>(gate);
  const f16* u = static_cast<const f16*>(up);
  f16* o = static_cast<f16*>(out);
  if (aligned16(gate) && aligned16(up) && aligned16(out)) {
    const int64_t threads = (n + 7) / 8;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, g, u, o, n);
  } else {
    hipLaunchKernelGGL(silu_mul_kernel_scalar, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, g, u, o, n);
  }
  return check_launch("tilemix_silu_mul_f16");
}

}  // namespace tmx
