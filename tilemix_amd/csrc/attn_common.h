// Shared pieces of the attention kernels: argument block, numerics helpers,
// LDS access primitives and swizzles.
#pragma once

#include "common.h"

#include <math.h>

namespace tmx {

constexpr int kBN = 64;  // keys per compute tile (block_n)

struct AttnKArgs {
  const f16* q;
  const f16* k;
  const f16* v;
  const f16* bias;
  f16* out;
  const uint64_t* bitmask;
  const int8_t* q8;
  const int8_t* k8;
  const int8_t* v8;
  const f16* sq;
  const f16* sk;
  const f16* sv;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* cu_qs;
  const int32_t* cu_ks;
  const int32_t* cu_vs;
  int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, so_t, so_h;
  int64_t sq8_t, sq8_h, sk8_t, sk8_h, sv8_t, sv8_h;
  int64_t sb_h, sb_m, sb_n;
  int32_t* dump_i32;
  f16* dump_f16;
  int64_t dump_t, dump_h;
  float qk_scale;
  int hq, hk, group, d;
  int m_blocks;   // ceil(max_seqlen_q / rows per workgroup)
  int route_shift; // log2(block_m / rows per workgroup) of the 128-row kernel: block_m 128 / 256 / 512
  int mask_tiles; // 64-key tiles per routing block: block_n_mask / 64
  int ng;         // 64-key tiles per online-softmax step: block_n / 64 (GEN kernels)
  int blkq, blkk;
  int causal;
  int q_fused;      // Q quantised in the attention kernel (128-row workgroups, BLKQ == 128)
  int total_items;  // (sequence, query head, query block) work items
  int per_xcd;
  int pipe;         // the pipelined assembly tile body may serve this launch
  int ilv;          // groups of an XCD interleaved item by item (interleave_groups)
};

// Work item of workgroup `bid`, or -1.  Items are numbered
// ((z * hk + kv_head) * m_blocks + mrev) * group + g, so one (sequence, kv head)
// "group" is ipg = m_blocks * group consecutive items, its query blocks
// longest first.  Workgroups reach the 8 XCDs round-robin (bid & 7); the j-th
// workgroup of XCD x takes
//   * while whole rounds of 8 groups remain: from XCD x's groups x, x + 8,
//     x + 16, ... -- a group stays on one XCD (its L2 serves every re-read of
//     the group's K/V tiles) and groups are dealt round-robin, so every XCD
//     gets the same mix of long and short sequences.  The XCD's groups run ilv
//     at a time, interleaved item by item (chunk c = j / (ilv ipg) holds groups
//     c ilv .. c ilv + kc - 1, kc = min(ilv, groups left); position w = j mod
//     (ilv ipg) takes item w / kc of group c ilv + w mod kc): the last items
//     dispatched are then the short query blocks of ilv groups instead of
//     every block of the last group, which shortens the launch's tail, as
//     long as ilv groups' K/V stay in the XCD's L2 (interleave_groups);
//   * for the last G % 8 groups: their items dealt over all 8 XCDs (item
//     8 j' + x), which also covers a launch with fewer than 8 groups.
// per_xcd (the grid is 8 * per_xcd) = (G / 8) * ipg + ceil((G % 8) * ipg / 8).
__host__ __device__ inline int64_t work_items_per_xcd(int64_t groups, int64_t ipg) {
  return (groups / 8) * ipg + ((groups % 8) * ipg + 7) / 8;
}
__host__ __device__ __forceinline__ int work_item(int bid, int total_items, int ipg, int ilv) {
  const int x = bid & 7, j = bid >> 3;
  const int groups = total_items / ipg;
  const int gpx = groups / 8;            // whole-round groups per XCD
  const int full_j = gpx * ipg;          // workgroups per XCD in whole rounds
  if (j < full_j) {
    const int c = j / (ilv * ipg);
    const int kc = min(ilv, gpx - c * ilv);
    const int w = j - c * ilv * ipg;
    return (x + 8 * (c * ilv + w % kc)) * ipg + w / kc;
  }
  const int item = gpx * 8 * ipg + 8 * (j - full_j) + x;
  return item < total_items ? item : -1;
}

// Groups interleaved per XCD (work_item): as many as keep their K/V tiles
// (fp16 K and V, int8 K: 5 bytes per key and head-dim column) within ~5.5 MB,
// a little over one XCD's 4 MB L2, at most 4.  Measured on cfg2-like
// launches: 4096 keys (2.6 MB per group) -> 2, 2048 keys -> 4 (-2.6% / -4.3%
// kernel time); 8192-key groups stay at 1 (2 or 4 of them thrash the L2:
// +15% / +46%).
__host__ __device__ inline int interleave_groups(int64_t max_seqlen_k, int head_dim) {
  const int64_t group_bytes = max_seqlen_k * (int64_t)head_dim * 5;
  const int64_t k = group_bytes > 0 ? (int64_t)(5632 * 1024) / group_bytes : 4;
  return k < 1 ? 1 : k > 4 ? 4 : (int)k;
}

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// fp32(h) - m with one rounding (v_fma_mix: the fp16 operand is converted exactly).
__device__ __forceinline__ float sub_lo(uint32_t h2, float negm) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(negm));
  return r;
}
__device__ __forceinline__ float sub_hi(uint32_t h2, float negm) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(negm));
  return r;
}

// Packed fp16 max without the operand canonicalisation the generic builtin
// adds (the operands are conversion results or -inf: never signalling NaNs).
__device__ __forceinline__ uint32_t pk_max(uint32_t x, uint32_t y) {
  uint32_t r;
  asm("v_pk_max_f16 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
  return r;
}

// Packed fp16 maximum of three (IEEE maximum: the scores are never NaN for
// finite inputs, and the sign of a zero maximum does not reach the results:
// exp2(s - m) and exp2(m_old - m_new) are the same for m = +0 and -0).
__device__ __forceinline__ uint32_t pk_max3(uint32_t x, uint32_t y, uint32_t z) {
  uint32_t r;
  asm("v_pk_maximum3_f16 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
  return r;
}

// Eight int8 codes (bytes of w[0], then w[1]) to fp16, exactly: with the
// sign bit flipped a code b is the byte u = b + 128, the fp16 with bits
// 0x64XX is 1024 + u, and 1024 + u - 1152 = b (all exact small integers).
// One byte permute builds two fp16 values, one packed add unbiases them.
__device__ __forceinline__ f16x8 int8x8_to_f16(i32x2 w) {
  const uint32_t w0 = (uint32_t)w[0] ^ 0x80808080u, w1 = (uint32_t)w[1] ^ 0x80808080u;
  const f16x2 bias = {(f16)-1152.0f, (f16)-1152.0f};
  // v_perm_b32: selector byte k < 4 picks byte k of the second source, k = 4
  // picks byte 0 of the first (0x64).  (A plain array, not a vector: clang
  // bit-casts an element of a vector variable from the vector's first bytes.)
  const uint32_t r[4] = {__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                         __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u),
                         __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)};
  f16x8 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 v = __builtin_bit_cast(f16x2, r[i]) + bias;
    out[2 * i] = v[0];
    out[2 * i + 1] = v[1];
  }
  return out;
}

// Materialise an fp32 value.  The reference rounds to fp32 and then to fp16
// (Triton: mul.f32 / fma, then cvt.rn.f16.f32); without this barrier the
// compiler fuses fptrunc(fma(a, b, c)) / fptrunc(fmul(a, b)) into one
// v_fma_mix*_f16, a single rounding that differs on double ties.
__device__ __forceinline__ float fp32_round(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  f16x2 v;
  v[0] = (f16)a;
  v[1] = (f16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// RN(h * s) for the low / high fp16 half of h2: the fp16 operand converts
// exactly, so the product is rounded once, as RN(fp32(h) * s); the addend
// -0 keeps the sign of a zero product.
__device__ __forceinline__ float mul_lo(uint32_t h2, float s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "v"(-0.0f));
  return r;
}
__device__ __forceinline__ float mul_hi(uint32_t h2, float s) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "v"(-0.0f));
  return r;
}

// x / s correctly rounded, from r = RN(1/s): q0 = RN(x r), rem = x - q0 s
// (exact, one FMA), RN(q0 + rem r) (Markstein's correction step).  For the
// quantisation domain (x an fp16 value, s = RN(amax/127) with |x| <= amax, amax
// a positive fp16 value) this equals IEEE x / s on all 1.0e9 (x, amax) pairs
// up to the sign of a zero quotient, which the int8 code does not see.
__device__ __forceinline__ float div_by_recip(float x, float s, float r) {
  const float q0 = x * r;
  const float rem = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(rem, r, q0);
}

// Lane pairs (l, l^16) and (l, l^32): returns {value of the lower lane, value
// of the upper lane} on both lanes, so op(x, y) is bitwise identical on both.
__device__ __forceinline__ float2 pair16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 pair32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// HBM -> LDS copy of 16 bytes per lane (buffer_load_dwordx4 ... lds: lane l
// writes lds + 16 l) through a raw buffer over [base, base + bytes), so loads
// at offsets >= bytes return 0.  Issued from inline assembly: the kernels
// order the copies against their LDS reads themselves (s_waitcnt vmcnt(0) +
// barrier before a stage is read).  Through the compiler builtin, the
// compiler cannot tell the stage being filled from the stage being read and
// waits for the copy before every LDS read, which serialises the prefetch with
// the tile's compute.  rsrc and lds are wave-uniform (SGPRs); M0 carries the
// LDS address.  Five wait states precede the load: one is what an M0 write
// needs before it, five what a VALU write of an SGPR (v_readfirstlane, or a
// v_readlane that reloads a spilled descriptor) needs before a VMEM
// instruction reads that SGPR -- the compiler pads its own loads for both,
// but not a load inside an asm statement, and without the padding a spilled
// buffer descriptor reloaded right before the copy was read half-updated
// (a memory fault).  tests/test_asm_hazards.py scans every instantiation.
struct SRsrc {
  i32x4 w;
};
// A lane offset past every buffer's size: the copy reads nothing and writes
// zeros.  The host checks (max_seqlen_k + 64) * token stride < 2^31 bytes, so
// a sequence's buffer spans less than 2^31 bytes and a tile's offset plus the
// row offsets of its 64 rows, added to this value, stay below 2^32 (no wrap
// back into range).
constexpr int kOffOutside = (int)0x80000000u;
__device__ __forceinline__ SRsrc make_srsrc(const void* base, int bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  SRsrc r;
  r.w[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r.w[1] = __builtin_amdgcn_readfirstlane((int)((p >> 32) & 0xffffu));
  r.w[2] = __builtin_amdgcn_readfirstlane(bytes);
  r.w[3] = 0x00020000;
  return r;
}
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)reinterpret_cast<uintptr_t>((const lds_void*)p));
}
__device__ __forceinline__ void async_load16_asm(const SRsrc& rs, int voffset, uint32_t lds) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voffset), "s"(rs.w), "{m0}"(lds)
      : "memory");
}

// Transposed LDS read (gfx950): within each 16-lane group, output lane i,
// element c = element (i % 4) of the 8 bytes addressed by lane 4c + i/4.
__device__ __forceinline__ f16x4 lds_read_tr16(const unsigned char* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(f16x4, v);
}

// ---- LDS layouts ----------------------------------------------------------
// All tiles are 64 rows (keys).  A row is split in 16-byte chunks; logical
// chunk c of row r lives at physical chunk c ^ swz(r).  Each swizzle spreads
// one LDS pass (16 lanes of ds_read_b128, 32 lanes of a transposed b64 read)
// over all 64 banks:
//   K fp16 / int8 (ds_read_b128): 16 lanes read one chunk of 16 consecutive rows;
//   V fp16 (ds_read_b64_tr_b16): 32 lanes read 2 chunks of 8 consecutive rows.
// int8 V codes are copied like int8 K (swz_k) and widened to the fp16 V layout.
template <int ROWB>
__device__ __forceinline__ int swz_k(int r) {
  if constexpr (ROWB >= 256) return r & 15;
  else if constexpr (ROWB == 128) return (r >> 1) & 7;
  else return (r >> 2) & 3;  // 64-byte rows
}
template <int ROWB>
__device__ __forceinline__ int swz_v(int r) {
  if constexpr (ROWB >= 256) return 2 * (r & 7);
  else return 2 * ((r >> 1) & 3);  // 128-byte rows
}
// The 32-row kernel reads V with 16 lanes x 4 rows x 64 bytes per pass
// (ds_read_b64_tr_b16 over a 32-wide d block).
template <int ROWB>
__device__ __forceinline__ int swz_v32(int r) {
  if constexpr (ROWB >= 256) return 4 * (r & 3);
  else return 4 * ((r >> 1) & 1);  // 128-byte rows: row pairs share a bank line
}

// Which kernel runs a launch (chosen in launch_attn).
enum AttnKind : int {
  kAttn32 = 0,       // 32-row kernel, one routing block per 128-row workgroup
  kAttn32Split = 1,  // 32-row kernel, two 64-row routing blocks per workgroup
  kAttn16 = 2,       // 16-row kernel, one 64-row routing block per workgroup
};

// Launch one instantiation (defined in attn_inst_*.hip).  gen selects the
// GEN kernels (block_n > 64, or scale blocks that are not multiples of 64).
void dispatch_attn(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, bool dump, bool bias, bool gen,
                   hipStream_t stream);

}  // namespace tmx
