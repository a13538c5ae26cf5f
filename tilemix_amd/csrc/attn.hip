// Fused FP16/INT8-routed flash-attention prefill forward for gfx950.
//
// Numerics follow attn_fwd (attention/triton/tilemix.py:503-951):
//   qk_scale = fp32(sm_scale) * fp32(log2 e)                               (:641)
//   q16      = fp16(fp32(q) * qk_scale)                                     (:643-649)
//   FP16 tile: qk = fp16(sum_d q16 * k)            (fp32 MFMA accumulate)  (:254)
//   INT8 tile: acc = sum_d q8 * k8 (exact int32)                            (:401)
//              ss  = fp16(fp32(fp16(sq * sk)) * qk_scale)                   (:388,398)
//              qk  = fp16(fp32(acc) * fp32(ss))                             (:402-404)
//   mask -> -inf (key >= Lk, causal key > row + Lk - Lq)                    (:256-262)
//   online softmax in base 2, p rounded to fp16 before sum and PV           (:179-207)
//   acc += p16 . V (fp32), out = fp16(acc / l)                              (:299,935-951)
// Tiles are visited in ascending key order; tile n uses route bit
// (bitmask[hk*ceil(Lq/block_m)+m] >> (n / (block_n_mask/64))) & 1        (:818-933).
//
// Work decomposition (MI355X-first, not the reference's):
//   * one workgroup = one (sequence, query head, block_m query rows);
//     NW = block_m/32 waves, each wave owns 32 query rows;
//   * every wave computes S^T = K . Q^T with 32x32 MFMAs, so a lane owns ONE
//     query row: row max / row sum are in-lane reductions plus one
//     v_permlane32_swap, and the per-row rescale of O is a per-lane scalar;
//   * O^T = V^T . P^T re-uses the S^T register layout directly as the B
//     operand (no shuffle); V is stored transposed in LDS;
//   * the K tile is staged in LDS as fp16 or int8 according to the tile's
//     route (the bit is uniform per workgroup, so there is no divergence);
//   * next tile's global loads are issued into registers before the current
//     tile's MFMAs (register double buffering);
//   * blockIdx -> work mapping is XCD-aware: each of the 8 XCDs receives a
//     contiguous range of (sequence, kv-head) groups, so the query heads that
//     share K/V (GQA) and all query blocks of a head hit the same L2; within a
//     group, query blocks are issued longest-first (causal).
#include "common.h"

#include <math.h>

namespace tmx {

namespace {

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
  int m_blocks;   // ceil(max_seqlen_q / block_m)
  int mask_tiles; // block_n_mask / block_n
  int blkq, blkk;
  int causal;
  int total_items;
  int per_xcd;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int NW, int DP, int MODE, bool INT8V, bool DUMP>
__global__ void __launch_bounds__(NW * 64) attn_fwd_kernel(const AttnKArgs a) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  constexpr int KS16 = DP / 16;  // fp16 MFMA k-steps (32x32x16)
  constexpr int KS8 = DP / 32;   // int8 MFMA k-steps (32x32x32)
  constexpr int NDB = DP / 32;   // 32-wide d blocks of O^T
  constexpr int K16_LD = DP + 8; // halves per K16 row (16-byte pad: conflict-free 128-bit reads)
  constexpr int K8_LD = DP + 16; // bytes per K8 row
  constexpr int VT_LD = kBN + 4; // halves per V^T row (8-byte pad)
  constexpr int KBYTES = 64 * K16_LD * 2;
  constexpr int VBYTES = DP * VT_LD * 2;
  constexpr int CPR16 = DP / 8;  // 16-byte chunks per fp16 row
  constexpr int CPR8 = DP / 16;  // 16-byte chunks per int8 row
  constexpr int KCH16 = 64 * CPR16 / NT;
  constexpr int KCH8 = 64 * CPR8 / NT;
  constexpr int VPCH = 32 * CPR16 / NT;  // (key pair, 8 dims) chunks per thread
  static_assert(KCH16 * NT == 64 * CPR16 && KCH8 * NT == 64 * CPR8 && VPCH * NT == 32 * CPR16, "tile split");
  static_assert(64 * K8_LD <= KBYTES, "K8 aliases K16");

  __shared__ __attribute__((aligned(16))) unsigned char smem[KBYTES + VBYTES];
  f16* k16s = reinterpret_cast<f16*>(smem);
  int8_t* k8s = reinterpret_cast<int8_t*>(smem);
  f16* vts = reinterpret_cast<f16*>(smem + KBYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  // ---- work item ---------------------------------------------------------
  const int bid = blockIdx.x;
  const int lam = (bid & 7) * a.per_xcd + (bid >> 3);
  if (lam >= a.total_items) return;
  int t = lam;
  const int g = t % a.group;
  t /= a.group;
  const int mrev = t % a.m_blocks;
  t /= a.m_blocks;
  const int hk = t % a.hk;
  const int z = t / a.hk;
  const int m = a.m_blocks - 1 - mrev;
  const int h = hk * a.group + g;

  const int q_start = a.cu_q[z];
  const int Lq = a.cu_q[z + 1] - q_start;
  const int k_start = a.cu_k[z];
  const int Lk = a.cu_k[z + 1] - k_start;
  if (m * BM >= Lq) return;

  int n_blocks = (Lk + kBN - 1) / kBN;
  if (a.causal) {
    const int cn = ((m + 1) * BM + Lk - Lq + kBN - 1) / kBN;
    n_blocks = min(n_blocks, cn);
  }
  const int diag = Lk - Lq;  // causal: key valid iff key <= row + diag

  uint64_t bits = 0;
  if (MODE == TILEMIX_ROUTING_MIXED) {
    const int mbz = (Lq + BM - 1) / BM;  // per-sequence m_blocks (reference :819-820)
    bits = a.bitmask[hk * mbz + m];
  }

  const int row0w = m * BM + wave * 32;  // first row of this wave
  const int row = row0w + l32;            // this lane's query row
  const bool row_ok = row < Lq;

  // ---- Q fragments (B operand of S^T = K . Q^T) --------------------------
  f16x8 qf[KS16];
  i32x4 q8f[KS8];
  f16 sq16 = (f16)1.0f;
  if (MODE != TILEMIX_ROUTING_INT8) {
    const f16* qp = a.q + (int64_t)(q_start + row) * a.sq_t + (int64_t)h * a.sq_h;
#pragma unroll
    for (int s = 0; s < KS16; ++s) {
      const int d0 = 16 * s + 8 * hi;
      f16x8 raw = {};
      if (row_ok && d0 < a.d) raw = *reinterpret_cast<const f16x8*>(qp + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = (f16)((float)raw[e] * a.qk_scale);
    }
  }
  if (MODE != TILEMIX_ROUTING_FP16) {
    const int8_t* qp = a.q8 + (int64_t)(q_start + row) * a.sq8_t + (int64_t)h * a.sq8_h;
#pragma unroll
    for (int s = 0; s < KS8; ++s) {
      const int d0 = 32 * s + 16 * hi;
      i32x4 raw = {};
      if (row_ok && d0 < a.d) raw = *reinterpret_cast<const i32x4*>(qp + d0);
      q8f[s] = raw;
    }
    const int qb = a.cu_qs[z], qe = a.cu_qs[z + 1];
    if (qe > qb) {
      const int idx = min(qb + row / a.blkq, qe - 1);
      sq16 = a.sq[(int64_t)idx * a.hq + h];
    }
  }

  // ---- tile staging ------------------------------------------------------
  uint4 kreg[KCH16];
  uint4 vreg[2 * VPCH];
  const uint4 zero4 = make_uint4(0, 0, 0, 0);

  auto route_of = [&](int n) -> int {
    if (MODE == TILEMIX_ROUTING_FP16) return 0;
    if (MODE == TILEMIX_ROUTING_INT8) return 1;
    return (int)((bits >> (unsigned)(n / a.mask_tiles)) & 1ull);
  };

  auto load_tile = [&](int n, int route) {
    const int key0 = n * kBN;
    if (route == 0) {
#pragma unroll
      for (int i = 0; i < KCH16; ++i) {
        const int c = tid + i * NT;
        const int r = c / CPR16, col = (c % CPR16) * 8;
        const int key = key0 + r;
        kreg[i] = (key < Lk && col < a.d)
                      ? *reinterpret_cast<const uint4*>(a.k + (int64_t)(k_start + key) * a.sk_t +
                                                        (int64_t)hk * a.sk_h + col)
                      : zero4;
      }
    } else {
#pragma unroll
      for (int i = 0; i < KCH8; ++i) {
        const int c = tid + i * NT;
        const int r = c / CPR8, col = (c % CPR8) * 16;
        const int key = key0 + r;
        kreg[i] = (key < Lk && col < a.d)
                      ? *reinterpret_cast<const uint4*>(a.k8 + (int64_t)(k_start + key) * a.sk8_t +
                                                        (int64_t)hk * a.sk8_h + col)
                      : zero4;
      }
    }
    if (!INT8V || route == 0) {
#pragma unroll
      for (int i = 0; i < VPCH; ++i) {
        const int c = tid + i * NT;
        const int kp = c / CPR16, col = (c % CPR16) * 8;
        const int key = key0 + 2 * kp;
        const f16* vp = a.v + (int64_t)(k_start + key) * a.sv_t + (int64_t)hk * a.sv_h + col;
        const bool cok = col < a.d;
        vreg[2 * i] = (cok && key < Lk) ? *reinterpret_cast<const uint4*>(vp) : zero4;
        vreg[2 * i + 1] = (cok && key + 1 < Lk) ? *reinterpret_cast<const uint4*>(vp + a.sv_t) : zero4;
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPCH; ++i) {
        const int c = tid + i * NT;
        const int kp = c / CPR16, col = (c % CPR16) * 8;
        const int key = key0 + 2 * kp;
        const int8_t* vp = a.v8 + (int64_t)(k_start + key) * a.sv8_t + (int64_t)hk * a.sv8_h + col;
        const bool cok = col < a.d;
        const uint2 v0 = (cok && key < Lk) ? *reinterpret_cast<const uint2*>(vp) : make_uint2(0, 0);
        const uint2 v1 = (cok && key + 1 < Lk) ? *reinterpret_cast<const uint2*>(vp + a.sv8_t) : make_uint2(0, 0);
        vreg[2 * i] = make_uint4(v0.x, v0.y, 0, 0);
        vreg[2 * i + 1] = make_uint4(v1.x, v1.y, 0, 0);
      }
    }
  };

  auto store_tile = [&](int route) {
    if (route == 0) {
#pragma unroll
      for (int i = 0; i < KCH16; ++i) {
        const int c = tid + i * NT;
        const int r = c / CPR16, col = (c % CPR16) * 8;
        *reinterpret_cast<uint4*>(k16s + r * K16_LD + col) = kreg[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < KCH8; ++i) {
        const int c = tid + i * NT;
        const int r = c / CPR8, col = (c % CPR8) * 16;
        *reinterpret_cast<uint4*>(k8s + r * K8_LD + col) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VPCH; ++i) {
      const int c = tid + i * NT;
      const int kp = c / CPR16, col = (c % CPR16) * 8;
      f16x8 v0, v1;
      if (!INT8V || route == 0) {
        v0 = __builtin_bit_cast(f16x8, vreg[2 * i]);
        v1 = __builtin_bit_cast(f16x8, vreg[2 * i + 1]);
      } else {
        const uint32_t w[4] = {vreg[2 * i].x, vreg[2 * i].y, vreg[2 * i + 1].x, vreg[2 * i + 1].y};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v0[e] = (f16)(float)(int8_t)((w[e >> 2] >> (8 * (e & 3))) & 0xff);
          v1[e] = (f16)(float)(int8_t)((w[2 + (e >> 2)] >> (8 * (e & 3))) & 0xff);
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        f16x2 pr;
        pr[0] = v0[j];
        pr[1] = v1[j];
        *reinterpret_cast<f16x2*>(vts + (col + j) * VT_LD + 2 * kp) = pr;
      }
    }
  };

  // ---- online softmax state (one query row per lane) ----------------------
  float m_i = -INFINITY;
  float l_i = 1.0f;
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = (f32x16){};

  int route_next = 0;
  if (n_blocks > 0) {
    route_next = route_of(0);
    load_tile(0, route_next);
  }

  for (int n = 0; n < n_blocks; ++n) {
    const int route = route_next;
    if (n > 0) __syncthreads();  // every wave finished reading tile n-1
    store_tile(route);
    __syncthreads();
    if (n + 1 < n_blocks) {
      route_next = route_of(n + 1);
      load_tile(n + 1, route_next);
    }

    const int key0 = n * kBN;
    // Fully masked for this wave (or rows past the sequence end): the
    // reference's update is then an exact no-op (p = 0, alpha = 1).
    const bool wave_skip = (row0w >= Lq) || (a.causal && key0 > row0w + 31 + diag);
    if (wave_skip) continue;

    // ---- S^T = K . Q^T --------------------------------------------------
    float s[2][16];
    if (route == 0) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 c = {};
#pragma unroll
        for (int ks = 0; ks < KS16; ++ks) {
          const f16x8 av = *reinterpret_cast<const f16x8*>(k16s + (kb * 32 + l32) * K16_LD + 16 * ks + 8 * hi);
          c = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qf[ks], c, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = (float)(f16)c[r];
      }
    } else {
      f16 sk16 = (f16)1.0f;
      {
        const int kbase = a.cu_ks[z], kend = a.cu_ks[z + 1];
        if (kend > kbase) {
          const int idx = min(kbase + key0 / a.blkk, kend - 1);
          sk16 = a.sk[(int64_t)idx * a.hk + hk];
        }
      }
      const f16 sqk = sq16 * sk16;
      const float ss = (float)(f16)((float)sqk * a.qk_scale);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        i32x16 c = {};
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
          const i32x4 av = *reinterpret_cast<const i32x4*>(k8s + (kb * 32 + l32) * K8_LD + 32 * ks + 16 * hi);
          c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, q8f[ks], c, 0, 0, 0);
        }
        if (DUMP && a.dump_i32 != nullptr && row_ok) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
            if (key < Lk) a.dump_i32[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = c[r];
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = (float)(f16)((float)c[r] * ss);
      }
    }
    if (DUMP && a.dump_f16 != nullptr && row_ok) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (key < Lk) a.dump_f16[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = (f16)s[kb][r];
        }
    }

    // ---- mask + optional bias ------------------------------------------
    const bool need_mask = (key0 + kBN > Lk) || (a.causal && key0 + kBN - 1 > row0w + diag);
    if (need_mask || a.bias != nullptr) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
          const bool valid = key < Lk && (!a.causal || key <= row + diag);
          if (!valid) {
            s[kb][r] = -INFINITY;
          } else if (a.bias != nullptr && row_ok) {
            // Reference :264-272: qk(fp16) += fp16(b * LOG2E) with LOG2E taken
            // as an fp16 constant against the fp16 bias (weak scalar typing);
            // the bias row pointer carries no batch offset (quirk kept).
            const f16 b = a.bias[(int64_t)h * a.sb_h + (int64_t)row * a.sb_m + (int64_t)key * a.sb_n];
            const f16 bl = b * (f16)1.4426950408889634f;
            s[kb][r] = (float)((f16)s[kb][r] + bl);
          }
        }
    }

    // ---- online softmax (reference _softmax_prefix_update) -------------
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    {
      const float2 sw = swap_halves(mx);
      mx = fmaxf(sw.x, sw.y);
    }
    const bool has = mx != -INFINITY;
    const float m_next = has ? fmaxf(m_i, mx) : m_i;
    const float alpha = has ? fast_exp2(m_i - m_next) : 1.0f;
    f16x8 pb[4];
    float ls = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const f16 p = has ? (f16)fast_exp2(s[kb][r] - m_next) : (f16)0.0f;
        ls += (float)p;
        pb[kb * 2 + (r >> 3)][r & 7] = p;
      }
    {
      const float2 sw = swap_halves(ls);
      ls = sw.x + sw.y;
    }
    l_i = l_i * alpha + ls;
    m_i = m_next;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;

    if (INT8V && route == 1) {
      // Reference :449-497: PV on int8 V codes with p scaled by the V block
      // scale in fp16: p_scaled = fp16(p * sv).
      f16 sv16 = (f16)1.0f;
      const int vb = a.cu_vs[z], ve = a.cu_vs[z + 1];
      if (ve > vb) {
        const int idx = min(vb + key0 / a.blkk, ve - 1);
        sv16 = a.sv[(int64_t)idx * a.hk + hk];
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[ks][e] = pb[ks][e] * sv16;
    }

    // ---- O^T += V^T . P^T ----------------------------------------------
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16* vrow = vts + (db * 32 + l32) * VT_LD + 16 * ks + 4 * hi;
        const f16x4 lo = *reinterpret_cast<const f16x4*>(vrow);
        const f16x4 up = *reinterpret_cast<const f16x4*>(vrow + 8);
        const f16x8 av = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb[ks], acc[db], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: out = fp16(acc / l) --------------------------------------
  if (row_ok) {
    f16* op = a.out + (int64_t)(q_start + row) * a.so_t + (int64_t)h * a.so_h;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = db * 32 + 8 * rq + 4 * hi;
        if (d0 < a.d) {
          f16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (f16)(acc[db][4 * rq + e] / l_i);
          *reinterpret_cast<f16x4*>(op + d0) = o;
        }
      }
  }
}

template <int NW, int DP, int MODE, bool INT8V, bool DUMP>
void launch_one(const AttnKArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<NW, DP, MODE, INT8V, DUMP>), dim3(8 * a.per_xcd), dim3(NW * 64), 0,
                     stream, a);
}

template <int NW, int DP, bool DUMP>
void dispatch_mode(const AttnKArgs& a, int mode, bool int8v, hipStream_t stream) {
  if (mode == TILEMIX_ROUTING_FP16) {
    launch_one<NW, DP, TILEMIX_ROUTING_FP16, false, DUMP>(a, stream);
  } else if (mode == TILEMIX_ROUTING_INT8) {
    if (int8v) launch_one<NW, DP, TILEMIX_ROUTING_INT8, true, DUMP>(a, stream);
    else launch_one<NW, DP, TILEMIX_ROUTING_INT8, false, DUMP>(a, stream);
  } else {
    if (int8v) launch_one<NW, DP, TILEMIX_ROUTING_MIXED, true, DUMP>(a, stream);
    else launch_one<NW, DP, TILEMIX_ROUTING_MIXED, false, DUMP>(a, stream);
  }
}

template <bool DUMP>
void dispatch(const AttnKArgs& a, int nw, int dp, int mode, bool int8v, hipStream_t stream) {
  if (nw == 4) {
    if (dp == 128) dispatch_mode<4, 128, DUMP>(a, mode, int8v, stream);
    else dispatch_mode<4, 64, DUMP>(a, mode, int8v, stream);
  } else {
    if (dp == 128) dispatch_mode<2, 128, DUMP>(a, mode, int8v, stream);
    else dispatch_mode<2, 64, DUMP>(a, mode, int8v, stream);
  }
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace

int launch_attn(const tilemix_attn_params& p, int32_t* dump_i32, void* dump_f16, int64_t dump_t,
                int64_t dump_h, hipStream_t stream) {
  const char* fn = (dump_i32 || dump_f16) ? "tilemix_attn_fwd_debug" : "tilemix_attn_fwd";
  if (!p.q || !p.k || !p.v || !p.out || !p.cu_seqlens_q || !p.cu_seqlens_k) {
    set_error("%s: null q/k/v/out/cu_seqlens pointer", fn);
    return TILEMIX_E_INVALID;
  }
  if (p.routing_mode < 0 || p.routing_mode > 2) {
    set_error("%s: routing_mode must be 0 (mixed), 1 (fp16) or 2 (int8), got %d", fn, p.routing_mode);
    return TILEMIX_E_INVALID;
  }
  if (p.heads_q <= 0 || p.heads_k <= 0 || p.heads_q % p.heads_k != 0) {
    set_error("%s: Q heads (%d) must be a positive multiple of KV heads (%d)", fn, p.heads_q, p.heads_k);
    return TILEMIX_E_INVALID;
  }
  if (p.head_dim <= 0 || p.head_dim > 128 || p.head_dim % 16 != 0) {
    set_error("%s: head_dim must be a multiple of 16 in [16, 128], got %d", fn, p.head_dim);
    return TILEMIX_E_INVALID;
  }
  if (p.block_m != 64 && p.block_m != 128) {
    set_error("%s: block_m must be 64 or 128 in this build, got %d", fn, p.block_m);
    return TILEMIX_E_INVALID;
  }
  if (p.block_n != kBN) {
    set_error("%s: block_n must be 64 in this build, got %d", fn, p.block_n);
    return TILEMIX_E_INVALID;
  }
  if (p.block_n_mask <= 0 || p.block_n_mask % p.block_n != 0) {
    set_error("%s: block_n_mask (%d) must be a positive multiple of block_n (%d)", fn, p.block_n_mask,
              p.block_n);
    return TILEMIX_E_INVALID;
  }
  if (p.max_seqlen_q < 0 || p.max_seqlen_k < 0 || p.batch < 0) {
    set_error("%s: negative sizes", fn);
    return TILEMIX_E_INVALID;
  }
  if ((p.max_seqlen_k + p.block_n_mask - 1) / p.block_n_mask > 64) {
    set_error("%s: packed routing exceeds 64 mask blocks (max_seqlen_k=%d, block_n_mask=%d)", fn,
              p.max_seqlen_k, p.block_n_mask);
    return TILEMIX_E_INVALID;
  }
  const bool need_int8 = p.routing_mode != TILEMIX_ROUTING_FP16;
  const bool int8v = need_int8 && !p.int8_use_fp16_v;
  if (p.routing_mode == TILEMIX_ROUTING_MIXED && !p.precision_bitmask) {
    set_error("%s: mixed routing needs precision_bitmask", fn);
    return TILEMIX_E_INVALID;
  }
  if (need_int8) {
    if (!p.q8 || !p.k8 || !p.sq || !p.sk || !p.cu_q_scale || !p.cu_k_scale) {
      set_error("%s: int8 routing needs q8/k8/sq/sk/cu_q_scale/cu_k_scale", fn);
      return TILEMIX_E_INVALID;
    }
    if (p.blkq <= 0 || p.blkk <= 0 || p.blkk % kBN != 0) {
      set_error("%s: BLKQ must be positive and BLKK a multiple of 64 in this build (BLKQ=%d, BLKK=%d)", fn,
                p.blkq, p.blkk);
      return TILEMIX_E_INVALID;
    }
    if (!aligned(p.q8, 16) || !aligned(p.k8, 16) || (p.stride_q8_token | p.stride_q8_head) % 16 ||
        (p.stride_k8_token | p.stride_k8_head) % 16) {
      set_error("%s: q8/k8 must be 16-byte aligned with strides multiple of 16 elements", fn);
      return TILEMIX_E_INVALID;
    }
    if (int8v) {
      if (!p.v8 || !p.sv || !p.cu_v_scale) {
        set_error("%s: int8 V path needs v8/sv/cu_v_scale", fn);
        return TILEMIX_E_INVALID;
      }
      if (!aligned(p.v8, 8) || (p.stride_v8_token | p.stride_v8_head) % 8) {
        set_error("%s: v8 must be 8-byte aligned with strides multiple of 8 elements", fn);
        return TILEMIX_E_INVALID;
      }
    }
  }
  if (!aligned(p.q, 16) || !aligned(p.k, 16) || !aligned(p.v, 16) || !aligned(p.out, 8) ||
      (p.stride_q_token | p.stride_q_head | p.stride_k_token | p.stride_k_head | p.stride_v_token |
       p.stride_v_head) % 8 ||
      (p.stride_o_token | p.stride_o_head) % 4) {
    set_error("%s: q/k/v must be 16-byte aligned with strides multiple of 8 elements (out: 8-byte, 4)", fn);
    return TILEMIX_E_INVALID;
  }
  if ((dump_i32 || dump_f16) && (dump_t < 0 || dump_h < 0)) {
    set_error("%s: invalid dump strides", fn);
    return TILEMIX_E_INVALID;
  }

  const int m_blocks = (p.max_seqlen_q + p.block_m - 1) / p.block_m;
  const int64_t total = (int64_t)m_blocks * p.heads_q * p.batch;
  if (total == 0) return TILEMIX_OK;
  if (total > (int64_t)1 << 30) {
    set_error("%s: too many work items (%lld)", fn, (long long)total);
    return TILEMIX_E_INVALID;
  }

  AttnKArgs a;
  a.q = static_cast<const f16*>(p.q);
  a.k = static_cast<const f16*>(p.k);
  a.v = static_cast<const f16*>(p.v);
  a.bias = static_cast<const f16*>(p.bias);
  a.out = static_cast<f16*>(p.out);
  a.bitmask = p.precision_bitmask;
  a.q8 = p.q8;
  a.k8 = p.k8;
  a.v8 = p.v8;
  a.sq = static_cast<const f16*>(p.sq);
  a.sk = static_cast<const f16*>(p.sk);
  a.sv = static_cast<const f16*>(p.sv);
  a.cu_q = p.cu_seqlens_q;
  a.cu_k = p.cu_seqlens_k;
  a.cu_qs = p.cu_q_scale;
  a.cu_ks = p.cu_k_scale;
  a.cu_vs = p.cu_v_scale;
  a.sq_t = p.stride_q_token;
  a.sq_h = p.stride_q_head;
  a.sk_t = p.stride_k_token;
  a.sk_h = p.stride_k_head;
  a.sv_t = p.stride_v_token;
  a.sv_h = p.stride_v_head;
  a.so_t = p.stride_o_token;
  a.so_h = p.stride_o_head;
  a.sq8_t = p.stride_q8_token;
  a.sq8_h = p.stride_q8_head;
  a.sk8_t = p.stride_k8_token;
  a.sk8_h = p.stride_k8_head;
  a.sv8_t = p.stride_v8_token;
  a.sv8_h = p.stride_v8_head;
  a.sb_h = p.stride_bias_head;
  a.sb_m = p.stride_bias_m;
  a.sb_n = p.stride_bias_n;
  a.dump_i32 = dump_i32;
  a.dump_f16 = static_cast<f16*>(dump_f16);
  a.dump_t = dump_t;
  a.dump_h = dump_h;
  a.qk_scale = p.sm_scale * kLog2eF32;
  a.hq = p.heads_q;
  a.hk = p.heads_k;
  a.group = p.heads_q / p.heads_k;
  a.d = p.head_dim;
  a.m_blocks = m_blocks;
  a.mask_tiles = p.block_n_mask / p.block_n;
  a.blkq = p.blkq > 0 ? p.blkq : 1;
  a.blkk = p.blkk > 0 ? p.blkk : kBN;
  a.causal = p.causal ? 1 : 0;
  a.total_items = (int)total;
  a.per_xcd = (int)((total + 7) / 8);

  const int nw = p.block_m / 32;
  const int dp = p.head_dim <= 64 ? 64 : 128;
  if (dump_i32 || dump_f16) dispatch<true>(a, nw, dp, p.routing_mode, int8v, stream);
  else dispatch<false>(a, nw, dp, p.routing_mode, int8v, stream);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", fn, hipGetErrorString(err));
    return TILEMIX_E_LAUNCH;
  }
  return TILEMIX_OK;
}

}  // namespace tmx
