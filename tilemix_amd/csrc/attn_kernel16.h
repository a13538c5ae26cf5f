// Fused FP16/INT8-routed flash-attention prefill forward for gfx950: the
// 16-row kernel, which runs block_m = 64 with mixed routing on int8 V codes
// (the 32-row kernel's split workgroups would need both V formats in LDS).
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
//     NW = block_m/16 waves, each wave owns 16 query rows.  16-row waves fit
//     in 128 VGPRs: 4 waves per SIMD at head_dim 64 (the MFMAs of one wave
//     run beside the softmax of the others); at head_dim 128 the 64 KB of LDS
//     per workgroup allows 2;
//   * every wave computes S^T = K . Q^T with 16x16 MFMAs (16x16x32 f16,
//     16x16x64 i8).  Lane l owns query row l%16 and keys 16 kb + 4 (l/16) + r
//     (kb, r = 0..3) of each 64-key tile; a row's 4 lanes combine with one
//     v_permlane16_swap and one v_permlane32_swap;
//   * O^T = V^T . P^T takes P^T straight from those registers: the MFMA's k
//     slots 8 (l/16) + t are mapped to keys 32 ks + 4 (l/16) + (t%4) + 16 (t/4),
//     and the V^T operand is read in the same key order with two
//     ds_read_b64_tr_b16 (int8 V codes are first widened to fp16 in LDS);
//   * the row sum l is kept per lane (partial over the lane's keys, rescaled
//     by the row's alpha) and combined across the row's 4 lanes once, at the end;
//   * K (fp16 or int8, by the tile's route) and V tiles are streamed straight
//     from HBM into double-buffered LDS with buffer_load_dwordx4 ... lds (no
//     staging registers), in XOR-swizzled layouts that make every LDS read
//     pattern of the MFMA operands bank-conflict free;
//   * INT8 tiles accumulate on top of a magic bias (1.5*2^23 as int bits) so
//     the exact fp32(acc)*ss of the reference is one FMA;
//   * blockIdx -> work mapping is XCD-aware (work_item in attn_common.h):
//     whole (sequence, kv-head) groups are dealt round-robin to the 8 XCDs, so
//     the query heads that share K/V (GQA) and all query blocks of a head hit
//     the same L2 and every XCD gets the same mix of sequence lengths; within a
//     group, query blocks are issued longest-first (causal).
#pragma once

#include "attn_common.h"

namespace tmx {

// Occupancy target: 4 waves per SIMD at head_dim 64; at 128 the LDS allows 2.
template <int NW, int DP, int MODE, bool INT8V, bool DUMP, bool BIAS, bool GEN>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(DP <= 64 ? 4 : 2, DP <= 64 ? 4 : 2)))
attn16_kernel(const AttnKArgs a) {
  constexpr int BM = NW * 16;
  // K/V scales per tile and lane: one, or (GEN) one per 4-key group kb of the
  // lane's keys 16 kb + 4 lg .. + 3.
  constexpr int NSG = GEN ? 4 : 1;
  constexpr int KS16 = DP / 32;  // fp16 k-steps (16x16x32)
  constexpr int KS8 = DP / 64;   // int8 k-steps (16x16x64)
  constexpr int NDB = DP / 16;   // 16-wide d blocks of O^T
  constexpr int ROW16 = DP * 2;  // bytes per fp16 row
  constexpr int ROW8 = DP;       // bytes per int8 row
  constexpr int KBUF = 64 * ROW16;  // K stage (fp16 or int8)
  constexpr int VBUF = 64 * ROW16;  // V stage (fp16; int8 V codes are widened into it)
  constexpr int STAGE = KBUF + VBUF;
  // int8 V codes land in the half of the K slot an int8 K tile leaves free.
  constexpr int V8OFF = 64 * ROW8;
  // 1 KB wave loads per tile, and how many each wave issues.
  constexpr int K16_T = 64 * ROW16 / 1024, K8_T = 64 * ROW8 / 1024;
  constexpr int K16_I = (K16_T + NW - 1) / NW, K8_I = (K8_T + NW - 1) / NW;
  static_assert(KS8 >= 1 && DP % 64 == 0, "head_dim tile must be 64 or 128");

  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar control flow)
  const int li = lane & 15;  // query row within the wave
  const int lg = lane >> 4;  // key group

  // ---- work item ---------------------------------------------------------
  const int bid = blockIdx.x;
  const int lam = work_item(bid, a.total_items, a.m_blocks * a.group, a.ilv);
  if (lam < 0) return;
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

  const int row0w = m * BM + wave * 16;  // first row of this wave
  const int row = row0w + li;             // this lane's query row
  const bool row_ok = row < Lq;

  // ---- Q fragments (B operand of S^T = K . Q^T) --------------------------
  f16x8 qf[KS16];
  i32x4 q8f[KS8];
  f16 sq16 = (f16)1.0f;
  if (MODE != TILEMIX_ROUTING_INT8) {
    const f16* qp = a.q + (int64_t)(q_start + row) * a.sq_t + (int64_t)h * a.sq_h;
#pragma unroll
    for (int s = 0; s < KS16; ++s) {
      const int d0 = 32 * s + 8 * lg;
      f16x8 raw = {};
      if (row_ok && d0 < a.d) raw = *reinterpret_cast<const f16x8*>(qp + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = (f16)fp32_round((float)raw[e] * a.qk_scale);
    }
  }
  if (MODE != TILEMIX_ROUTING_FP16) {
    const int8_t* qp = a.q8 + (int64_t)(q_start + row) * a.sq8_t + (int64_t)h * a.sq8_h;
#pragma unroll
    for (int s = 0; s < KS8; ++s) {
      const int d0 = 64 * s + 16 * lg;
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

  auto route_of = [&](int n) -> int {
    if (MODE == TILEMIX_ROUTING_FP16) return 0;
    if (MODE == TILEMIX_ROUTING_INT8) return 1;
    return (int)((bits >> (unsigned)(n / a.mask_tiles)) & 1ull);
  };
  // K (and int8 V) scales of tile n (reference :380-390: clamped block
  // index of each key), fp16, fetched with the tile's copy: one per tile, or
  // (GEN) one per 4-key group of the lane, exact for BLKK divisible by 4.
  auto load_scales = [&](const f16* sc, const int32_t* cus, int n, f16 (&out)[NSG]) {
    const int base = cus[z], end = cus[z + 1];
#pragma unroll
    for (int kb = 0; kb < NSG; ++kb) {
      f16 s = (f16)1.0f;
      if (end > base) {
        const int key = n * kBN + (GEN ? 16 * kb + 4 * lg : 0);
        const int idx = min(base + key / a.blkk, end - 1);
        s = sc[(int64_t)idx * a.hk + hk];
      }
      out[kb] = s;
    }
  };

  // ---- asynchronous tile loads (HBM -> LDS, no registers) -----------------
  // Each stream is one raw buffer over the sequence's keys (built once per
  // item); a tile adds its byte offset to the lane offsets, and rows past the
  // end read as 0 (finite bytes for masked keys, which contribute exactly 0
  // through p = 0).  The host keeps (max_seqlen_k + 64) * token stride below
  // 2^31 bytes, so the sums stay below 2^31 and a padded-column lane's offset
  // (kOffOutside + tile offset) below 2^32.
  const int64_t kt_bytes = a.sk_t * 2, vt_bytes = a.sv_t * 2;
  const int64_t k8t_bytes = a.sk8_t, v8t_bytes = a.sv8_t;
  const unsigned char* kseq = reinterpret_cast<const unsigned char*>(a.k + (int64_t)k_start * a.sk_t + (int64_t)hk * a.sk_h);
  const unsigned char* vseq = reinterpret_cast<const unsigned char*>(a.v + (int64_t)k_start * a.sv_t + (int64_t)hk * a.sv_h);
  const unsigned char* k8seq = MODE != TILEMIX_ROUTING_FP16
      ? reinterpret_cast<const unsigned char*>(a.k8 + (int64_t)k_start * a.sk8_t + (int64_t)hk * a.sk8_h) : nullptr;
  const unsigned char* v8seq = INT8V
      ? reinterpret_cast<const unsigned char*>(a.v8 + (int64_t)k_start * a.sv8_t + (int64_t)hk * a.sv8_h) : nullptr;
  // 0 = K (fp16 or int8) and int8 V codes, 1 = V fp16.
  // A lane whose 16-byte row chunk lies at or past head_dim gets an offset
  // beyond every buffer's size: the copy writes zeros there and never reads a
  // byte outside [0, head_dim) of a row.
  auto lane_off = [&](int L, int rowb, int64_t tok_bytes, int kind) -> int {
    const int rpi = 1024 / rowb, cpr = rowb / 16;
    const int r = L * rpi + lane / cpr;
    int sw;
    if (kind == 1) sw = rowb == 256 ? swz_v<256>(r) : swz_v<128>(r);
    else sw = rowb == 256 ? swz_k<256>(r) : rowb == 128 ? swz_k<128>(r) : swz_k<64>(r);
    const int chunk = (lane % cpr) ^ sw;  // the row chunk this lane copies
    if (chunk * 16 >= (rowb == ROW16 ? 2 * a.d : a.d)) return kOffOutside;
    return (int)(r * tok_bytes) + chunk * 16;
  };
  // Copies are issued from inline assembly (async_load16_asm): the loop
  // orders them against its LDS reads itself (s_waitcnt + barrier per tile).
  const uint32_t smem_lds = lds_addr(smem);
  const SRsrc rs_k16 = make_srsrc(kseq, (int)(Lk * kt_bytes));
  const SRsrc rs_k8 = make_srsrc(k8seq, (int)(Lk * k8t_bytes));
  const SRsrc rs_v16 = make_srsrc(vseq, (int)(Lk * vt_bytes));
  const SRsrc rs_v8 = make_srsrc(v8seq, (int)(Lk * v8t_bytes));
  // with_v = false (a GEN max pass) copies the K tile only.
  auto issue_tile = [&](int n, int route, uint32_t stage, bool with_v) {
    const int key0 = n * kBN;
    if (route == 0) {
      const int toff = key0 * (int)kt_bytes;
#pragma unroll
      for (int i = 0; i < K16_I; ++i) {
        const int L = i * NW + wave;
        if (L < K16_T) async_load16_asm(rs_k16, lane_off(L, ROW16, kt_bytes, 0) + toff, stage + L * 1024);
      }
    } else {
      const int toff = key0 * (int)k8t_bytes;
#pragma unroll
      for (int i = 0; i < K8_I; ++i) {
        const int L = i * NW + wave;
        if (L < K8_T) async_load16_asm(rs_k8, lane_off(L, ROW8, k8t_bytes, 0) + toff, stage + L * 1024);
      }
    }
    const uint32_t vstage = stage + KBUF;
    if (!with_v) {
    } else if (!INT8V || route == 0) {
      const int toff = key0 * (int)vt_bytes;
#pragma unroll
      for (int i = 0; i < K16_I; ++i) {
        const int L = i * NW + wave;
        if (L < K16_T) async_load16_asm(rs_v16, lane_off(L, ROW16, vt_bytes, 1) + toff, vstage + L * 1024);
      }
    } else {
      const int toff = key0 * (int)v8t_bytes;
#pragma unroll
      for (int i = 0; i < K8_I; ++i) {
        const int L = i * NW + wave;
        if (L < K8_T) async_load16_asm(rs_v8, lane_off(L, ROW8, v8t_bytes, 0) + toff, stage + V8OFF + L * 1024);
      }
    }
  };

  // int8 V codes -> fp16 V tile (the layout of an fp16 V copy).  Each wave
  // widens exactly the 1 KB pieces it copied itself, so its own vmcnt wait is
  // enough; the tile's barrier then publishes the fp16 tile to every wave.
  auto widen_v8 = [&](unsigned char* stg) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    constexpr int rpi = 1024 / ROW8, cpr = ROW8 / 16;
#pragma unroll
    for (int i = 0; i < K8_I; ++i) {
      const int L = i * NW + wave;
      if (L < K8_T) {
        const int r = L * rpi + lane / cpr;               // key row of this lane's 16 codes
        const int cc = (lane % cpr) ^ swz_k<ROW8>(r);     // their 16-column chunk
        const i32x4 w = *reinterpret_cast<const i32x4*>(stg + V8OFF + L * 1024 + lane * 16);
        const f16x8 lo = int8x8_to_f16((i32x2){w[0], w[1]});
        const f16x8 hi8 = int8x8_to_f16((i32x2){w[2], w[3]});
        const int sv = swz_v<ROW16>(r);
        unsigned char* row = stg + KBUF + r * ROW16;
        *reinterpret_cast<f16x8*>(row + (((2 * cc) ^ sv) * 16)) = lo;
        *reinterpret_cast<f16x8*>(row + (((2 * cc + 1) ^ sv) * 16)) = hi8;
      }
    }
  };

  // ---- online softmax state -------------------------------------------------
  // m_i: running max of the row (identical on the row's 4 lanes).  l_part:
  // this lane's share of the row sum; every lane starts at 1.0 like the
  // reference's l: the first tile with a valid key has alpha = 0, and a row
  // with no valid key keeps acc = 0, so the start value never reaches out.
  float m_i = -INFINITY;
  float l_part = 1.0f;
  f32x4 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

  int route_next = 0;
  f16 sk_next[NSG], sv_next[NSG];
#pragma unroll
  for (int kb = 0; kb < NSG; ++kb) sk_next[kb] = sv_next[kb] = (f16)1.0f;
  // Route, scales and copies of tile n (with_v: also its V tile).
  auto fetch_issue = [&](int n, uint32_t stage, bool with_v) {
    route_next = route_of(n);
    if (MODE != TILEMIX_ROUTING_FP16 && route_next == 1) {
      load_scales(a.sk, a.cu_ks, n, sk_next);
      if (INT8V && with_v) load_scales(a.sv, a.cu_vs, n, sv_next);
    }
    issue_tile(n, route_next, stage, with_v);
  };

  // ---- GEN: steps over (tile, pass) ---------------------------------------
  // Group gs .. ge-1 of ng consecutive 64-key tiles is one block_n tile; with
  // more than one tile it is visited twice (pass 0: max, pass 1: update),
  // else once (pass 1).  The sequence ends when n reaches n_blocks.
  const int ng = GEN ? a.ng : 1;
  struct Step {
    int n, pass, gs, ge;
  };
  auto first_step = [&]() -> Step {
    const int ge = min(ng, n_blocks);
    return Step{0, ge > 1 ? 0 : 1, 0, ge};
  };
  auto next_step = [&](const Step& s) -> Step {
    if (s.n + 1 < s.ge) return Step{s.n + 1, s.pass, s.gs, s.ge};
    if (s.pass == 0) return Step{s.gs, 1, s.gs, s.ge};
    const int ge = min(s.ge + ng, n_blocks);
    return Step{s.ge, ge - s.ge > 1 ? 0 : 1, s.ge, ge};
  };

  if (n_blocks > 0) {
    if constexpr (GEN) fetch_issue(0, smem_lds, first_step().pass == 1);
    else fetch_issue(0, smem_lds, true);
  }

  // ---- S^T = K . Q^T of a staged tile, rounded to fp16 (packed pairs r, r+1)
  auto tile_scores = [&](const unsigned char* stage, int route, const f16 (&skc)[NSG], int key0,
                         uint32_t (&s16)[4][2]) {
    if (route == 0) {
      f32x4 c[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) c[kb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS16; ++ks)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int r = kb * 16 + li;
          const int ch = (4 * ks + lg) ^ swz_k<ROW16>(r);
          const f16x8 av = *reinterpret_cast<const f16x8*>(stage + r * ROW16 + ch * 16);
          c[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, qf[ks], c[kb], 0, 0, 0);
        }
      if (DUMP && a.dump_i32 != nullptr && row_ok) {
        // FP16 tiles: the raw fp32 accumulator (bit pattern) before fp16 rounding.
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = key0 + kb * 16 + 4 * lg + r;
            if (key < Lk)
              a.dump_i32[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = __float_as_int(c[kb][r]);
          }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        s16[kb][0] = pack_h2(c[kb][0], c[kb][1]);
        s16[kb][1] = pack_h2(c[kb][2], c[kb][3]);
      }
    } else {
      // acc is accumulated on top of the integer bits of 1.5*2^23, so
      // float(bits) = 1.5*2^23 + acc exactly (|acc| < 2^22); fma(F, ss,
      // -1.5*2^23*ss) is then the single rounding of acc*ss (1.5*2^23*ss is
      // exact: ss has 11 significant bits).
      constexpr float kMagic = 12582912.0f;
      float ss[NSG], negms[NSG];
#pragma unroll
      for (int kb = 0; kb < NSG; ++kb) {
        const f16 sqk = sq16 * skc[kb];
        ss[kb] = (float)(f16)fp32_round((float)sqk * a.qk_scale);
        negms[kb] = -kMagic * ss[kb];
      }
      const i32x4 magic = {0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
      i32x4 c[4];
#pragma unroll
      for (int ks = 0; ks < KS8; ++ks)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int r = kb * 16 + li;
          const int ch = (4 * ks + lg) ^ swz_k<ROW8>(r);
          const i32x4 av = *reinterpret_cast<const i32x4*>(stage + r * ROW8 + ch * 16);
          c[kb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, q8f[ks], ks == 0 ? magic : c[kb], 0, 0, 0);
        }
      if (DUMP && a.dump_i32 != nullptr && row_ok) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = key0 + kb * 16 + 4 * lg + r;
            if (key < Lk)
              a.dump_i32[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = c[kb][r] - 0x4B400000;
          }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int g = GEN ? kb : 0;
        s16[kb][0] = pack_h2(fp32_round(__builtin_fmaf(__int_as_float(c[kb][0]), ss[g], negms[g])),
                             fp32_round(__builtin_fmaf(__int_as_float(c[kb][1]), ss[g], negms[g])));
        s16[kb][1] = pack_h2(fp32_round(__builtin_fmaf(__int_as_float(c[kb][2]), ss[g], negms[g])),
                             fp32_round(__builtin_fmaf(__int_as_float(c[kb][3]), ss[g], negms[g])));
      }
    }
    if (DUMP && a.dump_f16 != nullptr && row_ok) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + kb * 16 + 4 * lg + r;
          const f16x2 pr = __builtin_bit_cast(f16x2, s16[kb][r >> 1]);
          if (key < Lk)
            a.dump_f16[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = pr[r & 1];
        }
    }
  };

  // ---- mask + optional bias ------------------------------------------------
  auto tile_mask = [&](int key0, uint32_t (&s16)[4][2]) {
    const bool need_mask = (key0 + kBN > Lk) || (a.causal && key0 + kBN - 1 > row0w + diag);
    if (need_mask || BIAS) {
      const int lim = a.causal ? min(Lk - 1, row + diag) : Lk - 1;  // last valid key
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f16x2 pr = __builtin_bit_cast(f16x2, s16[kb][j]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int key = key0 + kb * 16 + 4 * lg + 2 * j + e;
            if (key > lim) {
              pr[e] = (f16)(-INFINITY);
            } else if (BIAS && row_ok) {
              // Reference :264-272: qk(fp16) += fp16(b * LOG2E) with LOG2E taken
              // as an fp16 constant against the fp16 bias (weak scalar typing);
              // the bias row pointer carries no batch offset (quirk kept).
              const f16 b = a.bias[(int64_t)h * a.sb_h + (int64_t)row * a.sb_m + (int64_t)key * a.sb_n];
              const f16 bl = b * (f16)1.4426950408889634f;
              pr[e] = pr[e] + bl;
            }
          }
          s16[kb][j] = __builtin_bit_cast(uint32_t, pr);
        }
    }
  };

  // ---- the row maximum of a tile (the row's 4 lanes) -----------------------
  auto tile_max = [&](const uint32_t (&s16)[4][2]) -> float {
    uint32_t mx2 = pk_max(pk_max(pk_max(s16[0][0], s16[0][1]), pk_max(s16[1][0], s16[1][1])),
                          pk_max(pk_max(s16[2][0], s16[2][1]), pk_max(s16[3][0], s16[3][1])));
    const f16x2 mxh = __builtin_bit_cast(f16x2, mx2);
    float mx = fmaxf((float)mxh[0], (float)mxh[1]);
    const float2 p1 = pair16(mx);
    mx = fmaxf(p1.x, p1.y);
    const float2 p2 = pair32(mx);
    return fmaxf(p2.x, p2.y);
  };

  // ---- online softmax update (reference _softmax_prefix_update) ------------
  // m_next is the row's new maximum, alpha = exp2(m_i - m_next) (1 if the
  // step brings no valid key); p = fp16(exp2(s - m_next)), l and O are
  // rescaled by alpha, O^T += V^T . P^T.  svc: the tile's V scales (int8 V).
  auto tile_update = [&](const unsigned char* stage, int route, const f16 (&svc)[NSG],
                         const uint32_t (&s16)[4][2], float m_next, float alpha) {
    // With no valid key yet the tile is all -inf and p must be 0: subtract 0.
    const float negm = m_next == -INFINITY ? 0.0f : -m_next;
    uint32_t p16[4][2];
    float ls = 0.0f;
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float e0 = fast_exp2(sub_lo(s16[kb][j], negm));
        const float e1 = fast_exp2(sub_hi(s16[kb][j], negm));
        p16[kb][j] = pack_h2(e0, e1);
        ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p16[kb][j]), ones, ls, false);
      }
    l_part = l_part * alpha + ls;
    // alpha == 1 makes the reference's rescale an exact no-op, and so does a
    // row that has seen no valid key yet (acc is still 0): skip it when one of
    // the two holds for every row of the wave (always on a wave's first tile).
    const bool rescale_noop = alpha == 1.0f || m_i == -INFINITY;
    m_i = m_next;
    if (!__all(rescale_noop)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
    }

    if (INT8V && route == 1) {
      // Reference :449-497: PV on int8 V codes with p scaled by the V block
      // scale in fp16: p_scaled = fp16(p * sv) (l keeps the unscaled p).
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const f16 s = svc[GEN ? kb : 0];
        const f16x2 sv2 = {s, s};
#pragma unroll
        for (int j = 0; j < 2; ++j)
          p16[kb][j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, p16[kb][j]) * sv2);
      }
    }

    // ---- O^T += V^T . P^T ----------------------------------------------
    // k slot 8 lg + t  <->  key 32 ks + 4 lg + (t % 4) + 16 (t / 4).
    const unsigned char* vst = stage + KBUF;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      f16x8 pb;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const f16x2 pr = __builtin_bit_cast(f16x2, p16[2 * ks + hb][j]);
          pb[4 * hb + 2 * j] = pr[0];
          pb[4 * hb + 2 * j + 1] = pr[1];
        }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        // tr16: input lane li points at V[k0 + li/4][16 db + 4 (li%4)];
        // output lane li gets V[k0..k0+3][16 db + li] (int8 V codes were
        // widened to this fp16 layout at the tile's start).
        f16x8 av;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          const int vr = 32 * ks + 16 * hb + 4 * lg + (li >> 2);
          const int col = 16 * db + 4 * (li & 3);
          const int ch = (col >> 3) ^ swz_v<ROW16>(vr);
          const f16x4 v4 = lds_read_tr16(vst + vr * ROW16 + ch * 16 + (col & 7) * 2);
          av[4 * hb + 0] = v4[0];
          av[4 * hb + 1] = v4[1];
          av[4 * hb + 2] = v4[2];
          av[4 * hb + 3] = v4[3];
        }
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb, acc[db], 0, 0, 0);
      }
    }
  };

  // Tiles fully masked for this wave (or rows past the sequence end): the
  // reference's update is then an exact no-op (p = 0, alpha = 1), in either
  // pass of a GEN step.
  auto wave_skip = [&](int key0) { return (row0w >= Lq) || (a.causal && key0 > row0w + 15 + diag); };
  if constexpr (!GEN) {
    for (int n = 0; n < n_blocks; ++n) {
      const int route = route_next;
      const f16 skc[NSG] = {sk_next[0]};
      const f16 svc[NSG] = {sv_next[0]};
      unsigned char* stage = smem + (n & 1) * STAGE;
      // Tile n has landed (own loads), then every wave's loads have landed and
      // every wave is done with the other stage (tile n-1).
      __builtin_amdgcn_s_waitcnt(0);
      if (INT8V && route == 1) widen_v8(stage);
      __syncthreads();
      if (n + 1 < n_blocks) fetch_issue(n + 1, smem_lds + ((n + 1) & 1) * STAGE, true);

      const int key0 = n * kBN;
      if (wave_skip(key0)) continue;
      uint32_t s16[4][2];
      tile_scores(stage, route, skc, key0, s16);
      tile_mask(key0, s16);
      const float mx = tile_max(s16);
      const bool has = mx != -INFINITY;
      const float m_next = has ? fmaxf(m_i, mx) : m_i;
      const float alpha = has ? fast_exp2(m_i - m_next) : 1.0f;
      tile_update(stage, route, svc, s16, m_next, alpha);
    }
  } else {
    float gmx = -INFINITY;  // row maximum of the current group's max pass
    Step cur = first_step();
    for (int si = 0; cur.n < n_blocks; ++si) {
      const Step nxt = next_step(cur);
      const int route = route_next;
      f16 skc[NSG], svc[NSG];
#pragma unroll
      for (int kb = 0; kb < NSG; ++kb) {
        skc[kb] = sk_next[kb];
        svc[kb] = sv_next[kb];
      }
      unsigned char* stage = smem + (si & 1) * STAGE;
      __builtin_amdgcn_s_waitcnt(0);
      if (INT8V && route == 1 && cur.pass == 1) widen_v8(stage);
      __syncthreads();
      if (nxt.n < n_blocks) fetch_issue(nxt.n, smem_lds + ((si + 1) & 1) * STAGE, nxt.pass == 1);

      const int key0 = cur.n * kBN;
      if (!wave_skip(key0)) {
        uint32_t s16[4][2];
        tile_scores(stage, route, skc, key0, s16);
        tile_mask(key0, s16);
        const float mx = tile_max(s16);
        if (cur.pass == 0) {
          gmx = fmaxf(gmx, mx);
        } else {
          // The group's maximum enters at its first tile (alpha once per
          // block_n tile); later tiles of the group keep m (alpha = 1).
          float m_next = m_i, alpha = 1.0f;
          if (cur.n == cur.gs) {
            const float gm = fmaxf(gmx, mx);
            gmx = -INFINITY;
            if (gm != -INFINITY) {
              m_next = fmaxf(m_i, gm);
              alpha = fast_exp2(m_i - m_next);
            }
          }
          tile_update(stage, route, svc, s16, m_next, alpha);
        }
      }
      cur = nxt;
    }
  }

  // ---- epilogue: out = fp16(acc / l) --------------------------------------
  float l_i = l_part;
  {
    const float2 p1 = pair16(l_i);
    l_i = p1.x + p1.y;
    const float2 p2 = pair32(l_i);
    l_i = p2.x + p2.y;
  }
  if (row_ok) {
    f16* op = a.out + (int64_t)(q_start + row) * a.so_t + (int64_t)h * a.so_h;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d0 = 16 * db + 4 * lg;
      if (d0 < a.d) {
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (f16)(acc[db][e] / l_i);
        *reinterpret_cast<f16x4*>(op + d0) = o;
      }
    }
  }
}

}  // namespace tmx
