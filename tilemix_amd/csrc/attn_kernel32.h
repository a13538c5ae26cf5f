// Fused FP16/INT8-routed flash-attention prefill forward for gfx950: the
// 32-row kernel (4 waves x 32 query rows = 128 rows per workgroup).  It runs
// block_m = 128; block_m = 256 and 512 as 128-row workgroups that read their
// block's routing row; and, with SPLIT, block_m = 64: the workgroup's two
// 64-row halves are two routing blocks, and a key tile whose route differs
// between the halves is staged in both K formats.
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
// The kernel computes in 64-key tiles.  GEN instantiations serve the other
// launch shapes of the reference:
//   * block_n = 64 * ng (ng = 2, 4): the reference's online-softmax step covers
//     block_n keys, m' = max(m, max over the block_n keys) and p = fp16(exp2(s
//     - m')) (:179-207).  Each block_n tile is streamed twice, 64 keys at a
//     time: a max pass (K only: scores, mask, row maximum) and an update pass
//     (scores again, p against that maximum, one rescale per block_n tile, PV);
//   * K/V scale blocks (BLKK) that are not multiples of 64: the scale is
//     looked up per 4-key group of a lane, sk[key // BLKK] (:390,485), which is
//     exact for every BLKK divisible by 4 (no scale block starts inside a
//     4-aligned group of keys).
//
// Work decomposition (MI355X-first, not the reference's):
//   * one workgroup = one (sequence, query head, block_m query rows);
//     NW = block_m/32 waves, each wave owns 32 query rows;
//   * every wave computes S^T = K . Q^T with 32x32 MFMAs, so a lane owns ONE
//     query row: row max / row sum are in-lane reductions plus one
//     v_permlane32_swap, and the per-row rescale of O is a per-lane scalar;
//   * O^T = V^T . P^T uses the S^T register layout directly as the B operand;
//     the A operand (V^T) is read from row-major V with ds_read_b64_tr_b16;
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
#include "attn_pipe_asm.h"

namespace tmx {

template <int NW, int DP, int MODE, bool INT8V, bool DUMP, bool BIAS, bool SPLIT, bool GEN, bool PIPE = false>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn32_kernel(const AttnKArgs a) {
  static_assert(!SPLIT || (NW % 2 == 0 && !INT8V), "split workgroups: even wave count, fp16 V");
  static_assert(!PIPE || (NW == 4 && DP == 128 && !INT8V && !DUMP && !BIAS && !GEN),
                "the pipelined tile body serves the plain and split 4-wave head_dim-128 launches");
  constexpr int BM = NW * 32;
  // K/V scales per tile and lane: one, or (GEN) one per 4-key group g = 4 kb + jj
  // of the lane's keys 32 kb + 8 jj + 4 hi .. + 3.
  constexpr int NSG = GEN ? 8 : 1;
  constexpr int KS16 = DP / 16;  // fp16 MFMA k-steps (32x32x16)
  constexpr int KS8 = DP / 32;   // int8 MFMA k-steps (32x32x32)
  constexpr int NDB = DP / 32;   // 32-wide d blocks of O^T
  constexpr int ROW16 = DP * 2;  // bytes per fp16 row
  constexpr int ROW8 = DP;       // bytes per int8 row
  constexpr int KBUF = 64 * ROW16;               // K stage (fp16 or int8)
  constexpr int VBUF = 64 * ROW16;               // V stage (fp16; int8 V codes are widened into it)
  // A split stage holds K in both formats (int8 K after V); otherwise an
  // int8 K tile takes the fp16 K slot.
  constexpr int K8OFF = SPLIT ? KBUF + VBUF : 0;
  // int8 V codes land in the half of the K slot an int8 K tile leaves free and
  // are widened to fp16 into the V slot before the tile's barrier.
  constexpr int V8OFF = 64 * ROW8;
  constexpr int STAGE = KBUF + VBUF + (SPLIT ? 64 * ROW8 : 0);
  constexpr int K16_INS = KBUF / 1024 / NW;      // 1 KB wave loads per wave per tile
  constexpr int K8_INS = (64 * ROW8) / 1024 / NW;
  constexpr int V16_INS = VBUF / 1024 / NW;
  constexpr int V8_INS = (64 * ROW8) / 1024 / NW;
  static_assert(K16_INS >= 1 && K8_INS >= 1 && V16_INS >= 1 && V8_INS >= 1, "tile split");

  // The Q block (128 rows) is staged through stage 1 in the prologue (that
  // stage is first written by tile 1's copy, after the loop's first barrier).
  // It fills a plain stage; a split stage has room after it.
  constexpr int QBYTES = BM * ROW16;
  static_assert(QBYTES <= STAGE, "Q block fits a stage");
  constexpr int QRED_EXTRA = QBYTES + 4 * NW <= STAGE ? 0 : 4 * NW;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * STAGE + QRED_EXTRA];
  // Per-wave partial max of the in-kernel Q quantisation: after the Q block in
  // stage 1 when it fits (split: a separate array would push the DP=128
  // workgroup past 80 KB and halve the workgroups per CU), else after stage 1.
  float* const q_red = reinterpret_cast<float*>(smem + (QRED_EXTRA ? 2 * STAGE : 2 * STAGE - 4 * NW));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;

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

  // Route bits of the workgroup's rows (SPLIT: bits of the low half, bits_hi
  // of the high half; a high half past the sequence end takes the low half's).
  uint64_t bits = 0, bits_hi = 0;
  if (MODE == TILEMIX_ROUTING_MIXED) {
    // Rows per routing block: BM / 2 (SPLIT), else block_m = BM << route_shift.
    // block_m 256 / 512 run as BM-row workgroups that share a routing row: a
    // row's result depends only on its own route bits and causal range (the
    // reference's extra tiles of a larger block are fully masked for it).
    constexpr int LOG_BM = __builtin_ctz(BM);
    const int rb_log = SPLIT ? LOG_BM - 1 : LOG_BM + a.route_shift;
    const int mbz = (Lq + (1 << rb_log) - 1) >> rb_log;  // per-sequence m_blocks (reference :819-820)
    const int mb = SPLIT ? 2 * m : m >> a.route_shift;
    bits = a.bitmask[hk * mbz + mb];
    if (SPLIT) bits_hi = mb + 1 < mbz ? a.bitmask[hk * mbz + mb + 1] : bits;
  }
  // Last key any row of the low half attends to: later tiles need only the
  // high half's format.
  const int lo_last_key = a.causal ? m * BM + BM / 2 - 1 + Lk - Lq : Lk;

  const int row0w = m * BM + wave * 32;  // first row of this wave
  const int row = row0w + l32;            // this lane's query row
  const bool row_ok = row < Lq;

  // ---- asynchronous tile loads (HBM -> LDS, no registers) -----------------
  // Each stream is one raw buffer over the sequence's keys (built once per
  // item); a tile adds its byte offset to the lane offsets, and rows past the
  // end read as 0 (finite bytes for masked keys, which contribute exactly 0
  // through p = 0).  Per-lane offsets are loop-invariant.  The
  // swizzle of a copied row depends only on its index mod 16, and the rows of
  // copy i are those of copy 0 plus i * NW * rows-per-copy (a multiple of 16),
  // so one lane offset per stream serves every copy of a tile.
  const int64_t kt_bytes = a.sk_t * 2, vt_bytes = a.sv_t * 2;
  const int64_t k8t_bytes = a.sk8_t, v8t_bytes = a.sv8_t;
  const unsigned char* kseq = reinterpret_cast<const unsigned char*>(a.k + (int64_t)k_start * a.sk_t + (int64_t)hk * a.sk_h);
  const unsigned char* vseq = reinterpret_cast<const unsigned char*>(a.v + (int64_t)k_start * a.sv_t + (int64_t)hk * a.sv_h);
  const unsigned char* k8seq = MODE != TILEMIX_ROUTING_FP16
      ? reinterpret_cast<const unsigned char*>(a.k8 + (int64_t)k_start * a.sk8_t + (int64_t)hk * a.sk8_h) : nullptr;
  const unsigned char* v8seq = INT8V
      ? reinterpret_cast<const unsigned char*>(a.v8 + (int64_t)k_start * a.sv8_t + (int64_t)hk * a.sv8_h) : nullptr;
  // A lane whose 16-byte row chunk lies at or past head_dim (columns the
  // padded tile width adds) gets an offset beyond every buffer's size, so the
  // copy writes zeros there: no byte outside [0, head_dim) of a row is ever
  // read, and the padded columns are finite (0 * x = 0 in the MFMAs).  The
  // swizzle of copy i's rows is that of copy 0's, so the chunk is per lane.
  auto lane_off0 = [&](int rowb, int64_t tok_bytes, bool vswz, int valid_bytes) -> int {
    const int rpi = 1024 / rowb, cpr = rowb / 16;
    const int r = wave * rpi + lane / cpr;
    int sw;
    if (rowb == 256) sw = vswz ? swz_v32<256>(r) : swz_k<256>(r);
    else if (rowb == 128) sw = vswz ? swz_v32<128>(r) : swz_k<128>(r);
    else sw = swz_k<64>(r);
    const int chunk = (lane % cpr) ^ sw;  // the row chunk this lane copies
    if (chunk * 16 >= valid_bytes) return kOffOutside;
    return (int)(r * tok_bytes) + chunk * 16;
  };
  const int dma_k16 = lane_off0(ROW16, kt_bytes, false, 2 * a.d);
  const int dma_k8 = MODE != TILEMIX_ROUTING_FP16 ? lane_off0(ROW8, k8t_bytes, false, a.d) : 0;
  const int dma_v16 = lane_off0(ROW16, vt_bytes, true, 2 * a.d);
  const int dma_v8 = INT8V ? lane_off0(ROW8, v8t_bytes, false, a.d) : 0;
  const int step_k16 = NW * (1024 / ROW16) * (int)kt_bytes;
  const int step_k8 = NW * (1024 / ROW8) * (int)k8t_bytes;
  const int step_v16 = NW * (1024 / ROW16) * (int)vt_bytes;
  const int step_v8 = NW * (1024 / ROW8) * (int)v8t_bytes;
  const uint32_t smem_lds = lds_addr(smem);
  // route: 0 fp16 / 1 int8; SPLIT: bit 0 the low half's route, bit 1 the high half's.
  // Byte offset of the next tile in each stream, advanced by one tile per
  // issue (tiles are issued in order, one per call; GEN steps set it from the
  // tile index): one scalar add per stream and tile, the buffer descriptors
  // stay fixed.
  const SRsrc rs_k16 = make_srsrc(kseq, (int)(Lk * kt_bytes));
  const SRsrc rs_k8 = make_srsrc(k8seq, (int)(Lk * k8t_bytes));
  const SRsrc rs_v16 = make_srsrc(vseq, (int)(Lk * vt_bytes));
  const SRsrc rs_v8 = make_srsrc(v8seq, (int)(Lk * v8t_bytes));
  int toff_k16 = 0, toff_k8 = 0, toff_v16 = 0, toff_v8 = 0;
  const int tstep_k16 = kBN * (int)kt_bytes, tstep_k8 = kBN * (int)k8t_bytes;
  const int tstep_v16 = kBN * (int)vt_bytes, tstep_v8 = kBN * (int)v8t_bytes;
  // K part of a tile copy (the format(s) of the tile's route) into stage's K slot.
  auto issue_k = [&](int route, uint32_t stage) {
    const bool need16 = MODE != TILEMIX_ROUTING_INT8 && (SPLIT ? route != 3 : route == 0);
    const bool need8 = MODE != TILEMIX_ROUTING_FP16 && route != 0;
    if (need16) {
      const SRsrc rs = rs_k16;
      // Opaque copy of the lane offset: the per-copy sums are formed here, one
      // add each, instead of being hoisted into loop-invariant VGPRs (the
      // same for the LDS read bases below).
      int o = dma_k16 + toff_k16;
      asm volatile("" : "+v"(o));
#pragma unroll
      for (int i = 0; i < K16_INS; ++i)
        async_load16_asm(rs, o + i * step_k16, stage + (i * NW + wave) * 1024);
    }
    if (need8) {
      const SRsrc rs = rs_k8;
      int o = dma_k8 + toff_k8;
      asm volatile("" : "+v"(o));
#pragma unroll
      for (int i = 0; i < K8_INS; ++i)
        async_load16_asm(rs, o + i * step_k8, stage + K8OFF + (i * NW + wave) * 1024);
    }
    toff_k16 += tstep_k16;
    if (MODE != TILEMIX_ROUTING_FP16) toff_k8 += tstep_k8;
  };
  // V part of a tile copy into stage's V slot (int8 V codes: the free half of the K slot).
  auto issue_v = [&](int route, uint32_t stage) {
    const uint32_t vstage = stage + KBUF;
    if (!INT8V || route == 0) {
      const SRsrc rs = rs_v16;
      int o = dma_v16 + toff_v16;
      asm volatile("" : "+v"(o));
#pragma unroll
      for (int i = 0; i < V16_INS; ++i)
        async_load16_asm(rs, o + i * step_v16, vstage + (i * NW + wave) * 1024);
    } else {
      const SRsrc rs = rs_v8;
      int o = dma_v8 + toff_v8;
      asm volatile("" : "+v"(o));
#pragma unroll
      for (int i = 0; i < V8_INS; ++i)
        async_load16_asm(rs, o + i * step_v8, stage + V8OFF + (i * NW + wave) * 1024);
    }
    toff_v16 += tstep_v16;
    if (INT8V) toff_v8 += tstep_v8;
  };
  // with_v = false (a GEN max pass) copies the K tile only.
  auto issue_tile = [&](int route, uint32_t stage, bool with_v) {
    issue_k(route, stage);
    if (with_v) issue_v(route, stage);
  };

  // int8 V codes -> fp16 V tile (the layout of an fp16 V copy).  Each wave
  // widens exactly the 1 KB pieces it copied itself, so its own vmcnt wait is
  // enough; the tile's barrier then publishes the fp16 tile to every wave.
  // One conversion per code and workgroup, instead of one per code and wave
  // in the PV loop.
  auto widen_v8 = [&](unsigned char* stg) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    constexpr int rpi = 1024 / ROW8, cpr = ROW8 / 16;
#pragma unroll
    for (int i = 0; i < V8_INS; ++i) {
      const int r = (i * NW + wave) * rpi + lane / cpr;  // key row of this lane's 16 codes
      const int cc = (lane % cpr) ^ swz_k<ROW8>(r);      // their 16-column chunk
      const i32x4 w = *reinterpret_cast<const i32x4*>(stg + V8OFF + (i * NW + wave) * 1024 + lane * 16);
      const f16x8 lo = int8x8_to_f16((i32x2){w[0], w[1]});
      const f16x8 hi8 = int8x8_to_f16((i32x2){w[2], w[3]});
      const int sv = swz_v32<ROW16>(r);
      unsigned char* row = stg + KBUF + r * ROW16;
      *reinterpret_cast<f16x8*>(row + (((2 * cc) ^ sv) * 16)) = lo;
      *reinterpret_cast<f16x8*>(row + (((2 * cc + 1) ^ sv) * 16)) = hi8;
    }
  };

  // Per-tile route bit and K/V scale block, advanced tile by tile (no
  // divisions in the loop): tile t has route group t / mask_tiles and scale
  // block key0 / blkk = t / (blkk / 64).
  const int kb_tiles = a.blkk / kBN;
  int nx_grp = 0, nx_gc = 0, nx_sc = 0;  // of the next tile to issue
  // Scale of the next tile's block (clamped at the sequence's last block, the
  // reference's min(block, last) lookup), advanced by pointer.
  bool has_ks = false, has_vs = false;
  const f16 *skp = nullptr, *sk_last = nullptr, *svp = nullptr, *sv_last = nullptr;
  int ks_base = 0, ks_end = 0, vs_base = 0, vs_end = 0;
  if (MODE != TILEMIX_ROUTING_FP16) {
    ks_base = a.cu_ks[z];
    ks_end = a.cu_ks[z + 1];
    has_ks = ks_end > ks_base;
    skp = a.sk + (int64_t)ks_base * a.hk + hk;
    sk_last = a.sk + (int64_t)(ks_end - 1) * a.hk + hk;
  }
  if (INT8V) {
    vs_base = a.cu_vs[z];
    vs_end = a.cu_vs[z + 1];
    has_vs = vs_end > vs_base;
    svp = a.sv + (int64_t)vs_base * a.hk + hk;
    sv_last = a.sv + (int64_t)(vs_end - 1) * a.hk + hk;
  }
  // Route of tile nx in route group grp (0 fp16 / 1 int8; SPLIT: two bits).
  auto tile_route = [&](int nx, int grp) -> int {
    if (MODE == TILEMIX_ROUTING_FP16) return 0;
    if (MODE == TILEMIX_ROUTING_INT8) return SPLIT ? 3 : 1;
    if (!SPLIT) return (int)((bits >> (unsigned)grp) & 1ull);
    const int rhi = (int)((bits_hi >> (unsigned)grp) & 1ull);
    const int rlo = nx * kBN > lo_last_key ? rhi : (int)((bits >> (unsigned)grp) & 1ull);
    return rlo | (rhi << 1);
  };
  // Issues the next tile (index nx) and fetches its scales; the loads land
  // before the barrier that precedes the tile's compute.
  // The K part (with the K scale and the route/scale bookkeeping) and the V
  // part can go out at different times (the pipelined loop copies K a tile
  // ahead of V); issue_next issues both.
  auto issue_next_k = [&](int nx, uint32_t stage, int& route, f16 (&skv)[NSG], f16 (&svv)[NSG]) {
    route = tile_route(nx, nx_grp);
    issue_k(route, stage);
    if (MODE != TILEMIX_ROUTING_FP16 && route != 0) {
      skv[0] = has_ks ? *skp : (f16)1.0f;
      if (INT8V) svv[0] = has_vs ? *svp : (f16)1.0f;
    }
    if (++nx_gc == a.mask_tiles) {
      nx_gc = 0;
      ++nx_grp;
    }
    if (++nx_sc == kb_tiles) {
      nx_sc = 0;
      if (MODE != TILEMIX_ROUTING_FP16 && skp != sk_last) skp += a.hk;
      if (INT8V && svp != sv_last) svp += a.hk;
    }
  };
  auto issue_next = [&](int nx, uint32_t stage, int& route, f16 (&skv)[NSG], f16 (&svv)[NSG]) {
    issue_next_k(nx, stage, route, skv, svv);
    issue_v(route, stage);
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
  // Scale of each of this lane's 4-key groups of tile n (the reference's
  // clamped per-key lookup, sk[min(base + key // BLKK, end - 1)]).
  auto group_scales = [&](int n, const f16* sh, int base, int end, bool has, f16 (&out)[NSG]) {
#pragma unroll
    for (int g = 0; g < NSG; ++g) {
      const unsigned key = (unsigned)(n * kBN + 32 * (g >> 2) + 8 * (g & 3) + 4 * hi);
      const int idx = min(base + (int)(key / (unsigned)a.blkk), end - 1);
      out[g] = has ? sh[(int64_t)idx * a.hk] : (f16)1.0f;
    }
  };
  // Issues step s's tile: the stream bases are set from the tile index (the
  // steps revisit tiles), and a max pass copies K only.
  auto issue_step = [&](const Step& s, uint32_t stage, int& route, f16 (&skv)[NSG], f16 (&svv)[NSG]) {
    route = tile_route(s.n, s.n / a.mask_tiles);
    toff_k16 = s.n * tstep_k16;
    toff_v16 = s.n * tstep_v16;
    if (MODE != TILEMIX_ROUTING_FP16) toff_k8 = s.n * tstep_k8;
    if (INT8V) toff_v8 = s.n * tstep_v8;
    issue_tile(route, stage, s.pass == 1);
    if (MODE != TILEMIX_ROUTING_FP16 && route != 0) {
      group_scales(s.n, a.sk + hk, ks_base, ks_end, has_ks, skv);
      if (INT8V && s.pass == 1) group_scales(s.n, a.sv + hk, vs_base, vs_end, has_vs, svv);
    }
  };

  // ---- Q block -> LDS stage 1 ----------------------------------------------
  // The fp16 Q rows (QK operand and the in-kernel quantisation's input) are
  // copied like a K tile: 1 KB per copy, 16 lanes per 256-byte row, the K
  // swizzle, zeros past the sequence end (buffer size) and past head_dim
  // (kOffOutside).  Wave w copies rows 32 w .. 32 w + 31 of the block, the rows
  // it reads back, so it needs no barrier.  (Loading the fragments straight
  // into registers touches 32 rows per load instruction.)  They go out before
  // the first tile's copies, so the two latencies overlap.
  const bool q_fused = MODE != TILEMIX_ROUTING_FP16 && a.q_fused;
  const bool q_lds = MODE != TILEMIX_ROUTING_INT8 || q_fused;
  if (q_lds) {
    constexpr int QRPI = 1024 / ROW16, QCPR = ROW16 / 16, QINS = 32 / QRPI;
    const int64_t qt_bytes = a.sq_t * 2;
    const unsigned char* qwave =
        reinterpret_cast<const unsigned char*>(a.q + (int64_t)(q_start + row0w) * a.sq_t + (int64_t)h * a.sq_h);
    // Sized to the rows this wave reads (at most 32): the host keeps 128 * Q
    // token stride below 2^31 bytes, so the size and every row offset stay
    // below 2^31 and a padded-column lane's kOffOutside lies past the end.
    const SRsrc rs = make_srsrc(qwave, row0w < Lq ? (int)(min(Lq - row0w, 32) * qt_bytes) : 0);
    const uint32_t qlds = smem_lds + STAGE + (uint32_t)(wave * 32 * ROW16);
#pragma unroll
    for (int i = 0; i < QINS; ++i) {
      const int rl = i * QRPI + lane / QCPR;  // row within the wave's 32
      const int chunk = (lane % QCPR) ^ swz_k<ROW16>(wave * 32 + rl);
      const int off = chunk * 16 >= 2 * a.d ? kOffOutside : (int)(rl * qt_bytes) + chunk * 16;
      async_load16_asm(rs, off, qlds + (uint32_t)(i * QRPI * ROW16));
    }
  }

  // The first tile's copies go out right behind the Q copies, before Q is
  // read back, so the two latencies overlap.
  int route_next = 0;
  f16 sk_next[NSG], sv_next[NSG];
#pragma unroll
  for (int g = 0; g < NSG; ++g) sk_next[g] = sv_next[g] = (f16)1.0f;
  if (n_blocks > 0) {
    if constexpr (GEN) issue_step(first_step(), smem_lds, route_next, sk_next, sv_next);
    else issue_next(0, smem_lds, route_next, sk_next, sv_next);
  }

  // ---- Q fragments (B operand of S^T = K . Q^T) --------------------------
  // Lane (row, hi) holds Q[row][16 s + 8 hi .. + 7] for the fp16 k-steps s and
  // Q8[row][32 s + 16 hi .. + 15] for the int8 k-steps.
  f16x8 qf[KS16];
  i32x4 q8f[KS8];
  f16 sq16 = (f16)1.0f;
  f16x8 qraw[KS16];
  if (q_lds) {
    // The wave's own Q rows, copied above in the K-tile layout: row r, k-step
    // s, half hi is logical chunk 2 s + hi of LDS row r (rows past the
    // sequence end and columns past head_dim are zeros).  Its own copies
    // only, so its own wait suffices.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int qbase = (wave * 32 + l32) * ROW16 + ((16 * hi) ^ (16 * swz_k<ROW16>(l32)));
    asm volatile("" : "+v"(qbase));
#pragma unroll
    for (int s = 0; s < KS16; ++s) qraw[s] = *reinterpret_cast<const f16x8*>(smem + STAGE + (qbase ^ (32 * s)));
  }
  if (MODE != TILEMIX_ROUTING_INT8) {
    // fp16(RN(q * qk_scale)): one v_fma_mix per value (the fp16 operand
    // converts exactly), then one packing conversion per pair.
#pragma unroll
    for (int s = 0; s < KS16; ++s) {
      const u32x4 w = __builtin_bit_cast(u32x4, qraw[s]);
      u32x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = pack_h2(mul_lo(w[r], a.qk_scale), mul_hi(w[r], a.qk_scale));
      qf[s] = __builtin_bit_cast(f16x8, o);
    }
  }
  if (q_fused) {
    // In-kernel Q quantisation (the workgroup's 128 rows are exactly one
    // BLKQ = 128 block of this head): scale = max|q| / 127 over the block's
    // rows inside the sequence, code = trunc(q / scale +- 0.5), the same
    // arithmetic as quant_per_block_int8 with sm_scale = 1.
    // max|q| of the lane's 64 values as packed fp16 (exact: the maximum of
    // magnitudes, sign bits cleared), then over the wave: lanes l ^ 32 and
    // l ^ 16 by permlane swaps, the rest of a 16-lane row by DPP moves.
    uint32_t hm = 0;
#pragma unroll
    for (int s = 0; s < KS16; ++s) {
      const u32x4 w = __builtin_bit_cast(u32x4, qraw[s]);
#pragma unroll
      for (int r = 0; r < 4; ++r) hm = pk_max(hm, w[r] & 0x7fff7fffu);
    }
    const f16x2 hv = __builtin_bit_cast(f16x2, hm);
    float am = fmaxf((float)hv[0], (float)hv[1]);
    {
      const float2 pr = swap_halves(am);
      am = fmaxf(pr.x, pr.y);
      const float2 pq = pair16(am);
      am = fmaxf(pq.x, pq.y);
    }
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x128, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x124, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x4e, 0xf, 0xf, false)));
    am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0xb1, 0xf, 0xf, false)));
    if (lane == 0) q_red[wave] = am;
    __syncthreads();
    am = q_red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) am = fmaxf(am, q_red[w]);
    const float qs = am / 127.0f;  // IEEE division
    const float qr = 1.0f / qs;    // IEEE reciprocal (inf when qs == 0: codes are 0 then)
    sq16 = (f16)qs;
    // fp16 layout -> int8 layout: lanes l and l+32 exchange one half of each
    // pair of fp16 k-steps (2 s, 2 s + 1), so each lane then holds
    // Q[row][32 s + 16 hi .. + 15] as (x, y) = 8 + 8 consecutive values.
#pragma unroll
    for (int s = 0; s < KS8; ++s) {
      u32x4 x = __builtin_bit_cast(u32x4, qraw[2 * s]);
      u32x4 y = __builtin_bit_cast(u32x4, qraw[2 * s + 1]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const auto sw = __builtin_amdgcn_permlane32_swap(x[r], y[r], false, false);
        x[r] = sw[0];
        y[r] = sw[1];
      }
      const f16x8 xv = __builtin_bit_cast(f16x8, x), yv = __builtin_bit_cast(f16x8, y);
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      const u32x4 xw = __builtin_bit_cast(u32x4, xv), yw = __builtin_bit_cast(u32x4, yv);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        // div_by_recip with q0 = RN(x r) straight from the fp16 operand
        const uint32_t h2 = e < 8 ? xw[(e & 7) >> 1] : yw[(e & 7) >> 1];
        const float x = (float)(e < 8 ? xv[e] : yv[e - 8]);
        const float q0 = (e & 1) ? mul_hi(h2, qr) : mul_lo(h2, qr);
        float t = __builtin_fmaf(__builtin_fmaf(-q0, qs, x), qr, q0);
        // t + (t >= 0 ? 0.5 : -0.5); they differ only at t = -0, where both
        // truncate to code 0
        t += __builtin_copysignf(0.5f, t);
        const int code = (qs == 0.0f) ? 0 : (int)t;
        w[e >> 2] |= (uint32_t)(code & 0xff) << (8 * (e & 3));
      }
      q8f[s] = (i32x4){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
  } else if (MODE != TILEMIX_ROUTING_FP16) {
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

  // ---- online softmax state (one query row per lane) ----------------------
  // l_i is this lane's share of the row sum; both lanes of a row start at
  // 1.0 like the reference's l: the first tile with a valid key has
  // alpha = 0, and a row with no valid key keeps acc = 0, so the start value
  // never reaches the output.
  float m_i = -INFINITY;
  float l_i = 1.0f;
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = (f32x16){};

  // The magic bias as the MFMA C operand of the first k-step of every INT8
  // tile, kept in VGPRs for the whole loop (the barrier stops the compiler from
  // rebuilding the 16 constants before every INT8 tile).  The int8-V variant
  // needs those 16 VGPRs for its V path: it accumulates from zero and adds the
  // bias bits to the int32 result instead (the same float bits).
  constexpr bool kMagicC = !INT8V;
  constexpr int kBiasAdd = kMagicC ? 0 : 0x4B400000;
  i32x16 magic_c;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    int mv = 0x4B400000;
    if (MODE != TILEMIX_ROUTING_FP16 && kMagicC) asm volatile("" : "+v"(mv));
    magic_c[e] = mv;
  }

  const int half = SPLIT && wave >= NW / 2 ? 1 : 0;
  // Start of tile n, for every wave: the tile has landed (own loads), then
  // every wave's loads have landed and every wave is done with the other
  // stage (tile n-1), so the next tile's copies may go out from here on
  // (tile_start issues them at once; the compute loop after the QK reads).
  auto tile_wait = [&](int n) {
    const int route = SPLIT ? (route_next >> half) & 1 : route_next;
    __builtin_amdgcn_s_waitcnt(0);
    if (INT8V && route == 1) widen_v8(smem + (n & 1) * STAGE);
    __syncthreads();
  };
  auto tile_start = [&](int n) {
    tile_wait(n);
    if (n + 1 < n_blocks)
      issue_next(n + 1, smem_lds + ((n + 1) & 1) * STAGE, route_next, sk_next, sv_next);
  };
  // GEN: the same for step cur (stage si & 1), issuing step nxt.
  auto step_start = [&](int si, const Step& cur, const Step& nxt) {
    const int route = SPLIT ? (route_next >> half) & 1 : route_next;
    __builtin_amdgcn_s_waitcnt(0);
    if (INT8V && route == 1 && cur.pass == 1) widen_v8(smem + (si & 1) * STAGE);
    __syncthreads();
    if (nxt.n < n_blocks) issue_step(nxt, smem_lds + ((si + 1) & 1) * STAGE, route_next, sk_next, sv_next);
  };
  // Tiles [n_wave, n_blocks) are fully masked for this wave's rows (causal),
  // or the wave's rows lie past the sequence end: the reference's update is
  // then an exact no-op (p = 0, alpha = 1), so the wave only keeps the
  // workgroup's barriers and copies going for them.  (A per-tile skip inside
  // the compute loop made the register allocator copy the 64 accumulator
  // VGPRs on every tile in some instantiations.)
  int n_wave = n_blocks;
  if (row0w >= Lq) n_wave = 0;
  else if (a.causal) n_wave = min(n_blocks, row0w + 31 + diag < 0 ? 0 : (row0w + 31 + diag) / kBN + 1);

  // ---- S^T = K . Q^T of a staged tile, rounded to fp16 (packed pairs r, r+1)
  auto tile_scores = [&](const unsigned char* stage, int route, const f16 (&skc)[NSG], int key0,
                         uint32_t (&s16)[2][8]) {
    if (route == 0) {
      int kbase16 = l32 * ROW16 + ((16 * hi) ^ (16 * swz_k<ROW16>(l32)));
      asm volatile("" : "+v"(kbase16));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 c = {};
#pragma unroll
        for (int ks = 0; ks < KS16; ++ks) {
          const f16x8 av = *reinterpret_cast<const f16x8*>(stage + (kbase16 ^ (32 * ks)) + kb * 32 * ROW16);
          c = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qf[ks], c, 0, 0, 0);
        }
        if (DUMP && a.dump_i32 != nullptr && row_ok) {
          // FP16 tiles: the raw fp32 accumulator (bit pattern) before fp16 rounding.
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int key = key0 + kb * 32 + 8 * (rr >> 2) + 4 * hi + (rr & 3);
            if (key < Lk)
              a.dump_i32[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] =
                  __float_as_int(c[rr]);
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s16[kb][j] = pack_h2(c[2 * j], c[2 * j + 1]);
      }
    } else {
      // ss is fp16-exact; the barrier keeps it an fp32 operand (v_fma_f32
      // below, not the slower mixed-precision form).
      // acc is accumulated on top of the integer bits of 1.5*2^23, so
      // float(bits) = 1.5*2^23 + acc exactly (|acc| < 2^22); fma(F, ss,
      // -1.5*2^23*ss) is then the single rounding of acc*ss (1.5*2^23*ss is
      // exact: ss has 11 significant bits).
      constexpr float kMagic = 12582912.0f;
      float ss[NSG], negms[NSG];
#pragma unroll
      for (int g = 0; g < NSG; ++g) {
        const f16 sqk = sq16 * skc[g];
        ss[g] = fp32_round((float)(f16)fp32_round((float)sqk * a.qk_scale));
        negms[g] = -kMagic * ss[g];
      }
      int kbase8 = l32 * ROW8 + ((16 * hi) ^ (16 * swz_k<ROW8>(l32)));
      asm volatile("" : "+v"(kbase8));
      // Chain kb = 0 first; its dequant FMAs then run while the MFMAs of
      // chain kb = 1 execute (the fences keep the compiler from interleaving
      // the two chains, which would finish both at once).
      auto qk8_chain = [&](int kb) -> i32x16 {
        i32x16 c;
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
          const i32x4 av = *reinterpret_cast<const i32x4*>(stage + K8OFF + (kbase8 ^ (32 * ks)) + kb * 32 * ROW8);
          c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, q8f[ks], ks == 0 ? (kMagicC ? magic_c : (i32x16){}) : c, 0, 0, 0);
        }
        return c;
      };
      auto dequant = [&](int kb, const i32x16& c) {
        if (DUMP && a.dump_i32 != nullptr && row_ok) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int key = key0 + kb * 32 + 8 * (rr >> 2) + 4 * hi + (rr & 3);
            if (key < Lk)
              a.dump_i32[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] =
                  c[rr] + kBiasAdd - 0x4B400000;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int g = GEN ? 4 * kb + (j >> 1) : 0;  // keys 2 j, 2 j + 1 of the lane's 16 in kb
          s16[kb][j] = pack_h2(fp32_round(__builtin_fmaf(__int_as_float(c[2 * j] + kBiasAdd), ss[g], negms[g])),
                               fp32_round(__builtin_fmaf(__int_as_float(c[2 * j + 1] + kBiasAdd), ss[g], negms[g])));
        }
      };
      const i32x16 c0 = qk8_chain(0);
      __builtin_amdgcn_sched_barrier(0);
      const i32x16 c1 = qk8_chain(1);
      dequant(0, c0);
      __builtin_amdgcn_sched_barrier(0);
      dequant(1, c1);
    }
    if (DUMP && a.dump_f16 != nullptr && row_ok) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
          const int key = key0 + kb * 32 + 8 * (rr >> 2) + 4 * hi + (rr & 3);
          const f16x2 pr = __builtin_bit_cast(f16x2, s16[kb][rr >> 1]);
          if (key < Lk)
            a.dump_f16[(int64_t)(q_start + row) * a.dump_t + (int64_t)h * a.dump_h + key] = pr[rr & 1];
        }
    }
  };

  // ---- mask + optional bias ------------------------------------------------
  auto tile_mask = [&](int key0, uint32_t (&s16)[2][8]) {
    const bool need_mask = (key0 + kBN > Lk) || (a.causal && key0 + kBN - 1 > row0w + diag);
    if (need_mask || BIAS) {
      const int lim = a.causal ? min(Lk - 1, row + diag) : Lk - 1;  // last valid key
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          f16x2 pr = __builtin_bit_cast(f16x2, s16[kb][j]);
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int rr = 2 * j + e;
            const int key = key0 + kb * 32 + 8 * (rr >> 2) + 4 * hi + (rr & 3);
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

  // ---- the row maximum of a tile (both lanes of the row) -------------------
  auto tile_max = [&](const uint32_t (&s16)[2][8]) -> float {
    // 16 packed pairs -> 1 in 8 three-input maxima.
    const uint32_t u0 = pk_max3(s16[0][0], s16[0][1], s16[0][2]), u1 = pk_max3(s16[0][3], s16[0][4], s16[0][5]);
    const uint32_t u2 = pk_max3(s16[0][6], s16[0][7], s16[1][0]), u3 = pk_max3(s16[1][1], s16[1][2], s16[1][3]);
    const uint32_t u4 = pk_max3(s16[1][4], s16[1][5], s16[1][6]);
    const f16x2 mx2 = __builtin_bit_cast(f16x2, pk_max(pk_max3(u0, u1, u2), pk_max3(u3, u4, s16[1][7])));
    const float mx = fmaxf((float)mx2[0], (float)mx2[1]);
    const float2 sw = swap_halves(mx);
    return fmaxf(sw.x, sw.y);
  };

  // ---- online softmax update (reference _softmax_prefix_update) ------------
  // m_next is the row's new maximum, alpha = exp2(m_i - m_next) (1 if the
  // step brings no valid key); p = fp16(exp2(s - m_next)), l and O are
  // rescaled by alpha, O^T += V^T . P^T.  svc: the tile's V scales (int8 V).
  auto tile_update = [&](const unsigned char* stage, int route, const f16 (&svc)[NSG],
                         const uint32_t (&s16)[2][8], float m_next, float alpha) {
    // With no valid key yet the tile is all -inf and p must be 0: subtract 0.
    const float negm = m_next == -INFINITY ? 0.0f : -m_next;
    // P^T as the B operands of the PV MFMAs: pv[ks] holds keys 16 ks .. 16 ks + 15
    // of this lane's slots (pairs (kb, j) with ks = 2 kb + j / 4).
    u32x4 pv[4];
    float ls = 0.0f;
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e0 = fast_exp2(sub_lo(s16[kb][j], negm));
        const float e1 = fast_exp2(sub_hi(s16[kb][j], negm));
        const uint32_t pp = pack_h2(e0, e1);
        pv[2 * kb + (j >> 2)][j & 3] = pp;
        ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pp), ones, ls, false);
      }
    // Per-lane share of the row sum (the row's two lanes are combined at the end).
    l_i = l_i * alpha + ls;
    m_i = m_next;
    // The rescale runs on every tile (alpha == 1 is an exact no-op). Skipping
    // it when alpha == 1 on every row of the wave (a third of the tiles) made
    // the register allocator copy the 64 accumulator VGPRs between the two
    // paths on every tile, which cost more than the multiplies it saved.
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) acc[db][rr] *= alpha;

    if (INT8V && route == 1) {
      // Reference :449-497: PV on int8 V codes with p scaled by the V block
      // scale in fp16: p_scaled = fp16(p * sv).  GEN: elements 0-3 of pv[ks]
      // are keys of the lane's group 2 ks, elements 4-7 of group 2 ks + 1.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16 s0 = svc[GEN ? 2 * ks : 0], s1 = svc[GEN ? 2 * ks + 1 : 0];
        const f16x8 sv8 = {s0, s0, s0, s0, s1, s1, s1, s1};
        pv[ks] = __builtin_bit_cast(u32x4, __builtin_bit_cast(f16x8, pv[ks]) * sv8);
      }
    }

    // ---- O^T += V^T . P^T ----------------------------------------------
    const unsigned char* vst = stage + KBUF;
    const int j16 = lane & 15;
    const int g16 = (lane >> 4) & 1;
    const int vrl = 4 * hi + (j16 >> 2);
    int vbase = vrl * ROW16 + (((16 * (2 * g16 + ((j16 & 3) >> 1))) ^ (16 * swz_v32<ROW16>(vrl))) | (8 * (j16 & 1)));
    asm volatile("" : "+v"(vbase));
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // ds_read_b64_tr_b16: in a 16-lane group, input lane j points at
        // V[k0 + j/4][D0 + 4 (j%4)]; output lane i gets V[k0..k0+3][D0 + i]
        // (int8 V codes were widened to this fp16 layout at the tile's start).
        f16x8 av;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const unsigned char* p = vst + (vbase ^ (64 * db)) + (16 * ks + 8 * h2) * ROW16;
          const f16x4 v4 = lds_read_tr16(p);
          av[4 * h2 + 0] = v4[0];
          av[4 * h2 + 1] = v4[1];
          av[4 * h2 + 2] = v4[2];
          av[4 * h2 + 3] = v4[3];
        }
        const f16x8 pb = __builtin_bit_cast(f16x8, pv[ks]);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pb, acc[db], 0, 0, 0);
      }
    }
  };

  // ---- software-pipelined loop (PIPE) -------------------------------------
  // Tiles [0, n_sw) need no mask for any row of the workgroup (every key below
  // Lk and, causal, at or below the first row's diagonal).  They run through
  // the assembly tile body of attn_pipe_asm.h: iteration n computes tile n's
  // softmax and PV beside tile n+1's QK, conversion and row maximum.  K is
  // copied a tile ahead of V: iteration n issues K(n+2) into tile n's K slot
  // and V(n+1) into tile n-1's V slot, both free after the iteration's
  // barrier.  The remaining tiles (the causal diagonal, a ragged end) continue
  // through the C++ body below, with K(n_sw) and V(n_sw) already in flight.
  int n_sw = 0;
  if constexpr (PIPE) {
    int nf = Lk / kBN;
    if (a.causal) {
      const int lim = m * BM + diag + 1;  // keys below lim are valid for every row of the workgroup
      nf = min(nf, lim <= 0 ? 0 : lim / kBN);
    }
    n_sw = max(0, min(nf, n_blocks));
  }
  if constexpr (PIPE) {
    if (n_sw > 0) {
      PipeState st;
#pragma unroll
      for (int db = 0; db < NDB; ++db) st.acc[db] = acc[db];
      st.s16 = (u32x16){};
      st.mn = m_i;
      st.al = 1.0f;
      st.ng = 0.0f;
      st.li = l_i;
      PipeOps po;
      const int kb16 = l32 * ROW16 + ((16 * hi) ^ (16 * swz_k<ROW16>(l32)));
      const int kb8 = l32 * ROW8 + ((16 * hi) ^ (16 * swz_k<ROW8>(l32)));
      const int j16 = lane & 15, g16 = (lane >> 4) & 1, vrl = 4 * hi + (j16 >> 2);
      const int vb = vrl * ROW16 +
                     (((16 * (2 * g16 + ((j16 & 3) >> 1))) ^ (16 * swz_v32<ROW16>(vrl))) | (8 * (j16 & 1)));
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) po.ka[ks] = (int)smem_lds + (kb16 ^ (32 * ks));
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) po.k8a[ks] = (int)smem_lds + K8OFF + (kb8 ^ (32 * ks));
#pragma unroll
      for (int db = 0; db < 4; ++db) po.va[db] = (int)smem_lds + KBUF + (vb ^ (64 * db));
      if constexpr (MODE != TILEMIX_ROUTING_INT8) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) po.qf[ks] = qf[ks];
      }
      if constexpr (MODE != TILEMIX_ROUTING_FP16) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) po.q8f[ks] = q8f[ks];
      }
      po.fmax = 3.40282347e38f;

      PipeCopy c;
      c.tok16 = toff_k16;
      c.tok8 = toff_k8;
      c.tov16 = toff_v16;
      c.grp = nx_grp;
      c.gc = nx_gc;
      c.sc = nx_sc;
      c.rn = route_next;
      c.sk[0] = __builtin_bit_cast(uint16_t, sk_next[0]);
      c.sk[1] = 0;
      c.nsw = n_sw;
      c.nblk = n_blocks;
      c.act = row0w < Lq ? 1 : 0;
      c.bits = bits;
      c.bits_hi = bits_hi;
      // split: tile t lies past the low half's last key iff t * 64 > lo_last_key
      c.lolim = lo_last_key < 0 ? 0 : lo_last_key / kBN + 1;
      c.half = half;
      c.mt = a.mask_tiles;
      c.kbt = kb_tiles;
      c.hask = has_ks ? 1 : 0;
      c.hk2 = a.hk * 2;
      c.rsk16 = rs_k16.w;
      c.rsk8 = rs_k8.w;
      c.rsv16 = rs_v16.w;
      c.stpk16 = step_k16;
      c.stpk8 = step_k8;
      c.stpv16 = step_v16;
      c.tsk16 = tstep_k16;
      c.tsk8 = tstep_k8;
      c.tsv16 = tstep_v16;
      c.ldsw = (int)smem_lds + wave * 1024;
      c.dk16 = dma_k16;
      c.dk8 = dma_k8;
      c.dv16 = dma_v16;
      c.sq16 = __builtin_bit_cast(uint16_t, sq16);
      c.qks = a.qk_scale;
      c.magic2 = 0x4B4000004B400000ull;
      if constexpr (MODE != TILEMIX_ROUTING_FP16) {
        // K scales through a raw buffer over the whole array (every lookup is
        // clamped to the sequence's blocks); offsets in bytes.
        const SRsrc rs = make_srsrc(a.sk, 0x7fffffff);
        c.rssk = rs.w;
        c.skoff = has_ks ? (int)((skp - a.sk) * 2) : 0;
        c.sklast = has_ks ? (int)((sk_last - a.sk) * 2) : 0;
      } else {
        c.rssk = (i32x4){};
        c.skoff = c.sklast = 0;
      }
      // Every SGPR operand as a wave-uniform value (they are; readfirstlane
      // tells the compiler).
      {
        auto u = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
        auto u64 = [&](uint64_t x) {
          return (uint64_t)(uint32_t)u((int)(uint32_t)x) | ((uint64_t)(uint32_t)u((int)(x >> 32)) << 32);
        };
        auto u4 = [&](i32x4 x) { return (i32x4){u(x[0]), u(x[1]), u(x[2]), u(x[3])}; };
        c.tok16 = u(c.tok16); c.tok8 = u(c.tok8); c.tov16 = u(c.tov16);
        c.grp = u(c.grp); c.gc = u(c.gc); c.sc = u(c.sc); c.skoff = u(c.skoff); c.rn = u(c.rn);
        c.nsw = u(c.nsw); c.nblk = u(c.nblk); c.act = u(c.act); c.bits = u64(c.bits);
        c.bits_hi = u64(c.bits_hi); c.lolim = u(c.lolim); c.half = u(c.half);
        c.mt = u(c.mt); c.kbt = u(c.kbt); c.hask = u(c.hask); c.sklast = u(c.sklast); c.hk2 = u(c.hk2);
        c.rssk = u4(c.rssk); c.rsk16 = u4(c.rsk16); c.rsk8 = u4(c.rsk8); c.rsv16 = u4(c.rsv16);
        c.stpk16 = u(c.stpk16); c.stpk8 = u(c.stpk8); c.stpv16 = u(c.stpv16);
        c.tsk16 = u(c.tsk16); c.tsk8 = u(c.tsk8); c.tsv16 = u(c.tsv16); c.ldsw = u(c.ldsw);
        c.qks = __int_as_float(u(__float_as_int(c.qks)));
      }
      if constexpr (MODE == TILEMIX_ROUTING_FP16) pipe_loop_f16(st, po, c);
      else if constexpr (MODE == TILEMIX_ROUTING_INT8) pipe_loop_i8(st, po, c);
      else if constexpr (SPLIT) pipe_loop_split(st, po, c);
      else pipe_loop_mixed(st, po, c);

#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = st.acc[db];
      m_i = st.mn;
      l_i = st.li;
      toff_k16 = c.tok16;
      toff_k8 = c.tok8;
      toff_v16 = c.tov16;
      nx_grp = c.grp;
      nx_gc = c.gc;
      nx_sc = c.sc;
      route_next = c.rn;
      sk_next[0] = __builtin_bit_cast(f16, (uint16_t)((n_sw & 1) ? c.sk[1] : c.sk[0]));
      if constexpr (MODE != TILEMIX_ROUTING_FP16) {
        if (has_ks) skp = a.sk + c.skoff / 2;
      }
    }
  }

  if constexpr (!GEN) {
    for (int n = n_sw; n < n_wave; ++n) {
      const int route = SPLIT ? (route_next >> half) & 1 : route_next;
      const f16 skc[NSG] = {sk_next[0]};
      const f16 svc[NSG] = {sv_next[0]};
      unsigned char* stage = smem + (n & 1) * STAGE;
      tile_wait(n);
      const int key0 = n * kBN;
      uint32_t s16[2][8];
      tile_scores(stage, route, skc, key0, s16);
      // The next tile's copies go out after this tile's K reads: the loop
      // head's scalar work then no longer delays the QK chain.
      if (n + 1 < n_blocks)
        issue_next(n + 1, smem_lds + ((n + 1) & 1) * STAGE, route_next, sk_next, sv_next);
      tile_mask(key0, s16);
      const float mx = tile_max(s16);
      const bool has = mx != -INFINITY;
      const float m_next = has ? fmaxf(m_i, mx) : m_i;
      const float alpha = has ? fast_exp2(m_i - m_next) : 1.0f;
      tile_update(stage, route, svc, s16, m_next, alpha);
    }
    for (int n = max(n_wave, n_sw); n < n_blocks; ++n) tile_start(n);
  } else {
    // Steps of tiles n >= n_wave are no-ops for this wave (fully masked rows)
    // in both passes: the wave keeps the barriers and copies going only.
    float gmx = -INFINITY;  // row maximum of the current group's max pass
    Step cur = first_step();
    for (int si = 0; cur.n < n_blocks; ++si) {
      const Step nxt = next_step(cur);
      const int route = SPLIT ? (route_next >> half) & 1 : route_next;
      f16 skc[NSG], svc[NSG];
#pragma unroll
      for (int g = 0; g < NSG; ++g) {
        skc[g] = sk_next[g];
        svc[g] = sv_next[g];
      }
      unsigned char* stage = smem + (si & 1) * STAGE;
      step_start(si, cur, nxt);
      if (cur.n < n_wave) {
        const int key0 = cur.n * kBN;
        uint32_t s16[2][8];
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
  {
    const float2 sw = swap_halves(l_i);
    l_i = sw.x + sw.y;
  }
  if (row_ok) {
    f16* op = a.out + (int64_t)(q_start + row) * a.so_t + (int64_t)h * a.so_h;
    // acc / l from one IEEE reciprocal per row and Markstein's correction
    // step per element (3 instructions instead of a full division each); the
    // quotient is the correctly rounded one (checked against exact rational
    // arithmetic on random pairs in tests/test_quant_division.py).  The
    // barrier keeps it an fp32 value: folded into one mixed-precision FMA
    // that rounds straight to fp16, it would differ on double-rounding ties.
    const float rl = 1.0f / l_i;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = db * 32 + 8 * rq + 4 * hi;
        if (d0 < a.d) {
          f16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (f16)fp32_round(div_by_recip(acc[db][4 * rq + e], l_i, rl));
          *reinterpret_cast<f16x4*>(op + d0) = o;
        }
      }
  }
}


}  // namespace tmx
