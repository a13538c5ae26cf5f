// Host side of tilemix_attn_fwd / tilemix_attn_fwd_debug: argument validation
// and kernel selection (kernels: attn_kernel32.h, attn_kernel16.h; selection in attn_launch.h).
#include "attn_common.h"

#include <algorithm>
#include <cstdlib>

namespace tmx {

namespace {

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
  if (p.block_m != 64 && p.block_m != 128 && p.block_m != 256 && p.block_m != 512) {
    set_error("%s: block_m must be 64, 128, 256 or 512, got %d", fn, p.block_m);
    return TILEMIX_E_INVALID;
  }
  if (p.block_n != 64 && p.block_n != 128 && p.block_n != 256) {
    set_error("%s: block_n must be 64, 128 or 256, got %d", fn, p.block_n);
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
  // Kernel choice.  Every row's result depends only on its own route bits, so
  // block_m = 64 runs on the 128-row workgroups of the 32-row kernel: with
  // fp16 or int8 routing the map is not read, with mixed routing each half of
  // the workgroup reads its own routing block.  Only mixed routing with int8 V
  // (which has no room for both K formats in LDS) keeps 64-row workgroups.
  // block_m 256 / 512 run as 128-row workgroups too: the extra tiles a larger
  // block visits are fully masked for a 128-row block's rows (an exact no-op),
  // and each workgroup reads the routing row of the block that holds it.
  const int kind = p.block_m >= 128 ? kAttn32
                 : p.routing_mode != TILEMIX_ROUTING_MIXED ? kAttn32
                 : int8v ? kAttn16 : kAttn32Split;
  const int wg_rows = kind == kAttn16 ? 64 : 128;
  if (p.routing_mode == TILEMIX_ROUTING_MIXED && !p.precision_bitmask) {
    set_error("%s: mixed routing needs precision_bitmask", fn);
    return TILEMIX_E_INVALID;
  }
  // Tiles are streamed as 16-byte vectors: 16-byte aligned bases and strides.
  if (need_int8) {
    if (p.q_quant_in_kernel) {
      // The workgroup quantises its own 128 rows: one BLKQ = 128 block.
      if (wg_rows != 128 || p.blkq != 128) {
        set_error("%s: q_quant_in_kernel needs BLKQ == 128 and 128-row workgroups (block_m 128, 256 or 512, or "
                  "block_m 64 without mixed int8-V routing); block_m=%d, BLKQ=%d", fn, p.block_m, p.blkq);
        return TILEMIX_E_INVALID;
      }
    } else if (!p.q8 || !p.sq || !p.cu_q_scale) {
      set_error("%s: int8 routing needs q8/sq/cu_q_scale (or q_quant_in_kernel)", fn);
      return TILEMIX_E_INVALID;
    }
    if (!p.k8 || !p.sk || !p.cu_k_scale) {
      set_error("%s: int8 routing needs k8/sk/cu_k_scale", fn);
      return TILEMIX_E_INVALID;
    }
    // A K/V scale block is looked up per 4-key group of keys inside the kernel.
    if (p.blkq <= 0 || p.blkk <= 0 || p.blkk % 4 != 0) {
      set_error("%s: BLKQ must be positive and BLKK a positive multiple of 4 (BLKQ=%d, BLKK=%d)", fn, p.blkq,
                p.blkk);
      return TILEMIX_E_INVALID;
    }
    const bool q8_bad = !p.q_quant_in_kernel && (!aligned(p.q8, 16) || (p.stride_q8_token | p.stride_q8_head) % 16);
    if (q8_bad || !aligned(p.k8, 16) || (p.stride_k8_token | p.stride_k8_head) % 16) {
      set_error("%s: q8/k8 must be 16-byte aligned with strides multiple of 16 elements", fn);
      return TILEMIX_E_INVALID;
    }
    if (int8v) {
      if (!p.v8 || !p.sv || !p.cu_v_scale) {
        set_error("%s: int8 V path needs v8/sv/cu_v_scale", fn);
        return TILEMIX_E_INVALID;
      }
      if (!aligned(p.v8, 16) || (p.stride_v8_token | p.stride_v8_head) % 16) {
        set_error("%s: v8 must be 16-byte aligned with strides multiple of 16 elements", fn);
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
  if ((dump_i32 || dump_f16) && (p.bias != nullptr || int8v)) {
    set_error("%s: the debug dump supports neither bias nor the int8 V path", fn);
    return TILEMIX_E_INVALID;
  }

  // K/V tiles are read through 32-bit raw buffers spanning one sequence; the
  // per-lane offsets of the last tile reach up to 64 rows past its end.
  const int64_t span = ((int64_t)p.max_seqlen_k + 64) *
                       (int64_t)std::max(std::max(p.stride_k_token, p.stride_v_token) * 2,
                                         std::max(p.stride_k8_token, p.stride_v8_token));
  if (span >= ((int64_t)1 << 31)) {
    set_error("%s: (max_seqlen_k + 64) * token stride exceeds 2 GiB (%lld bytes)", fn, (long long)span);
    return TILEMIX_E_INVALID;
  }
  // The 128-row Q block is copied through a raw buffer as well.
  if ((int64_t)128 * p.stride_q_token * 2 >= ((int64_t)1 << 31)) {
    set_error("%s: 128 * Q token stride exceeds 2 GiB", fn);
    return TILEMIX_E_INVALID;
  }

  const int m_blocks = (p.max_seqlen_q + wg_rows - 1) / wg_rows;
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
  a.route_shift = p.block_m == 512 ? 2 : p.block_m == 256 ? 1 : 0;
  a.mask_tiles = p.block_n_mask / kBN;
  a.ng = p.block_n / kBN;
  a.blkq = p.blkq > 0 ? p.blkq : 1;
  a.blkk = p.blkk > 0 ? p.blkk : kBN;
  // The block_n = 64 kernels take one K/V scale per 64-key tile.
  const bool gen = a.ng > 1 || (need_int8 && a.blkk % kBN != 0);
  a.causal = p.causal ? 1 : 0;
  a.q_fused = (need_int8 && p.q_quant_in_kernel) ? 1 : 0;
  const bool dump = dump_i32 != nullptr || dump_f16 != nullptr;
  a.total_items = (int)total;
  // The pipelined assembly tile body (head_dim 128, 128-row workgroups, fp16 V,
  // no bias, block_n 64); TILEMIX_HIP_PIPE=0 selects the C++ tile body.
  {
    const char* env = getenv("TILEMIX_HIP_PIPE");
    a.pipe = (env != nullptr && env[0] == '0') ? 0 : 1;
  }
  a.per_xcd = (int)work_items_per_xcd((int64_t)p.heads_k * p.batch, (int64_t)m_blocks * a.group);
  // Groups interleaved per XCD (the work order only: outputs do not depend on
  // it); TILEMIX_HIP_INTERLEAVE=1..4 overrides the choice.
  a.ilv = interleave_groups(p.max_seqlen_k, p.head_dim);
  {
    const char* env = getenv("TILEMIX_HIP_INTERLEAVE");
    if (env != nullptr && env[0] >= '1' && env[0] <= '4' && env[1] == '\0') a.ilv = env[0] - '0';
  }

  const int dp = p.head_dim <= 64 ? 64 : 128;
  dispatch_attn(a, kind, dp, p.routing_mode, int8v, dump, p.bias != nullptr, gen, stream);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", fn, hipGetErrorString(err));
    return TILEMIX_E_LAUNCH;
  }
  return TILEMIX_OK;
}

}  // namespace tmx

namespace tmx {

void dispatch_attn_main(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);
void dispatch_attn_bias(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);
void dispatch_attn_dump(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);
void dispatch_attn_gen_main(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);
void dispatch_attn_gen_bias(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);
void dispatch_attn_gen_dump(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, hipStream_t stream);

void dispatch_attn(const AttnKArgs& a, int kind, int dp, int mode, bool int8v, bool dump, bool bias, bool gen,
                   hipStream_t stream) {
  if (gen) {
    if (dump) dispatch_attn_gen_dump(a, kind, dp, mode, int8v, stream);
    else if (bias) dispatch_attn_gen_bias(a, kind, dp, mode, int8v, stream);
    else dispatch_attn_gen_main(a, kind, dp, mode, int8v, stream);
  } else if (dump) {
    dispatch_attn_dump(a, kind, dp, mode, int8v, stream);
  } else if (bias) {
    dispatch_attn_bias(a, kind, dp, mode, int8v, stream);
  } else {
    dispatch_attn_main(a, kind, dp, mode, int8v, stream);
  }
}

}  // namespace tmx
