/*
 * tilemix_hip.h -- C ABI of the MI355X (gfx950) TileMix prefill library
 * (libtilemix_hip.so).
 *
 * The library replaces the two GPU launches of the reference's prefill hot path:
 *
 *   quant_per_block_int8_kernel[grid](...)
 *       attention/triton/quant_per_block_varlen.py:6-13 (kernel signature)
 *       attention/triton/quant_per_block_varlen.py:65-73 (launch site)
 *   attn_fwd[grid](...)
 *       attention/triton/tilemix.py:503-579 (kernel signature)
 *       attention/triton/tilemix.py:1286-1336 (launch site in launch_prequantized)
 *
 * and the three prefill helper kernels of the LLaMA glue
 * (models/tilemix_llama.py:718-869: squared-mean RMSNorm, token-major rotary,
 * SiLU * up).
 *
 * Conventions (all entry points):
 *   - Plain C types only: device pointers, element strides, sizes.  No torch
 *     types cross this boundary.  `stream` is a hipStream_t passed as void*
 *     (NULL = the default stream).
 *   - Tensors are token-major "[tokens, heads, dim]" (the reference's flattened
 *     varlen layout, attention/triton/tilemix.py:1169-1170).  Strides are in
 *     ELEMENTS; the dim stride must be 1.
 *   - fp16 data is IEEE binary16 (passed as void*).
 *   - Every call is asynchronous on `stream`, allocates nothing, never
 *     synchronises the host and is reentrant.
 *   - Return value: 0 on success, a TILEMIX_E* code otherwise; the message of
 *     the last failure on the calling thread is returned by tilemix_last_error().
 */
#ifndef TILEMIX_HIP_H
#define TILEMIX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TILEMIX_ABI_VERSION 3

enum tilemix_status {
    TILEMIX_OK = 0,
    TILEMIX_E_INVALID = 1,   /* argument validation failed (nothing launched) */
    TILEMIX_E_LAUNCH = 2,    /* the HIP runtime rejected the launch */
};

/* Routing modes, identical codes to the reference
 * (attention/triton/tilemix.py:159-161: ROUTING_MODE_MIXED/FP16/INT8). */
enum tilemix_routing_mode {
    TILEMIX_ROUTING_MIXED = 0,
    TILEMIX_ROUTING_FP16 = 1,
    TILEMIX_ROUTING_INT8 = 2,
};

/*
 * Per-block symmetric int8 quantisation of a varlen token-major tensor.
 * Replaces quant_per_block_int8_kernel (attention/triton/quant_per_block_varlen.py:6-45)
 * and the host arithmetic of per_block_int8_single (:48-75).
 *
 * For every sequence b, every block `blk` of `blk_tokens` tokens and every head:
 *   s    = max|x * sm_scale| / 127           (fp32, IEEE division)
 *   t    = (x * sm_scale) / s ; t += (t >= 0 ? 0.5 : -0.5)
 *   code = (int8) trunc(t)                   (code 0 for an all-zero block)
 * The scale of block blk of sequence b is stored at row cu_seqlens_scale[b] + blk.
 * cu_seqlens_scale ([batch + 1], int32) is computed and WRITTEN by the launch
 * (exclusive prefix sum of ceil(L_b / blk_tokens)), so the caller needs no
 * device->host copy to size it: scale_rows_capacity >= ceil(tokens/blk) + batch
 * always suffices.
 */
typedef struct tilemix_quant_params {
    const void* input;            /* fp16 [tokens, heads, head_dim]               */
    int8_t* output;               /* int8 codes, same logical layout               */
    float* scale;                 /* fp32 [scale_rows_capacity, heads], row-major */
    void* scale_half;             /* optional fp16 copy of `scale` (NULL = none)  */
    const int32_t* cu_seqlens;    /* [batch + 1] token offsets                     */
    int32_t* cu_seqlens_scale;    /* [batch + 1] written by the launch             */
    int64_t stride_in_token;
    int64_t stride_in_head;
    int64_t stride_out_token;
    int64_t stride_out_head;
    int64_t scale_rows_capacity;  /* rows allocated in scale / scale_half          */
    float sm_scale;
    int32_t heads;
    int32_t head_dim;             /* multiple of 8, <= 256                         */
    int32_t blk_tokens;           /* BLK of the reference (BLKQ=128 / BLKK=64)     */
    int32_t batch;
    int32_t max_seqlen;
} tilemix_quant_params;

int tilemix_quant_per_block_int8(const tilemix_quant_params* p, void* stream);

/*
 * Fused FP16/INT8-routed flash-attention prefill forward.
 * Replaces attn_fwd (attention/triton/tilemix.py:503-951) launched by
 * launch_prequantized (:1132-1337).  One launch computes, for every sequence z,
 * query head h and query block m (block_m rows), the causal/varlen
 * online-softmax attention over key tiles of block_n keys (one softmax step
 * per tile), routing each tile group (block_n_mask keys) to FP16 or INT8 QK^T
 * by bit j of precision_bitmask[hk * ceil(Lq_z / block_m) + m]
 * (hk = h / (heads_q/heads_k)).  The K (and V) scale of key n is
 * sk[cu_k_scale[z] + n / blkk], clamped to the sequence's last scale row.
 *
 * q_quant_in_kernel = 1 (blkq == 128, routing not FP16, and block_m 128, 256 or
 * 512, or block_m 64 unless mixed routing runs on int8 V codes): each 128-row
 * workgroup quantises its own 128-row Q block (scale = max|q|/127, code =
 * trunc(q/scale +- 0.5), exactly quant_per_block_int8 with sm_scale = 1, the
 * way tilemix_attention_with_quant quantises Q, tilemix.py:126-140) instead of
 * reading q8/sq/cu_q_scale, which may then be NULL.  This removes the Q
 * pre-pass of tilemix_attention_with_quant; the reference has no such field.
 *
 * Supported by this build: block_m in {64, 128, 256, 512}; block_n in {64, 128, 256};
 * block_n_mask a multiple of block_n with ceil(max_seqlen_k/block_n_mask) <= 64;
 * head_dim a multiple of 16, <= 128 (the Python layer zero-pads other widths);
 * blkk a positive multiple of 4; fp16 data; (max_seqlen_k + 64) times the
 * largest K/V token stride in bytes below 2 GiB and 128 Q token strides below
 * 2 GiB (tiles are read through 32-bit buffer offsets; the Python layer passes
 * a head-major copy of a stream whose strides exceed it, as the reference
 * addresses any strides with 64-bit pointers, tilemix.py:1259-1275).
 * block_n = 64 with blkk a multiple
 * of 64 runs the fastest kernels; other shapes run variants that stream each
 * block_n tile twice (max pass, then update pass) and look scales up per key.
 */
typedef struct tilemix_attn_params {
    const void* q;                /* fp16 [tokens_q, heads_q, head_dim]            */
    const void* k;                /* fp16 [tokens_k, heads_k, head_dim]            */
    const void* v;                /* fp16 [tokens_k, heads_k, head_dim]            */
    const void* bias;             /* fp16 [*, heads_q, max_q, max_k] or NULL       */
    void* out;                    /* fp16 [tokens_q, heads_q, head_dim]            */
    const uint64_t* precision_bitmask; /* [heads_k * ceil(max_seqlen_q/block_m)]   */
    const int8_t* q8;             /* int8 Q codes (BLKQ blocks)                    */
    const int8_t* k8;             /* int8 K codes (BLKK blocks)                    */
    const int8_t* v8;             /* int8 V codes (only if !int8_use_fp16_v)       */
    const void* sq;               /* fp16 Q scales [rows, heads_q]                 */
    const void* sk;               /* fp16 K scales [rows, heads_k]                 */
    const void* sv;               /* fp16 V scales [rows, heads_k] (int8 V only)   */
    const int32_t* cu_seqlens_q;  /* [batch + 1]                                   */
    const int32_t* cu_seqlens_k;  /* [batch + 1]                                   */
    const int32_t* cu_q_scale;    /* [batch + 1]                                   */
    const int32_t* cu_k_scale;    /* [batch + 1]                                   */
    const int32_t* cu_v_scale;    /* [batch + 1] (int8 V only)                     */
    int64_t stride_q_token, stride_q_head;
    int64_t stride_k_token, stride_k_head;
    int64_t stride_v_token, stride_v_head;
    int64_t stride_o_token, stride_o_head;
    int64_t stride_q8_token, stride_q8_head;
    int64_t stride_k8_token, stride_k8_head;
    int64_t stride_v8_token, stride_v8_head;
    int64_t stride_bias_head, stride_bias_m, stride_bias_n;
    float sm_scale;               /* softmax scale (default head_dim^-0.5)         */
    int32_t heads_q, heads_k, head_dim, batch;
    int32_t max_seqlen_q, max_seqlen_k;
    int32_t block_m, block_n, block_n_mask;
    int32_t blkq, blkk;           /* quantisation block sizes of Q and K (and V)  */
    int32_t causal;
    int32_t routing_mode;         /* enum tilemix_routing_mode                     */
    int32_t int8_use_fp16_v;      /* 1: INT8 tiles use fp16 V for PV (hot path)    */
    int32_t q_quant_in_kernel;    /* 1: quantise Q inside the attention kernel      */
} tilemix_attn_params;

int tilemix_attn_fwd(const tilemix_attn_params* p, void* stream);

/*
 * Same computation as tilemix_attn_fwd (same kernel template, a DUMP
 * instantiation), additionally writing, for every computed (row, key) score:
 *   qk_i32[(tok_q) * s_tok + h * s_head + key] = exact int32 Q8.K8 accumulator
 *                                                (INT8-routed tiles), or the bit
 *                                                pattern of the fp32 MFMA
 *                                                accumulator (FP16-routed tiles)
 *   qk_f16[(tok_q) * s_tok + h * s_head + key] = the fp16 score fed to softmax
 *                                                (before causal masking; both routes)
 * tok_q is the packed query token index, key is sequence-local.  Entries of
 * tiles that are not computed (causally skipped, other route) are left as is.
 * No reference counterpart: this is the observation point for the bit-exact
 * int32-accumulator parity tests.  Either dump pointer may be NULL.
 */
int tilemix_attn_fwd_debug(const tilemix_attn_params* p,
                           int32_t* qk_i32, void* qk_f16,
                           int64_t dump_stride_token, int64_t dump_stride_head,
                           void* stream);

/*
 * Prefill helpers of the LLaMA glue (all fp16 in / fp16 out, fp32 arithmetic).
 *
 * RMSNorm.  Replaces PrefillRMSNorm.forward (models/tilemix_llama.py:788-797):
 * the squared_mean extension (:718-760, fp32 mean of x^2 over the last dim)
 * and _norm_tail (:763-765).  For every row r of `rows` rows of `cols` values:
 *   var      = (sum_c fp32(x)^2) * fp32(1 / cols)
 *   out[r,c] = fp16( fp32(w[c]) * fp32( fp16( fp32(x[r,c]) * rsqrt(var + eps) ) ) )
 * Rows are `stride_x` / `stride_out` elements apart; the last dim is contiguous.
 */
typedef struct tilemix_rmsnorm_params {
    const void* x;                /* fp16 [rows, cols] (row stride stride_x)       */
    const void* weight;           /* fp16 [cols]                                   */
    void* out;                    /* fp16 [rows, cols] (row stride stride_out)     */
    int64_t rows;
    int64_t stride_x, stride_out;
    int32_t cols;
    float eps;
} tilemix_rmsnorm_params;

int tilemix_rms_norm_f16(const tilemix_rmsnorm_params* p, void* stream);

/*
 * Split-half rotary embedding of Q and K into token-major outputs.
 * Replaces the _rotary Triton kernel and its launch in rotary_token_major
 * (models/tilemix_llama.py:808-847).  For batch b, token t, head h, dim d
 * (D = head_dim, d' = (d + D/2) % D, sign = -1 for d < D/2 else +1):
 *   out[b,t,h,d] = fp16( fp32(fp16(x[b,h,t,d] * c)) + fp32(fp16(x[b,h,t,d'] * sign * s)) )
 * with c = cos[b,t,d], s = sin[b,t,d] (batch stride 0 broadcasts one row);
 * q_out is [batch, tokens, heads_q, D], k_out [batch, tokens, heads_k, D],
 * both contiguous.  Input strides are in elements; the dim stride is 1.
 */
typedef struct tilemix_rotary_params {
    const void* q;                /* fp16 [batch, heads_q, tokens, D] (strided)    */
    const void* k;                /* fp16 [batch, heads_k, tokens, D] (strided)    */
    const void* cos;              /* fp16 [batch or 1, tokens, D] (strided)        */
    const void* sin;
    void* q_out;                  /* fp16 [batch, tokens, heads_q, D] contiguous   */
    void* k_out;                  /* fp16 [batch, tokens, heads_k, D] contiguous   */
    int64_t stride_q_batch, stride_q_head, stride_q_token;
    int64_t stride_k_batch, stride_k_head, stride_k_token;
    int64_t stride_cos_batch, stride_cos_token;
    int64_t stride_sin_batch, stride_sin_token;
    int32_t batch, tokens, heads_q, heads_k, head_dim;  /* head_dim even          */
} tilemix_rotary_params;

int tilemix_rotary_f16(const tilemix_rotary_params* p, void* stream);

/*
 * SiLU(gate) * up.  Replaces the _silu_mul Triton kernel and silu_mul
 * (models/tilemix_llama.py:850-869):
 *   out[i] = fp16( fp32( fp16( g / (1 + exp(-g)) ) ) * fp32(up[i]) ),  g = fp32(gate[i])
 * with an IEEE fp32 division.  gate, up and out are contiguous, n elements.
 */
int tilemix_silu_mul_f16(const void* gate, const void* up, void* out, int64_t n, void* stream);

/* Library introspection. */
int tilemix_abi_version(void);
/* sizeof() of the parameter structs as compiled into the library:
 * 0 = quant, 1 = attn, 2 = rmsnorm, 3 = rotary. */
int64_t tilemix_params_size(int which);
const char* tilemix_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* TILEMIX_HIP_H */
