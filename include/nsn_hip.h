/*
 * nsn_hip.h -- C ABI of libnsn_hip.so, the MI355X (gfx950) NSN packed-KV hot path.
 *
 * The reference (metaSATOKEN/nsn) exposes this path as Python module
 * functions over Triton kernels and torch eager ops; each entry point below
 * replaces one group of them (citations relative to the reference root).
 * Conventions:
 *   - every pointer is device memory owned by the caller; the library never
 *     allocates; inputs are never written;
 *   - all work is enqueued on `stream` (a hipStream_t); calls are asynchronous;
 *   - data-dependent failures (nonfinite values, fp16 metadata overflow, code
 *     range) are OR-ed into the caller's device status word `status` (int32,
 *     NSN_ST_* bits) -- the caller reads it when it needs to raise;
 *   - the return value reports argument / launch errors (NSN_OK == 0).
 * Packed layout (the reference's, see loop_kv_pk01_cache.py:7-37):
 *   block = 64 tokens x 128 channels of one (sequence, kv-head);
 *   codes: LSB-first bitstream, code of (token t, channel c) at bits
 *          [(t*128+c)*bits, +bits) of the block's 64*128*bits/8 bytes;
 *   norm:  fp16 [64] per block; min, scale: fp16 [128] per block;
 *   header: 12 bytes '<QHBB' = (token offset u64, 64 u16, bits u8, 0 u8).
 */
#ifndef NSN_HIP_H
#define NSN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *nsn_stream_t; /* == hipStream_t */

enum { NSN_DTYPE_F16 = 0, NSN_DTYPE_BF16 = 1, NSN_DTYPE_F32 = 2 };

/* Order of the fp32 sum of squares in the encoder's token norm.  torch's CPU
 * vector_norm uses 8 fma lanes (elements j, j+8, ...; lanes summed in order)
 * for a contiguous row, and one fma chain when the row is strided. */
enum { NSN_NORM_LANES8 = 0, NSN_NORM_SEQUENTIAL = 1 };

/* Status-word bits. */
#define NSN_ST_NONFINITE_INPUT 0x01   /* encode: nonfinite input            */
#define NSN_ST_META_NONFINITE 0x02    /* encode: fp16 metadata overflow/NaN  */
#define NSN_ST_META_UNDERFLOW 0x04    /* encode: nonzero norm/step -> fp16 0 */
#define NSN_ST_CODE_RANGE 0x08        /* pack: code >= 2^bits                */
#define NSN_ST_NONFINITE_RESTORE 0x10 /* restore: nonfinite reconstruction   */
#define NSN_ST_NONFINITE_ATTN 0x20    /* attention: nonfinite score/weights  */
#define NSN_ST_NONFINITE_OUTPUT 0x40  /* attention merge: nonfinite context  */
#define NSN_ST_NONFINITE_SCAN 0x80    /* finite scan: nonfinite raw input    */
#define NSN_ST_TAIL_RANGE 0x200 /* tail append: device end position outside [n, tail_cap] */
#define NSN_ST_NONFINITE_ATTN_INPUT 0x100 /* attention: nonfinite raw input read by the kernel
                                             (q, tail tokens; block metadata in the REFERENCE kernel) */
#define NSN_ST_WORKSPACE 0x400  /* attention: the partial slots (n_splits) are too few for the FAST kernel's partition */
#define NSN_ST_CAPACITY 0x800   /* attention: a sequence's blocks or tail lie past the cache's capacity
                                   (blocks > block_cap or seq_len - 64*blocks > tail_cap); neither
                                   decode kernel reads anything of that sequence */
#define NSN_ST_EMPTY 0x1000     /* attention merge: a (sequence, q-head) attended no token (length 0,
                                   or a length refused by NSN_ST_CAPACITY); its output is zero */

/* Return codes. */
#define NSN_OK 0
#define NSN_EINVAL (-1)
#define NSN_ELAUNCH (-2)
#define NSN_ENOSPC (-3) /* nsn_decode_attention_static: workspace beyond the static scratch */

/* Library version string. */
const char *nsn_version(void);

/* sizeof of the argument structs this library was built with, for bindings
 * to check their own layouts against at load time: which = 0 nsn_kv_side,
 * 1 nsn_attn_args, 2 nsn_prefill_args, 3 nsn_kscore_args; -1 otherwise. */
int64_t nsn_abi_sizeof(int which);

/*
 * Encode 64x128 blocks: token norm, per-channel min/max over the block,
 * round-half-even codes, LSB-first packing, fp16 metadata, headers.
 * Replaces nsn_encode (experiments/ac08/source/loop_kv_pilot.py:195-213),
 * pack3 (experiments/ac08/source/loop_kv_pk01_cache.py:7-16) and the header
 * loop of encode_group (loop_kv_pk01_cache.py:31-37).
 *   x: input rows of 128 elements (x_dtype), contiguous within a row; block
 *      (o, i) starts at element o*x_outer_stride + (x_token_offset + 64*i)*128.
 *      16-byte aligned.
 *   Output block (o, i) lands at index ob = o*out_outer_blocks + out_block_offset + i
 *   of codes [*, 64*128*bits/8], norms [*, 64], mins/scales [*, 128] (fp16
 *   bits) and headers [*, 12] (nullable); its header token is
 *   header_start_token + 64*i.
 *   factors (nullable): [*, 64] fp32 decode factors (see nsn_block_factors).
 *   codes_unpacked (nullable): [n_outer*n_blocks, 64, 128] u8 codes.
 *   zero_flat_scale: 1 = nsn_encode (codes forced to 0 where scale == 0),
 *                    0 = nsn_int3_qdq (identical outputs for finite input).
 */
int nsn_encode_blocks(const void *x, int x_dtype, int64_t n_outer, int64_t n_blocks,
                      int64_t x_outer_stride, int64_t x_token_offset, int bits, int norm_order,
                      int zero_flat_scale, uint8_t *codes, uint16_t *norms, uint16_t *mins,
                      uint16_t *scales, uint8_t *headers, float *factors, int64_t out_outer_blocks,
                      int64_t out_block_offset, int64_t header_start_token,
                      uint8_t *codes_unpacked, int32_t *status, nsn_stream_t stream);

/*
 * LSB-first bitstream of `count` codes (bits in {3,4,5}) -> (count*bits+7)/8 bytes.
 * Replaces pack_codes (loop_kv_pilot.py:171-181) and pack3 (loop_kv_pk01_cache.py:7-16).
 * Codes >= 2^bits set NSN_ST_CODE_RANGE.
 */
int nsn_pack_codes(const uint8_t *codes, int64_t count, int bits, uint8_t *out, int32_t *status,
                   nsn_stream_t stream);

/*
 * Inverse of nsn_pack_codes.  Replaces unpack3 (loop_kv_pk01_cache.py:19-28),
 * the PU01 kernel (experiments/ac08/source/loop_kv_pu01_kernel.py:32-52) and
 * unpack_codes_reference (loop_kv_pilot.py:183-193).
 */
int nsn_unpack_codes(const uint8_t *payload, int64_t count, int bits, uint8_t *out,
                     nsn_stream_t stream);

/*
 * Reconstruct blocks (nsn_decode arithmetic: d = m + s*q, y = n*(d/max(|d|,1e-12)),
 * n==0 -> 0, RNE cast) and append a tail.
 * Replaces nsn_decode (loop_kv_pilot.py:216-225), restore_group
 * (loop_kv_pk01_cache.py:40-42, loop_kv_rf01_kernel.py:60-74,
 * loop_kv_pu01_kernel.py:54-56) and the bridge restore_v/materialize
 * (experiments/ac08/source/loop_kv_vf01_kernel.py:47-54,120-126).
 *   codes: packed [n_outer, in_outer_blocks, 64*128*bits/8] (codes_are_unpacked=0)
 *          or unpacked u8 [n_outer, in_outer_blocks, 64, 128] (codes_are_unpacked=1);
 *   norms/mins/scales: [n_outer, in_outer_blocks, 64|128] fp16 bits;
 *   out: [n_outer, out_outer_tokens, 128] out_dtype; tokens [0, 64*n_blocks)
 *        restored, tokens [64*n_blocks, 64*n_blocks + tail_len) copied from
 *        tail [n_outer, tail_outer_tokens, 128] tail_dtype (tail nullable when
 *        tail_len == 0).
 */
int nsn_restore_blocks(const uint8_t *codes, int codes_are_unpacked, const uint16_t *norms,
                       const uint16_t *mins, const uint16_t *scales, int64_t n_outer,
                       int64_t n_blocks, int64_t in_outer_blocks, int bits, void *out,
                       int out_dtype, int64_t out_outer_tokens, const void *tail,
                       int tail_dtype, int64_t tail_len, int64_t tail_outer_tokens,
                       int32_t *status, nsn_stream_t stream);

/*
 * Per-token decode factors f_t = n_t / max(|m + s*q_t|, 1e-12) of packed blocks
 * (fp16 metadata as fp32; the norm in nsn_decode's order), so that the restored
 * row is f_t * (m + s*q_t).  A block's factors never change once it is encoded,
 * so decode attention reads them instead of renormalising every token on every
 * step.  No counterpart in the reference (it renormalises inside each read,
 * experiments/ac08/source/loop_kv_vf01_kernel.py:28-34).
 *   codes/norms/mins/scales: [n_outer, in_outer_blocks, ...] as nsn_restore_blocks;
 *   factors: [n_outer, in_outer_blocks, 64] fp32.
 *   status (nullable): NSN_ST_NONFINITE_ATTN_INPUT is raised when a block's
 *   norms, mins or scales hold a NaN/Inf (the finite check of the raw
 *   metadata, loop_kv_vf01_checks.py:55-63, for callers that read factors).
 */
int nsn_block_factors(const uint8_t *codes, const uint16_t *norms, const uint16_t *mins,
                      const uint16_t *scales, int64_t n_outer, int64_t n_blocks,
                      int64_t in_outer_blocks, int bits, float *factors, int32_t *status,
                      nsn_stream_t stream);

/* K/V sources of the decode attention. */
enum {
    NSN_KV_PACKED = 0,  /* packed blocks for tokens < 64*blocks[b], then the tail buffer */
    NSN_KV_SCORES = 1   /* (K side only) fp32 logits given: the AF01 FULL=False readout */
};

/* Attention kernels. */
enum {
    NSN_ATTN_REFERENCE = 0, /* exact-order: nsn_decode restore, K/V rounded to kv_round_dtype,
                               fp32 QK / online softmax / PV (route-equal bridge and fused) */
    NSN_ATTN_FAST = 1       /* factored MFMA kernel (codes on matrix cores); tolerance-equal */
};

typedef struct {
    const uint8_t *codes;   /* [B, Hkv, block_cap, 64*128*bits/8] */
    const uint16_t *norms;  /* [B, Hkv, block_cap, 64]  fp16 */
    const uint16_t *mins;   /* [B, Hkv, block_cap, 128] fp16 */
    const uint16_t *scales; /* [B, Hkv, block_cap, 128] fp16 */
    const float *factors;   /* [B, Hkv, block_cap, 64] fp32 decode factors (NSN_ATTN_FAST) */
    const int32_t *blocks;  /* [B] packed blocks per sequence (nullable -> 0) */
    int64_t block_cap;
    const void *tail;       /* [B, Hkv, tail_cap, 128] tail_dtype: tokens 64*blocks[b] .. */
    int tail_dtype;
    int64_t tail_cap;
} nsn_kv_side;

typedef struct {
    const void *q;          /* [B, Hq, 128] q_dtype */
    int q_dtype;
    int64_t batch, heads_q, heads_kv; /* heads_q = G * heads_kv; q-head h reads kv-head h / G */
    float scale;            /* 1/sqrt(128) = 0.08838834764831845 */
    const int32_t *seq_len; /* [B] tokens per sequence (>0) */
    int max_seq_len;        /* >= every seq_len[b] */
    int bits;               /* 3, 4 or 5 */
    int k_mode;             /* NSN_KV_PACKED | NSN_KV_SCORES */
    nsn_kv_side k, v;
    const float *scores;    /* [B, Hq, scores_cap] fp32 (k_mode == NSN_KV_SCORES) */
    int64_t scores_cap;
    int kernel;             /* NSN_ATTN_REFERENCE | NSN_ATTN_FAST */
    int kv_round_dtype;     /* reference kernel: dtype restored K/V are rounded to */
    int split_tokens;       /* REFERENCE: tokens per split (multiple of 64) */
    int n_splits;           /* REFERENCE: ceil(max_seq_len / split_tokens); FAST: partial slots per
                               (b, hq), >= 2 (the FAST kernel splits the blocks of all sequences
                               evenly over a fixed grid; max_seq_len bounds the slots it needs) */
    float *partials;        /* workspace of nsn_attention_workspace_floats() floats: [B, Hq, n_splits, 132]
                               fp32 partials, then one int32 partial count per (b, hq) */
    float *ctx;             /* [B, Hq, 128] fp32 (nullable) */
    void *out;              /* [B, Hq, 128] out_dtype */
    int out_dtype;
    int32_t *status;
    int merge;              /* 1: also run the split merge; 0: partials only */
    /* REFERENCE kernel only (nullable; NSN_ATTN_FAST rejects them): what the kernel itself
       computed, for tokens t < seq_len[b] -- trace_scores [B, Hq, trace_cap] fp32 (the scaled
       q.k, or the given logits) and trace_v [B, Hkv, trace_cap, 128] fp32 (the V rows as
       restored and multiplied); trace_cap >= max_seq_len.  Replaces the TRACE stores of
       experiments/ac08/source/loop_kv_vf01_kernel.py:104,113. */
    float *trace_scores;
    float *trace_v;
    int64_t trace_cap;
} nsn_attn_args;

/*
 * Single-query decode attention over packed K/V (+ tail), split over the
 * context with a log-sum-exp merge.  Replaces the VF01 fused route
 * (experiments/ac08/source/loop_kv_vf01_kernel.py:56-139), AF01 partial/merge
 * (experiments/ac08/source/loop_kv_af01_kernel.py:13-111) and the GQA route
 * (experiments/nb06/source/loop_kv_nb06_kernel.py:54-154).  A dense fp16/bf16
 * K/V baseline is the same call with blocks == NULL.
 */
int nsn_decode_attention(const nsn_attn_args *args, nsn_stream_t stream);

/*
 * Log-sum-exp merge of the per-split partials written by nsn_decode_attention
 * (with merge == 0): ctx = sum_s u_s e^(m_s - M) / sum_s z_s e^(m_s - M),
 * out = RNE cast of ctx, over the partial count stored after the partials
 * (see nsn_attn_args.partials).  Replaces the AF01 merge kernel
 * (experiments/ac08/source/loop_kv_af01_kernel.py:70-82).
 */
int nsn_attention_merge(const float *partials, int64_t batch, int64_t heads_q, int n_splits, float *ctx,
                        void *out, int out_dtype, int32_t *status, nsn_stream_t stream);

/* Workspace floats needed by nsn_decode_attention for the given shape
 * (partials plus the per-(b, hq) partial counts that nsn_attention_merge reads). */
int64_t nsn_attention_workspace_floats(int64_t batch, int64_t heads_q, int n_splits);

/*
 * nsn_decode_attention with no caller workspace and no allocation: the
 * partials live in a file-scope device array of NSN_STATIC_SCRATCH_FLOATS
 * floats (16 MiB) that each GPU the library runs on holds until the process
 * ends.  args->partials is ignored.  A shape whose
 * nsn_attention_workspace_floats() exceeds the maximum returns NSN_ENOSPC
 * before anything is launched.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (concurrent streams, or another
 * launch before this one's merge has finished) race; calls in stream order
 * are safe.  Nothing in the array needs to start at zero: every partial
 * count the merge reads is written by the same call (0 for a (sequence,
 * q-head) with no usable token, whose output the merge sets to zero under
 * NSN_ST_EMPTY), and so is every partial slot below that count -- except
 * where the call raises NSN_ST_WORKSPACE, whose outputs are not valid.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
#define NSN_STATIC_SCRATCH_FLOATS (4 * 1024 * 1024)
int nsn_decode_attention_static(const nsn_attn_args *args, nsn_stream_t stream);

/*
 * Chunked-prefill attention: n_q chunk queries per (sequence, q-head) attend
 * the sequence's context -- k.blocks[b] packed blocks, then ctx_len[b] -
 * 64*blocks[b] tail tokens -- and the chunk's own K/V causally (chunk query i
 * sees chunk tokens 0..i).  Packed blocks are dequantised tile by tile into
 * LDS (direction m + s*z times the decode factor, in the compute dtype) and
 * never reach HBM densely; QK^T and PV run on MFMA in the compute dtype
 * (`dtype`: fp16 or bf16) with fp32 accumulation and an online log2-domain
 * softmax.  Replaces the reference's prefill route: materialise every packed
 * block and the tail (PackedCache.materialize / update,
 * experiments/ac08/source/loop_kv_pk01_cache.py:87-106, restore_group :40-42)
 * followed by dense attention over the materialised K/V.
 * append != 0 also performs the chunk's cache update (the tail concatenation
 * of PackedCache.update, loop_kv_pk01_cache.py:101-102) in the same launch:
 * the chunk's K/V rows go to rows ctx_len[b] - 64*k.blocks[b] .. + n_q - 1
 * of k.tail / v.tail (write access granted by the caller), rounded to the
 * tail dtype -- what nsn_tail_append_cast writes.  Needs both tails; a
 * sequence whose tail lacks the room raises NSN_ST_CAPACITY and is not
 * appended.
 * Needs k.blocks and v.blocks equal per sequence (or both NULL), decode
 * factors, 16-byte aligned arrays, one dtype for q, the chunk K/V and out,
 * and one tail dtype (fp16 or bf16) for both tails.
 */
typedef struct {
    const void *q;          /* [B, Hq, n_q, 128] dtype */
    int dtype;              /* NSN_DTYPE_F16 | NSN_DTYPE_BF16 */
    int64_t batch, heads_q, heads_kv, n_q;   /* heads_q = G * heads_kv */
    float scale;            /* 1/sqrt(128) */
    const int32_t *ctx_len; /* [B] context tokens before the chunk (device) */
    int bits;               /* 3 or 5 */
    nsn_kv_side k, v;       /* packed context + tail (tail_dtype == dtype) */
    const void *k_chunk;    /* [B, Hkv, n_q, 128] dtype: the chunk's own K */
    const void *v_chunk;    /* [B, Hkv, n_q, 128] dtype */
    void *out;              /* [B, Hq, n_q, 128] dtype */
    int32_t *status;        /* NSN_ST_NONFINITE_OUTPUT; NSN_ST_CAPACITY on an inconsistent cache or no room to append */
    int append;             /* 1: also append the chunk's K/V to the tails (see above) */
    int precise_weights;    /* bf16 only: 1 = the softmax weights enter the PV product as bf16 hi + lo
                               (~2^-17 relative) instead of one bf16 rounding (2^-9), at ~24 % more
                               time per block; for chunks with little or no context, whose first
                               queries attend a handful of tokens.  Ignored for fp16. */
} nsn_prefill_args;

int nsn_prefill_attention(const nsn_prefill_args *args, nsn_stream_t stream);

/*
 * Append n new K and V tokens of `rows` = B*Hkv rows to preallocated tails
 * in place: row r, token i of k_new (at (r*new_row_stride + i)*128 elements)
 * goes to token offset + i of row r of k_tail ([rows, tail_cap, 128]); the
 * same for v.  One launch for both sides.  Replaces the tail concatenation
 * of PackedCache.update (experiments/ac08/source/loop_kv_pk01_cache.py:101-102).
 */
int nsn_tail_append(const void *k_new, const void *v_new, int64_t rows, int64_t n, int64_t new_row_stride,
                    void *k_tail, void *v_tail, int64_t tail_cap, int64_t offset, int dtype, nsn_stream_t stream);

/*
 * nsn_tail_append with a dtype conversion: k_new / v_new hold src_dtype
 * (NSN_DTYPE_F16, NSN_DTYPE_BF16 or NSN_DTYPE_F32) and every element is
 * rounded to the tail dtype (NSN_DTYPE_F16 or NSN_DTYPE_BF16, round to
 * nearest even), so that an append of model activations in another dtype
 * needs no separate conversion pass.  Same layout and checks as
 * nsn_tail_append.  Replaces the same tail concatenation
 * (experiments/ac08/source/loop_kv_pk01_cache.py:101-102) where the new
 * tokens' dtype differs from the preallocated tail's.
 */
int nsn_tail_append_cast(const void *k_new, const void *v_new, int src_dtype, int64_t rows, int64_t n,
                         int64_t new_row_stride, void *k_tail, void *v_tail, int64_t tail_cap, int64_t offset,
                         int dtype, nsn_stream_t stream);

/*
 * nsn_tail_append with the position in device memory: the n new tokens of
 * each row go to [*tail_end - n, *tail_end).  The launch then has no host
 * argument that changes from step to step, so a captured HIP graph of a
 * decode step replays it unchanged while the caller advances *tail_end on
 * the device.  An end outside [n, tail_cap] writes nothing and raises
 * NSN_ST_TAIL_RANGE in *status.  Replaces the same tail concatenation
 * (experiments/ac08/source/loop_kv_pk01_cache.py:101-102) under graph replay.
 */
int nsn_tail_append_to(const void *k_new, const void *v_new, int64_t rows, int64_t n, int64_t new_row_stride,
                       void *k_tail, void *v_tail, int64_t tail_cap, const int32_t *tail_end, int dtype,
                       int32_t *status, nsn_stream_t stream);

/*
 * One decode token per sequence, fused: the rotary position embedding of q
 * [batch, heads_q, 128] and k [batch, heads_kv, 128] (sequence b's heads at
 * b * q_stride, resp. b * kv_stride elements -- slices of one fused QKV
 * projection work; model dtype `dtype`,
 * fp16 or bf16; cos, sin rows of 128, sequence b's at b * cs_stride --
 * 0 for one row shared by all) exactly as transformers'
 * apply_rotary_pos_emb computes it in that dtype (x*cos and rotate_half(x)*sin
 * each rounded, then their sum), the rotated q written to q_out, and the
 * rotated k and v converted to the tails' `tail_dtype` (fp16 or bf16, round
 * to nearest even) and appended to them
 * ([batch*heads_kv, tail_cap, 128]) at token *tail_end - 1 (device position,
 * as nsn_tail_append_to; NSN_ST_TAIL_RANGE outside [1, tail_cap]) or, with
 * tail_end NULL, at `offset`.  Replaces, for the packed decode route, the
 * rotary step and the tail concatenation of the patched attention
 * (experiments/ac08/source/loop_kv_ac08_attention.py:59-66) -- about a dozen
 * elementwise kernels per layer.
 */
int nsn_rope_append(const void *q, const void *k, const void *v, int64_t q_stride, int64_t kv_stride,
                    const void *cos, const void *sin, int64_t cs_stride, int64_t batch, int64_t heads_q, int64_t heads_kv, void *q_out, void *k_tail,
                    void *v_tail, int64_t tail_cap, const int32_t *tail_end, int64_t offset, int dtype,
                    int tail_dtype, int32_t *status, nsn_stream_t stream);

/*
 * NaN/Inf scan over up to 16 arrays; array i sets bit i of flags[0] (int32)
 * and NSN_ST_NONFINITE_SCAN in status.  Replaces the grouped finite checks
 * (experiments/ac08/source/loop_kv_vf01_checks.py:20-63,
 * loop_kv_iv01_kernel.py:29-46).
 */
int nsn_finite_scan(int n_arrays, const void *const *ptrs, const int64_t *counts,
                    const int *dtypes, int32_t *flags, int32_t *status, nsn_stream_t stream);

/*
 * K-score decode (the K side of one decode query, scores only) over the K1c
 * cache layout.  Replaces `_fused_score_kernel` and its launcher
 * `triton_decode_scores` (experiments/kernels/phase_k1c_triton_fused_kernel.py:207-281):
 *   out[b, h, t] = scale * en[b, hkv, t] * sum_d q[b, h, d] * (code[b, t, hkv*D + d] * step[b, hkv*D + d]
 *                                                              + min[b, hkv*D + d]),   hkv = h / (Hq / Hkv)
 * with en = 1 when eff_norm is NULL (KIVI), and K itself for NSN_KS_FP16.
 * Layouts (all contiguous):
 *   q        fp16 [B, Hq, D]
 *   codes    NSN_KS_U8:     u8 [B, T, Hkv*D] (one code per byte, the reference's layout)
 *            NSN_KS_PACKED: the same codes bit-packed LSB-first along each token
 *                           row, [B, T, Hkv*D*bits/8] (bits 3, 4, 5)
 *            NSN_KS_FP16:   fp16 K [B, T, Hkv*D]
 *   mins, steps  fp16 [B, Hkv*D] (unused for NSN_KS_FP16)
 *   eff_norm fp16 [B, Hkv, T] or NULL
 *   out      fp32 [B, Hq, T]
 * D is 128 or 256; Hq / Hkv <= 8.  codes 16-byte aligned when a lane's D/4
 * channels span a multiple of 16 bytes (u8, 4-bit, fp16), else 4-byte.
 */
enum { NSN_KS_U8 = 0, NSN_KS_PACKED = 1, NSN_KS_FP16 = 2 };

typedef struct {
    const void *q;
    int64_t batch, heads_q, heads_kv, head_dim, T;
    int mode;                /* NSN_KS_* */
    int bits;                /* NSN_KS_PACKED: 3, 4 or 5 */
    const void *codes;
    const void *mins, *steps;
    const void *eff_norm;
    float scale;             /* 1 / sqrt(D) in the reference */
    float *out;
} nsn_kscore_args;

int nsn_kscore(const nsn_kscore_args *args, nsn_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NSN_HIP_H */
