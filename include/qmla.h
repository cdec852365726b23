/*
 * qmla.h -- C ABI of libqmla.so, the gfx950 (MI355X) absorbed-MLA latent-KV decode library.
 *
 * Plain pointers, sizes and strides only. Every entry point is asynchronous on the stream it is
 * given, allocates nothing, never synchronizes the device, and returns 0 or a negative QMLA_ERR_*
 * code (no exceptions cross the boundary). Safe to record into a HIP graph: no host reads of
 * device data, no memsets.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   qmla_decode           <- decode_attention_fwd(q, k_buffer, v_buffer, o, lse, req_to_token,
 *                            b_seq_len, attn_logits, num_kv_splits, sm_scale, page_size, logit_cap,
 *                            k_scale, v_scale, is_mla, rms_offset, rms_bf16, rms_log8, qrows)
 *                            qwen_mla/ops/mla_decode_attention.py:1264-1359 (stage 1 :297-586,
 *                            stage 2 :1064-1181), and the FlashInfer run() it dispatches to instead
 *                            qwen_mla/fi_decode.py:338-384 / kernels/qwen_mla.cuh:1386-1480
 *                            Wide latents (d_c = 1792), which the reference routes to its two-pass
 *                            path _decode_mla_two_pass (ops/mla_decode_attention.py:778-849:
 *                            _mla2p_scores_kernel :602-678, _mla2p_pv_kernel :681-764), go through the
 *                            same entry points: the library runs them in one pass over the rows with
 *                            the latent columns split across the waves of a workgroup, so no scores
 *                            scratch exists and the partials/combine formats are the same.
 *   qmla_combine          <- _decode_softmax_reducev_fwd / _fwd_kernel_stage2
 *                            qwen_mla/ops/mla_decode_attention.py:1064-1181
 *   qmla_workspace_bytes  <- the split-K scratch sizing of splitk_cap / splitk_reserve_bytes
 *                            qwen_mla/mla_impl.py:89-111 and _RankPlan._workspace_bytes
 *                            qwen_mla/fi_decode.py:170-179
 */
#ifndef QMLA_H
#define QMLA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMLA_ABI_VERSION 2

/* error codes */
#define QMLA_OK 0
#define QMLA_ERR_NULL (-1)        /* a required pointer is NULL */
#define QMLA_ERR_SHAPE (-2)       /* unsupported or inconsistent dimension */
#define QMLA_ERR_ALIGN (-3)       /* a row, page or base address is off 4-byte boundaries, or off
                                     16-byte ones in a layout no narrow-row kernel serves */
#define QMLA_ERR_WORKSPACE (-4)   /* workspace missing or smaller than qmla_workspace_bytes() */
#define QMLA_ERR_MODE (-5)        /* unknown dtype / rms mode / split mode */
#define QMLA_ERR_LAUNCH (-6)      /* the HIP launch itself failed */
#define QMLA_ERR_NOKERNEL (-7)    /* no compiled kernel instance for this shape */
#define QMLA_ERR_PAGE (-8)        /* (stored into *status) a block-table entry outside [0, num_pages) */

/* cache element formats */
#define QMLA_KV_BF16 0
#define QMLA_KV_FP8 1             /* OCP e4m3fn, one per-layer scale for latent and rope */

/* rms (score divisor) tail formats, qwen_mla/mla_impl.py:125-145 and
 * qwen_mla/ops/mla_decode_attention.py:466-505 */
#define QMLA_RMS_NONE 0           /* rms_offset < 0: no divide */
#define QMLA_RMS_BF16 1           /* bf16 cache: one bf16 element per head */
#define QMLA_RMS_LOG8 2           /* fp8 cache: uint8 code c, rms = 2^(-3 + c*6/255) */
#define QMLA_RMS_BF16_BYTES 3     /* fp8 cache: two bytes per head holding a raw bf16 */
#define QMLA_RMS_E4M3 4           /* fp8 cache: one e4m3 byte per head, times k_scale */

/* output / lse element types */
#define QMLA_DT_BF16 0
#define QMLA_DT_F32 1
#define QMLA_DT_F16 2

/*
 * One decode call. Dimensions:
 *   rows       query rows as the caller flattened them (one per decode token; spec-verify
 *              requests contribute qrows consecutive rows sharing a block-table row, as built by
 *              MLATritonMetadataBuilder._build_decode, qwen_mla/mla_impl.py:628-662)
 *   heads      query heads per row; rms_heads rms slots per cached token (normally == heads)
 *   d_c        latent columns (kv_lora_rank); with groups = G > 1 (GLA) head h reads only the
 *              d_c/G columns of group h / (heads/G), and out holds d_c/G columns per head
 *   rope_w     rope columns after the latent; scores read cache columns [0, d_c + rope_w)
 * Strides are in ELEMENTS of the tensor they index (cache strides in cache elements).
 */
typedef struct qmla_decode_params {
  /* queries (bf16): q_nope [rows, heads, d_c/G], q_pe [rows, heads, rope_w] */
  const void* q_nope;
  int64_t q_nope_stride_row, q_nope_stride_head;
  const void* q_pe;
  int64_t q_pe_stride_row, q_pe_stride_head;

  /* paged cache [num_pages, page_size, (1,) row]: element (page, slot, col) at
   * kv_cache + page*page_stride + slot*token_stride + col. Base, page and row strides on 16-byte
   * boundaries (the plugin pads rows to 16 elements); rows on 4-byte boundaries only are served for
   * the unpadded 12-head bf16 layouts of the reference's numerics test (rope 256, ranks 256 / 768 /
   * 1792), else QMLA_ERR_ALIGN */
  const void* kv_cache;
  int64_t page_stride, token_stride;
  int32_t kv_dtype;               /* QMLA_KV_* */
  int32_t page_size;
  int32_t d_c, rope_w;
  int32_t rms_offset;             /* element offset of the rms tail in the row, < 0 = none */
  int32_t rms_mode;               /* QMLA_RMS_* */
  const float* k_scale;           /* device fp32 scalar, NULL = 1.0 (fp8 dequant and e4m3 rms) */
  float sm_scale;
  float logit_cap;                /* > 0: cap * tanh(s / cap) after scaling */

  /* block table [rows, bt_stride] int32 and seq_lens [rows] int32 (device) */
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seq_lens;
  int32_t rows, heads, rms_heads;
  int32_t qrows;                  /* > 1: fold each run of qrows rows into one request so the
                                     cache is read once; row j of a request of length L sees
                                     its first L - (qrows-1-j) tokens. A folded request takes L
                                     and its page ids from its LAST row (seq_lens and block_table
                                     row qrows*r + qrows-1), as the reference's folding does */
  int32_t groups;                 /* latent groups (1, or 2 for GLA-g2) */

  /* outputs: out [rows, heads, d_c/G] (out_dtype), lse [rows, heads] (lse_dtype, may be NULL),
   * natural-log LSE */
  void* out;
  int64_t out_stride_row, out_stride_head;
  int32_t out_dtype;
  void* lse;
  int64_t lse_stride_row;
  int32_t lse_dtype;

  /* split-K. num_splits > 0: the reference's fixed split count; split s of a request of length
   * L covers [s*per, min((s+1)*per, L)) with per = ceil(ceil(L/S)/split_align)*split_align
   * (split_align 0 = no rounding), and the partials live in the caller's workspace in the
   * reference layout attn_logits[rows, heads, S, d_c/G + 1] (strides below, in floats). With
   * S > 1 the call returns QMLA_ERR_WORKSPACE unless workspace_bytes >= qmla_workspace_bytes(),
   * every stride is positive and the largest partial offset (rows-1)*ws_stride_row +
   * (heads-1)*ws_stride_head + (S-1)*ws_stride_split + d_c/G lies inside workspace_bytes.
   * num_splits == 0: balanced mode. Every workgroup gets the same number of 64-token tiles
   * across request boundaries; partials go to the workspace at qmla_workspace_bytes() size and
   * the ws_stride_* fields are ignored. */
  int32_t num_splits;
  int32_t split_align;
  float* workspace;
  size_t workspace_bytes;
  int64_t ws_stride_row, ws_stride_head, ws_stride_split;

  /* balanced mode only: workgroups to launch, 0 = one per compute unit times occupancy */
  int32_t num_workgroups;

  /* page-id bound. num_pages > 0: every block-table entry a kernel reads is checked against
   * [0, num_pages); an entry outside it reads page 0 instead (in bounds; the outputs of that request
   * are then meaningless) and, when status is not NULL, the pass stores QMLA_ERR_PAGE into *status
   * (device int32) before it ends. The library never clears *status. num_pages == 0: there is no
   * upper bound, so non-negative entries are trusted as the reference trusts them; a negative entry
   * still reads page 0 and stores QMLA_ERR_PAGE into *status. */
  int32_t num_pages;
  int32_t* status;
} qmla_decode_params;

/* ABI version (QMLA_ABI_VERSION) and a static build string. */
int qmla_version(void);
const char* qmla_build_info(void);

/* Workspace bytes qmla_decode needs for these params (0 when no workspace is needed). For
 * num_splits > 0 this is rows*heads*num_splits*(d_c/G + 1)*4; for balanced mode it covers the
 * maximum number of partial segments. Pure host arithmetic, no device access except the
 * compute-unit count of the current device (queried once). */
size_t qmla_workspace_bytes(const qmla_decode_params* p);

/* Decode: scores, online softmax and P.V over the paged latent rows (split-K partials where the
 * split mode needs them) followed by the LSE combine, all on `stream` (a hipStream_t). Rows that see
 * no token get a zero output and lse -inf in every split mode (with num_splits == 1, where no
 * combine runs, a small pass writes the rows of requests of length 0). */
int qmla_decode(const qmla_decode_params* p, void* stream);

/* qmla_decode without a caller workspace, for callers that cannot allocate device memory (code
 * under HIP-graph capture, tight serving loops, harnesses that forbid it). No counterpart in the
 * reference. The split-K scratch (balanced partials, or the fixed-split partials, which are then kept
 * dense and p->ws_stride_* are ignored) lives in a library-owned device array of
 * QMLA_STATIC_SCRATCH_BYTES per GPU, held until the process ends; p->workspace and
 * p->workspace_bytes are ignored. Returns QMLA_ERR_WORKSPACE when qmla_workspace_bytes() of the call
 * exceeds that size (the headline B = 128 decode needs about 19 MB). Allocates nothing. Every call on
 * a GPU shares that GPU's array: calls that overlap on one GPU (two streams, two host threads) race;
 * order them on one stream. Nothing in the array needs to start at zero. */
#define QMLA_STATIC_SCRATCH_BYTES (64 << 20)
int qmla_decode_static(const qmla_decode_params* p, void* stream);

/* The stages of qmla_decode, callable one by one on the same stream and params:
 *   qmla_plan            balanced mode only: per-request tile counts and prefix sums into the
 *                        workspace (one small workgroup; no host involvement). Optional: the
 *                        decode pass derives the same plan itself and stores it for the combine
 *   qmla_decode_partial  the decode pass (stage 1, qwen_mla/ops/mla_decode_attention.py:297-586):
 *                        partials into attn_logits (fixed mode) or the balanced workspace, and the
 *                        final out / lse directly for requests a single workgroup covered (with
 *                        num_splits == 1 all rows, those of requests of length 0 included)
 *   qmla_combine         the LSE merge (stage 2, qwen_mla/ops/mla_decode_attention.py:1064-1137) */
int qmla_plan(const qmla_decode_params* p, void* stream);
int qmla_decode_partial(const qmla_decode_params* p, void* stream);
int qmla_combine(const qmla_decode_params* p, void* stream);

/* The balanced plan's per-request tile count is ceil(L / 64) plus this many tiles for a non-empty
 * request (0 for an empty one): the fixed work of a request piece (query load, output write),
 * charged as tokens so that workgroups holding more pieces get fewer tokens. It depends on the
 * kernel the params select; 0 in fixed-split mode. Negative QMLA_ERR_* for invalid params. No
 * counterpart in the reference (FlashInfer's work split, qwen_mla/fi_decode.py:210-233, counts
 * tokens only). */
int qmla_plan_switch_tiles(const qmla_decode_params* p);

/* QMLA_OK when a compiled kernel serves these params (cache format, rms tail, latent and rope
 * widths, heads, verify tokens per request, groups), else QMLA_ERR_NOKERNEL or the first check that
 * fails. Checks shapes and modes only: the pointers may be NULL. Pure host work. The host side uses
 * it to fold spec-verify rows: the reference folds up to QWEN_MLA_VERIFY_MAX_ROWS rows per request
 * group (qwen_mla/ops/mla_decode_attention.py:1291-1310); here a request's rows may split over up to
 * four workgroups that read its token range together. */
int qmla_decode_supported(const qmla_decode_params* p);

/* ---- cache-row writer ---------------------------------------------------------------------
 * Replaces QwenMLATritonImpl.do_kv_cache_update (qwen_mla/mla_impl.py:309-342) and, for the rows it
 * hands to vLLM (bf16 caches; FP8 caches whose rms is stored as e4m3), vLLM's concat_and_cache_mla:
 * one new token per input row, written at its flat cache slot as
 *   FP8:  [latent e4m3 | rope e4m3 | rms tail | (pad untouched)] with e4m3 = RNE of
 *         clamp(x * (1/k_scale), -448, 448) in fp32; rms tail = log8 code per head
 *         (round-half-even of (log2(max(r, 1e-30)) + 3) * 42.5, clamped to [0, 255]), or the rms
 *         as 2 bf16 bytes per head, or e4m3 like the rope, or nothing;
 *   bf16: [latent | rope | rms (rms_heads elements, or none)] copied.
 * Slot -1 (padding) is redirected to slot 0 (vLLM's never-read null block) as the reference does;
 * slots >= num_slots are skipped. Inputs are bf16. Asynchronous on `stream`, allocates nothing. */
typedef struct qmla_cache_write_params {
  const void* kv_c;               /* [n, d_c] bf16 */
  int64_t kv_c_stride;            /* elements between rows */
  const void* k_pe;               /* [n, rope_w + rms tail] bf16: rope, then the per-head rms */
  int64_t k_pe_stride;
  const int64_t* slots;           /* [n] page * page_size + token */
  int32_t n, d_c, rope_w, rms_heads;
  int32_t kv_dtype;               /* QMLA_KV_FP8 or QMLA_KV_BF16 */
  int32_t rms_mode;               /* FP8: QMLA_RMS_LOG8, _BF16_BYTES, _E4M3, _NONE; bf16: _BF16, _NONE */
  const float* k_scale;           /* FP8: device scalar (per-layer scale) */
  void* cache;                    /* [num_pages, page_size, (1,) row] */
  int64_t page_stride, token_stride;   /* bytes */
  int32_t page_size;
  int64_t num_slots;              /* num_pages * page_size */
} qmla_cache_write_params;

int qmla_cache_write(const qmla_cache_write_params* p, void* stream);

/* ---- prefill context gather -----------------------------------------------------------------
 * Replaces gather_cache_torch (qwen_mla/ops/mla_gather.py:28-76), the plugin's stand-in for vLLM's
 * gather_and_maybe_dequant_cache on the chunked-context prefill path. Destination row j reads
 *   s = token_to_seq[j], tok = j - cu_seq_lens[s] (+ seq_starts[s]), page block_table[s, tok / P],
 * slot tok % P. bf16 caches: the row is copied (row_elems elements). FP8 caches: dst[j, :rms_offset]
 * = e4m3 * scale (fp32 product, rounded to dst's dtype), then one element per head at rms_offset:
 * 2^(-3 + code*6/255) (log8), the raw bf16 (two bytes per head), or e4m3 * scale (e4m3 mode);
 * columns past rms_offset + rms_heads are not written. Rows whose metadata points outside
 * [0, num_seqs), [0, bt_cols) or [0, num_pages) are not written. Asynchronous, allocates nothing. */
typedef struct qmla_gather_params {
  const void* cache;              /* [num_pages, page_size, (1,) row] */
  int64_t page_stride, token_stride;   /* bytes */
  int32_t page_size, num_pages;
  int32_t kv_dtype;               /* QMLA_KV_FP8 or QMLA_KV_BF16 */
  int32_t rms_mode;               /* FP8: QMLA_RMS_LOG8, _BF16_BYTES, _E4M3 */
  int32_t rms_offset, rms_heads;  /* FP8: latent + rope columns, heads of the rms tail */
  int32_t row_elems;              /* bf16: elements copied per row */
  const float* scale;             /* FP8: device scalar */
  const int32_t* block_table;     /* [num_seqs, bt_cols] */
  int64_t bt_stride;
  int32_t num_seqs, bt_cols;
  const int32_t* cu_seq_lens;     /* [num_seqs + 1] first destination row of each sequence */
  const int32_t* token_to_seq;    /* [>= num_tokens] */
  const int32_t* seq_starts;      /* [num_seqs] or NULL: first sequence token of this chunk */
  int32_t num_tokens;
  void* dst;                      /* [>= num_tokens, >= width] */
  int64_t dst_stride;             /* elements between rows */
  int32_t dst_dtype;              /* QMLA_DT_BF16 or QMLA_DT_F16 */
} qmla_gather_params;

int qmla_gather(const qmla_gather_params* p, void* stream);

/* ---- decode q / k_pe prep --------------------------------------------------------------------
 * Replaces the per-token prep of the absorbed-MLA attention module between its projections and the
 * attention call (qwen_mla/qwen3_5_mla.py:262-301, rotation as in :341-354, rope table from
 * qwen_mla/partial_rope.py:52-76), fused into one launch:
 *   rms[t,h]   = sqrt((sum_j bf16(latent[t] . k_up[h*nope + j])^2 + sum_i k_rope[t, g*rd + i]^2)
 *                     / head_dim + eps),  g = (head_offset + h) / rope_group  (fp32)
 *   q_out[t,h] = [ q[t,h, rd:head_dim] | q_pe ],  q_pe (declared_rope wide) zero except the slot
 *                (g - rope_first)*rd .. +rd, which holds rot(q[t,h, :rd])
 *   k_pe[t]    = [ rot(bf16(k_rope[t, g*rd + i] * k_gain[i])) for g in rope_first.. +rope_span |
 *                  bf16(rms[t, :]) | zeros up to declared_rope ]
 * rot is the neox rotation in bf16 arithmetic (each product and sum rounded to bf16) with the
 * cos/sin table row of the token's position rounded to bf16: x1*cos - x2*sin | x2*cos + x1*sin.
 * With pos_rows == 3 (M-RoPE) frequency i takes its position from row rope_sec[i]. Positions
 * outside [0, max_pos) give NaN in the rotated elements. Asynchronous, allocates nothing. */
typedef struct qmla_prep_params {
  const void* q;                  /* bf16 [n, heads, head_dim], the normed query, rope dims first */
  int64_t q_token_stride, q_head_stride;          /* elements */
  const void* latent;             /* bf16 [n, d_c], the cached latent c */
  int64_t latent_stride;
  const void* k_rope;             /* bf16 [n, kv_heads * rope_dim], the raw rope key */
  int64_t k_rope_stride;
  const void* k_up;               /* bf16 [heads * nope, d_c], the raw (unscaled) key up-projection */
  const float* k_gain;            /* fp32 [rope_dim]: 1 + k_norm.weight[:rope_dim] */
  const void* cos_sin;            /* [max_pos, rope_dim] = cos | sin, dtype cos_sin_dtype */
  int32_t cos_sin_dtype;          /* QMLA_DT_BF16, QMLA_DT_F32 or QMLA_DT_F16 */
  int64_t max_pos;
  const int64_t* positions;       /* [pos_rows, n] */
  int64_t pos_row_stride;
  int32_t pos_rows;               /* 1, or 3 for M-RoPE */
  const int32_t* rope_sec;        /* M-RoPE: [rope_dim / 2] position row (0..2) per frequency */
  int32_t n, heads, head_dim, rope_dim, kv_heads, d_c;
  int32_t head_offset, rope_group, rope_first, rope_span, declared_rope;
  float eps;
  void* q_out;                    /* bf16 [n, heads, nope + declared_rope] */
  int64_t q_out_token_stride, q_out_head_stride;
  void* k_pe;                     /* bf16 [n, declared_rope] */
  int64_t k_pe_stride;
} qmla_prep_params;

int qmla_prep(const qmla_prep_params* p, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QMLA_H */
