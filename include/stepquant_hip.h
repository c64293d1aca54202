/*
 * stepquant_hip.h -- C ABI of the MI355X (gfx950) packed-state recurrent update.
 *
 * Plain C: device pointers, sizes and a hipStream_t passed as void*.  No torch
 * types cross this boundary.  Every entry point is asynchronous on the given
 * stream, allocates no device memory, and returns 0 on success, a negative
 * SQ_E* code for invalid arguments, or a positive hipError_t from the launch.
 * sq_last_error() returns a message for the most recent failure.
 *
 * Each entry point replaces one operation of the reference's
 * stepquant.kernels.pool.PackedStatePool (reference paths below are relative
 * to the reference repository).
 */
#ifndef STEPQUANT_HIP_H
#define STEPQUANT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: sq_prefill_args gained `events` and `beta_logits` (and a reserved word) */
#define SQ_ABI_VERSION 2

/* dtype codes for q/k/v/g/beta/out and slot indices */
enum {
    SQ_F32 = 0,
    SQ_BF16 = 1,
    SQ_F16 = 2,
    SQ_I32 = 3,
    SQ_I64 = 4
};

/* error codes (negative; positive values are hipError_t) */
enum {
    SQ_OK = 0,
    SQ_EINVAL = -22,     /* bad argument: null pointer, dtype, shape */
    SQ_ESHAPE = -23,     /* K/V/group combination outside the supported set */
    SQ_ESTORAGE = -24    /* storage variant not supported by this entry point */
};

/*
 * One layer's page pool.  Mirrors the state of PackedStatePool.__init__
 * (pool.py:70-119) and the tables of packed_layout (pool.py:19-66):
 *   data      [num_slots, page_bytes] uint8 pages; the allocation must extend
 *             at least 16 bytes past the last page (aligned over-reads).
 *   bits      [H*K]   per key-row width, 16 = FP16 pivot row
 *   offsets   [H*K+H] packed row byte offsets, then per-head tile strides
 *             (byte storage: per-head code-plane bases)
 *   rows      [H*K]   byte offset of each row's fp16 scale(s), -1 for pivots
 *   columns   [H]     byte offset of each head's fp16 column scales, -1 if none
 *   impact    [H*K]   fit weights w (float32)
 *   head_meta [H*4]   per head: code region start, code region bytes,
 *                     row-scale region start, row-scale region bytes
 *   max_code_bytes    largest code region of any head (LDS staging size)
 *   max_row_bytes     largest row-scale region of any head
 *   flags             sq_pool_flags() of the host copies of the tables
 */
typedef struct sq_pool {
    uint8_t *data;
    int64_t page_bytes;
    int64_t num_slots;
    const int32_t *bits;
    const int32_t *offsets;
    const int32_t *rows;
    const int32_t *columns;
    const float *impact;
    const int32_t *head_meta;
    int32_t heads;        /* H: value heads of this shard */
    int32_t keys;         /* K */
    int32_t values;       /* V */
    int32_t group;        /* value_group_size (GDN 2-bit row scales) */
    int32_t kda;          /* 0: GDN (per-head widths), 1: KDA (per-row widths) */
    int32_t storage;      /* 0: packed, 1: byte carriers */
    int32_t max_code_bytes;
    int32_t max_row_bytes;   /* largest row-scale region of any head */
    int32_t flags;           /* SQ_POOL_* bits, from sq_pool_flags() */
    int32_t reserved;
} sq_pool;

/* sq_pool.flags: the pool qualifies for the K=V=128 uniform-width GDN kernel,
 * or for the K=V=128 KDA kernel */
#define SQ_POOL_FAST_GDN128 1
#define SQ_POOL_FAST_KDA128 2

/*
 * Inputs of one decode step (PackedStatePool.step, pool.py:200-282).
 *   q, k     [B, HK*K] rows with row strides q_stride/k_stride (elements,
 *            non-negative: SQ_EINVAL otherwise);
 *            value head h reads key head h / (H/HK) (GQA).
 *   v        [B, H*V] rows with row stride v_stride (non-negative).
 *   g        GDN: [B, H] log-decay (raw gate a when a_log != NULL);
 *            KDA: [B, H*K] per-channel values.
 *   beta     [B, H] (raw logits when a_log != NULL: beta = sigmoid(b)).
 *   a_log    [H] or NULL; dt_bias [H] (GDN) or [H*K] (KDA), with a_log.
 *   out      [B, H, V] contiguous, dtype out_dtype; slot <= 0 rows are zero.
 *   slots    [B] page indices, dtype slots_dtype (SQ_I32 or SQ_I64).
 */
typedef struct sq_step_args {
    const void *q;
    const void *k;
    const void *v;
    const void *g;
    const void *beta;
    const void *a_log;
    const void *dt_bias;
    void *out;
    const void *slots;
    int64_t batch;
    int64_t q_stride;
    int64_t k_stride;
    int64_t v_stride;
    int32_t key_heads;   /* HK */
    int32_t qkv_dtype;   /* dtype of q, k, v */
    int32_t gate_dtype;  /* dtype of g, beta, a_log, dt_bias */
    int32_t out_dtype;
    int32_t slots_dtype;
    int32_t normalize;   /* L2-normalise q and k (eps 1e-6) */
    float scale;         /* query scale */
    int32_t reserved;
} sq_step_args;

/*
 * Writer hand-off of the asynchronous path (the reference keeps the same
 * four tensors in PackedStatePool.scratch, pool.py:137-158):
 *   key [B,H,K] f32 prepared keys, decay [B,H,K] f32 per-row retention,
 *   delta [B,H,V] f32, stable_slots [B] int64 snapshot of the slot indices.
 */
typedef struct sq_writeback_scratch {
    float *key;
    float *decay;
    float *delta;
    int64_t *stable_slots;
    int64_t capacity;    /* rows available in each buffer (>= batch) */
} sq_writeback_scratch;

/* ABI version, and the message for the most recent non-zero return. */
int sq_abi_version(void);
const char *sq_last_error(void);

/*
 * Dense fp32 state [B,H,K,V] -> pages of `slots`, requantised exactly as the
 * reference CPU fit_state (quantization.py:54-98): codes, row/column scales
 * and FP16 pivots bit-identical.  Replaces PackedStatePool.encode
 * (pool.py:184-190 -> _writeback, pool.py:319-331).
 */
int sq_encode(const sq_pool *pool, const float *state, const void *slots, int32_t slots_dtype,
              int64_t batch, void *stream);

/*
 * Pages of `slots` -> dense fp32 state [B,H,K,V] (zeros for slot <= 0).
 * Replaces PackedStatePool.decode (pool.py:192-198, codec_kernel fused.py:50-59).
 */
int sq_decode_dense(const sq_pool *pool, const void *slots, int32_t slots_dtype, int64_t batch,
                    float *state, void *stream);

/*
 * Fused decode step: one pass reads each (request, head) page tile, applies
 * the gated delta update, writes the readout and writes back the requantised
 * tile.  Replaces PackedStatePool.step without a writeback stream
 * (pool.py:200-282 with update_kernel fused.py:182-248 and _writeback
 * pool.py:319-331).
 */
int sq_decode_step(const sq_pool *pool, const sq_step_args *args, void *stream);

/*
 * Asynchronous split of the same step.  sq_decode_readout runs on the
 * foreground stream: readout `out`, plus the writer hand-off in `scratch`
 * (replaces the readers readout.py:7-121 / segment_read.py:6-104).
 * sq_writeback runs on the writeback stream after it: it re-reads the old
 * tile and stores the requantised one (replaces prepare_rows_kernel
 * rows.py:52-63 + fit fit.py:152-167 in _finish_update, pool.py:299-316).
 */
int sq_decode_readout(const sq_pool *pool, const sq_step_args *args,
                      const sq_writeback_scratch *scratch, void *stream);
int sq_writeback(const sq_pool *pool, const sq_writeback_scratch *scratch, int64_t batch,
                 void *stream);

/*
 * Chunked prefill of whole sequences (replaces the decode -> upstream chunk
 * kernel -> encode round trip of kernel_extend, sglang/runtime.py:193-202).
 *   q, k      [T, HK*K] bf16 rows (row strides in elements, multiples of 8,
 *             rows 16-byte aligned); v [T, H*V] bf16; T = cu_seqlens[batch].
 *   g, beta   [T, H] log decay and write strength.  With a_log/dt_bias, g
 *             is the raw gate a and the log decay is
 *             -exp(a_log[h]) * softplus(a + dt_bias) (softplus threshold 20),
 *             as sq_step_args.  KDA pools: g [T, H, K], one value per key
 *             channel, dt_bias [H * K].
 *   beta_logits  1: beta holds logits b and the write strength is
 *             sigmoid(b) (the decode hooks' convention); 0: beta is the
 *             write strength itself (the chunk kernels' convention).
 *             Independent of a_log.
 *   out       [T, H, V], dtype out_dtype.
 *   cu_seqlens [batch + 1] int32 token offsets of the sequences.
 *   init_slots [batch] pages holding the initial states (slot <= 0: zero
 *             state; NULL: all zero).
 *   checkpoints [batch * n_checkpoints] int32 token counts, ascending per
 *             sequence, after which the state is requantised into
 *             slots[b * n_checkpoints + c] (positions <= 0 or beyond the
 *             sequence are unused and their slots must be <= 0).
 *   init_state      workspace [batch, H, K, V] f32 for the decoded initial
 *             states; pools flagged SQ_POOL_FAST_GDN128 or
 *             SQ_POOL_FAST_KDA128 are decoded inside the recurrence kernel
 *             from init_slots' pages (to the same bits), leave it untouched
 *             and accept NULL;
 *   checkpoint_state workspace [batch * n_checkpoints, H, K, V] f32.
 *   events    NULL, or two hipEvent_t recorded on the stream right before
 *             and after the recurrence kernel (a timing hook for
 *             benchmarks; the reference's kernel_extend has no
 *             counterpart).
 * Pools with K = V = 128, packed or byte storage.  GDN: the chunked kernel
 * (chunks of 64 tokens, bf16 MFMA).  KDA: a chunked kernel with per-channel
 * decays (chunks of 32 tokens, bf16 MFMA; in-chunk decays formed pairwise
 * when a chunk's decay exceeds 2^96 on some channel).
 */
typedef struct sq_prefill_args {
    const void *q;
    const void *k;
    const void *v;
    const void *g;
    const void *beta;
    const void *a_log;
    const void *dt_bias;
    void *out;
    const int32_t *cu_seqlens;
    const int32_t *checkpoints;
    const void *init_slots;
    const void *slots;
    float *init_state;
    float *checkpoint_state;
    int64_t batch;
    int64_t q_stride;
    int64_t k_stride;
    int64_t v_stride;
    int32_t key_heads;
    int32_t n_checkpoints;
    int32_t qkv_dtype;
    int32_t gate_dtype;
    int32_t out_dtype;
    int32_t slots_dtype;
    int32_t normalize;
    float scale;
    void *const *events;
    int32_t beta_logits;
    int32_t reserved;
} sq_prefill_args;

int sq_prefill(const sq_pool *pool, const sq_prefill_args *args, void *stream);

/*
 * Slot operations (pool.py:358-365).  sq_clear_slots zeroes whole pages.
 * sq_copy_slots copies pages src[i] -> dst[i] through `temp`
 * ([n, page_bytes] bytes) so overlapping index sets behave like the
 * reference's gather-then-scatter.  Negative indices wrap like Python; a
 * pair whose source or destination lies outside the pool is skipped.
 * Only data, page_bytes and num_slots of `pool` are read, so format pools
 * pass an sq_pool holding just those.
 */
int sq_clear_slots(const sq_pool *pool, const void *slots, int32_t slots_dtype, int64_t n,
                   void *stream);
int sq_copy_slots(const sq_pool *pool, const void *src, const void *dst, int32_t slots_dtype,
                  int64_t n, uint8_t *temp, void *stream);

/*
 * No counterpart in the reference.  sq_copy_slots without the `temp`
 * argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the pages are staged in a static device array of
 * SQ_COPY_STATIC_BYTES bytes that the library holds on every GPU it runs
 * on until the process ends.  n * page_bytes above that size is rejected
 * with SQ_EINVAL; nothing is allocated or freed.  Every call on one GPU
 * shares that GPU's array, so calls that overlap on one GPU (concurrent
 * streams, or host threads) race; calls ordered on one stream do not.
 */
#define SQ_COPY_STATIC_BYTES (16u << 20)
int sq_copy_slots_static(const sq_pool *pool, const void *src, const void *dst, int32_t slots_dtype,
                         int64_t n, void *stream);

/*
 * Baseline state formats: one layer's pool of FormatStatePool pages
 * (reference kernels/format_pool.py:29-128; layout format_layout,
 * format_pool.py:9-25).  Every row of the pool has the same code width.
 *   kind      SQ_FMT_FP32 (fp32 state, bits = 32), SQ_FMT_SYMMETRIC (per row
 *             and 128-value group: fp16 scale and zero point, bits 4/6/8) or
 *             SQ_FMT_DSQ (fp16 row and column scales, bits 4/6/8)
 *   offsets   [H*K] byte offset of each row's codes (fp32 values)
 *   rows      [H*K] byte offset of each row's fp16 metadata (unused for FP32)
 *   columns   [H]   byte offset of each head's column metadata (DSQ)
 * K is a power of two <= 128; V a power of two >= 4 (SYMMETRIC: a multiple
 * of 128; DSQ: <= 128).
 */
enum {
    SQ_FMT_FP32 = 0,
    SQ_FMT_SYMMETRIC = 1,
    SQ_FMT_DSQ = 2
};

typedef struct sq_format_pool {
    uint8_t *data;
    int64_t page_bytes;
    int64_t num_slots;
    const int32_t *offsets;
    const int32_t *rows;
    const int32_t *columns;
    int32_t heads;
    int32_t keys;
    int32_t values;
    int32_t kind;       /* SQ_FMT_* */
    int32_t bits;       /* code width (32 for SQ_FMT_FP32) */
    int32_t group;      /* value group of SQ_FMT_SYMMETRIC (128) */
    int32_t kda;        /* 1: per-key-row retention g [B, H*K] */
    int32_t flags;      /* SQ_FMT_ROWS_CONTIGUOUS: offsets[h*K + i] = offsets[0] + (h*K + i) * V * bits / 8 */
} sq_format_pool;

#define SQ_FMT_ROWS_CONTIGUOUS 1

/*
 * Dense fp32 [B,H,K,V] -> pages (FormatStatePool.encode, format_pool.py:68-80);
 * bit-identical to the CPU group_fit / dual_fit (formats.py:53-86) of the
 * same input.  Pages -> dense fp32 (FormatStatePool.decode,
 * format_pool.py:82-90).  One fused decode step: read, gated delta update,
 * readout, re-encode (FormatStatePool.step, format_pool.py:92-113).  The
 * step's arguments are those of sq_decode_step.
 */
int sq_format_encode(const sq_format_pool *pool, const float *state, const void *slots,
                     int32_t slots_dtype, int64_t batch, void *stream);
int sq_format_decode(const sq_format_pool *pool, const void *slots, int32_t slots_dtype,
                     int64_t batch, float *state, void *stream);
int sq_format_step(const sq_format_pool *pool, const sq_step_args *args, void *stream);

/*
 * Flags for sq_pool.flags, computed from host copies of bits [H*K],
 * head_meta [H*4] and columns [H].  Returns a non-negative flag set, or a
 * negative SQ_E* code.  Host-only; no device access.
 */
int sq_pool_flags(const int32_t *bits, const int32_t *head_meta, const int32_t *columns, int32_t heads,
                  int32_t keys, int32_t values, int32_t group, int32_t kda, int32_t storage,
                  int64_t page_bytes);

/*
 * Capture state of a stream for the writer's event bookkeeping: capturing is
 * 0 (not capturing), 1 (active) or 2 (invalidated); id identifies the
 * capture.  Replaces _capture_id (pool.py:11-16, cudaStreamGetCaptureInfo).
 */
int sq_stream_capture_id(void *stream, int32_t *capturing, uint64_t *id);

/*
 * Events that order work across graphs, the role of the reference's
 * external events (torch.cuda.Event(external=True) and cudaEventRecordExternal
 * / cudaEventWaitExternal nodes: pool.py:131-135, 338-355; writeback.py:43,
 * 103, 110-116).  sq_event_record / sq_event_wait act on `stream` now when it
 * is not capturing; on a capturing stream they add an event record / wait
 * node to the capture's graph after the stream's current dependencies, so
 * every replay records the event, or waits for its latest record.
 * sq_event_query returns 0 when the event's work is done and 1 when it is
 * not.  Events are created without timing.
 */
int sq_event_create(void **event);
int sq_event_destroy(void *event);
int sq_event_record(void *event, void *stream);
int sq_event_wait(void *stream, void *event);
int sq_event_query(void *event);
int sq_event_synchronize(void *event);

/*
 * A stream restricted to `cus` compute units spread across all XCDs
 * (hipExtStreamCreateWithCUMask), at default priority.  A restricted stream
 * is a blocking stream (hipExtStreamCreateWithCUMask takes no flags), so work
 * on the legacy default stream waits for it; cus == 0 or cus equal to the
 * device's CU count gives an unrestricted non-blocking stream.  Replaces the
 * Green Context SM split of writeback_resources (kernels/resources.py:19-53).
 * The stream lives until process exit.
 */
int sq_create_cu_stream(int32_t device, int32_t cus, void **stream, int32_t *actual, int32_t *total);

#ifdef __cplusplus
}
#endif

#endif /* STEPQUANT_HIP_H */
