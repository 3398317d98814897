/*
 * C ABI of the MI355X (gfx950) Gated DeltaNet decode library, liblightdelta_hip.so.
 *
 * Every entry point takes plain pointers, element/byte strides and sizes, plus the
 * HIP stream (hipStream_t passed as void*) to launch on.  Nothing here allocates,
 * synchronises the host or reads device metadata on the host, so every launch can be
 * recorded into a HIP graph.  All entry points return 0 on success and a non-zero
 * LD_ERR_* code otherwise; ld_last_error() then returns a message for the calling
 * thread.  Empty work (zero requests / rows / pairs) is a successful no-op.
 *
 * Tensors are caller-owned device memory.  bf16 values are raw uint16 bit patterns.
 */
#ifndef LIGHTDELTA_HIP_H
#define LIGHTDELTA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LD_ABI_VERSION 12

#define LD_OK 0
#define LD_ERR_INVALID_ARGUMENT 1
#define LD_ERR_LAUNCH 2

#define LD_DTYPE_F32 0
#define LD_DTYPE_BF16 1

/* State cache policy of ld_gdn_decode / ld_gdn_decode_conv (kernel shape and cache hints of
 * the state traffic; never a change of results).  KEEP: tuned for a working set that stays in
 * the 256 MB Infinity Cache until the next step (one layer stepped repeatedly).  STREAM: tuned
 * for working sets far larger than the caches (many layers between two steps of one layer):
 * non-temporal loads and system-scope stores for one token. */
#define LD_CACHE_KEEP 0
#define LD_CACHE_STREAM 1

/* Head geometry fixed by the kernels: dk = dv = 128. */
#define LD_HEAD_DIM 128
/* Tokens per request accepted by the decode / MTP-verify step. */
#define LD_MAX_TOKENS 4

/*
 * Arguments of one fused post-conv GDN decode / MTP-verify step.
 *
 * Replaces lightdelta::decode (reference include/lightdelta/ops.h:5-9, launcher
 * csrc/gdn_decode.cu:360-420, kernel csrc/gdn_decode.cu:130-354), generalised from
 * the hard-coded 16/48 heads to any num_k_heads / num_v_heads with
 * num_v_heads % num_k_heads == 0.
 *
 * Element strides (not bytes).  Layouts:
 *   qkv     bf16 [tokens, (2*H + HV)*128], row stride qkv_row_stride, unit column stride;
 *           q of k-head kh at column kh*128, k at H*128 + kh*128, v of v-head h at 2*H*128 + h*128
 *   a, b    bf16 [tokens, HV], row strides a_row_stride / b_row_stride
 *   a_log   fp32 [HV]; dt_bias fp32 or bf16 [HV] (dt_bias_dtype)
 *   indices int32 [requests, width] contiguous; cu int32 [requests+1]; accepted int32 [requests]
 *   state   fp32 [slots, HV, 128(V), 128(K)], K contiguous, slot stride state_slot_stride
 *   gate    bf16 [tokens, HV, 128], row stride gate_row_stride, head stride 128
 *   norm_weight fp32 or bf16 [128] (norm_weight_dtype)
 *   out     bf16 [tokens, HV, 128] contiguous
 * Request r covers tokens cu[r] .. cu[r+1]-1.  Its source state is slot
 * indices[r, accepted[r]-1] when 1 <= accepted[r] <= width; the state after token t is
 * written to slot indices[r, t].  A slot <= 0 is padding: never read, never written.
 * A request with an invalid source, or with more tokens than width, gets zero outputs
 * and leaves the pool untouched; a request with no tokens writes nothing.
 */
typedef struct ld_gdn_decode_args {
  const void* qkv;
  int64_t qkv_row_stride;
  const void* a;
  int64_t a_row_stride;
  const void* b;
  int64_t b_row_stride;
  const float* a_log;
  const void* dt_bias;
  int32_t dt_bias_dtype;
  int32_t norm_weight_dtype;
  const int32_t* indices;
  const int32_t* cu;
  const int32_t* accepted;
  float* state;
  int64_t state_slot_stride;
  const void* gate;
  int64_t gate_row_stride;
  const void* norm_weight;
  void* out;
  int32_t num_requests;
  int32_t width;
  int32_t num_k_heads;
  int32_t num_v_heads;
  float scale;          /* q scale, 128^-0.5 in the reference (csrc/gdn_decode.cu:417) */
  float eps;            /* gated RMSNorm epsilon, > 0 */
  int32_t cache_policy; /* LD_CACHE_KEEP or LD_CACHE_STREAM (no effect on results) */
} ld_gdn_decode_args;

/* Fused decode step; see ld_gdn_decode_args.  Replaces lightdelta::decode
 * (reference include/lightdelta/ops.h:5-9, csrc/gdn_decode.cu:360-420). */
int ld_gdn_decode(const ld_gdn_decode_args* args, void* stream);

/*
 * Pre-conv inputs and conv-state pool of the conv-fused step (ld_gdn_decode_conv).
 *   x       bf16 [tokens, conv_dim] pre-conv activations (conv_dim = (2*H + HV)*128, the
 *           same column layout as the post-conv qkv), row stride x_row_stride, unit column
 *           stride
 *   state   bf16 conv-state pool of `state_slots` slots; element (slot, channel, column) at
 *           slot*state_slot_stride + channel*state_dim_stride + column*state_len_stride
 *           (vLLM's dim-first [slots, conv_dim, len] and dim-last [slots, len, conv_dim]
 *           layouts are both covered); column state_len-1 is the most recent input
 *   weight  bf16 [conv_dim, width] contiguous, 8-byte aligned; bias bf16 [conv_dim] or NULL
 * Element strides.  width must be 4 and 3 <= state_len <= 8.  The conv slot of request r is
 * indices[r, 0], the slot its SSM state lives in.
 */
typedef struct ld_conv_args {
  const void* x;
  int64_t x_row_stride;
  void* state;
  int64_t state_slots;
  int64_t state_slot_stride;
  int64_t state_dim_stride;
  int64_t state_len_stride;
  int32_t state_len;
  int32_t width;
  const void* weight;
  int32_t weight_dtype;
  int32_t bias_dtype;
  const void* bias;
} ld_conv_args;

/*
 * Conv-fused decode / speculative-verify step (args->qkv is not read; `conv->x` holds the
 * pre-conv activations).  Per request with n tokens, the causal depthwise conv1d (width 4,
 * plus bias, SiLU, rounded to bf16) runs over the 3 conv-state columns from accepted - 1
 * followed by the n new inputs, and its outputs become the tokens' q/k/v; the conv state of
 * slot indices[r, 0] becomes its columns accepted .. accepted + state_len - n - 1 followed by
 * the n inputs (vLLM's causal_conv1d_update with num_accepted_tokens; n = 1, accepted = 1
 * is the plain one-column shift); then the GDN step of ld_gdn_decode runs.  Requests that
 * are invalid for the GDN step, or whose conv columns would fall outside the state
 * (accepted - 1 + 2 > state_len - 1, or accepted > n < state_len), or whose conv slot
 * indices[r, 0] is padding, get zero outputs and leave both pools untouched.  Conv slots
 * must be distinct within one launch, and launches that use the same slot id must be
 * stream-ordered, whatever conv pools they pass: the v-heads of a k-head group decide which
 * of them writes the shared q/k conv state with one ticket per (slot id, k-head) in
 * library-owned device memory (slots x k-heads at most 2^20), and the tickets are keyed by
 * slot id alone, so every layer and every conv pool of the process shares them.  Launches of
 * different layers on one stream (the serving step, a captured graph of it) are ordered
 * already; two launches in flight at once on different streams must use disjoint slot ids
 * even when their pools differ.  Either violation makes those launches' conv states
 * undefined; the tickets themselves return to their state, so later launches are unaffected.
 * No counterpart in the reference, whose conv is vLLM's causal_conv1d_update run before
 * lightdelta::decode (python/lightdelta/integration/vllm_layer.py:150-172, 199-220).
 */
int ld_gdn_decode_conv(const ld_gdn_decode_args* args, const ld_conv_args* conv, void* stream);

/*
 * Prefill of N sequences (varlen, one token per row of qkv; sequence n covers rows
 * cu_seqlens[n] .. cu_seqlens[n+1]-1).  Per (sequence, v-head): the state starts from
 * state[slots[n]] when slots[n] > 0 and has_initial[n] != 0, else from zeros; every token
 * runs the decode recurrence (same numerics as ld_gdn_decode, token by token) and writes
 * its gated-RMSNorm output to out[row]; the state after the last token is written to
 * state[slots[n]] when slots[n] > 0 (an empty sequence writes its initial state back).
 * Layouts as ld_gdn_decode (qkv, a, b, gate, out row strides; state [slots, HV, 128,
 * 128]); has_initial is one byte per sequence; cu_seqlens is trusted device metadata
 * (non-decreasing, sequences contiguous from cu_seqlens[0]).  Algorithms with the same
 * contract: token-serial (the decode's arithmetic, token by token; a head's state rows are
 * split over several workgroups when sequences x heads are too few to fill the GPU) and
 * chunked (chunks of 64 or 32 tokens in the WY form on the matrix cores; faster unless the
 * prompts are very short; results within rounding of the token-serial ones).  Either may
 * run the norm as a second launch on the same stream.
 * Replaces the reference's prefill composition (python/lightdelta/integration/
 * vllm_layer.py:93-135: fused_post_conv_prep, gather_state with has_initial_state,
 * chunk_gated_delta_rule, scatter_state, gated RMSNorm) in one launch.
 */
typedef struct ld_gdn_prefill_args {
  const void* qkv;
  int64_t qkv_row_stride;
  const void* a;
  int64_t a_row_stride;
  const void* b;
  int64_t b_row_stride;
  const float* a_log;
  const void* dt_bias;
  int32_t dt_bias_dtype;
  int32_t norm_weight_dtype;
  const int32_t* slots;
  const uint8_t* has_initial;
  const int32_t* cu_seqlens;
  float* state;
  int64_t state_slot_stride;
  const void* gate;
  int64_t gate_row_stride;
  const void* norm_weight;
  void* out;
  int64_t num_tokens;  /* rows of qkv / out (cu_seqlens[num_sequences] <= num_tokens) */
  int32_t num_sequences;
  int32_t num_k_heads;
  int32_t num_v_heads;
  float scale;
  float eps;
  int32_t algorithm;       /* LD_PREFILL_AUTO / _TOKEN_SERIAL / _CHUNKED / _CHUNKED_32 */
  void* workspace;         /* device memory for the chunked form (NULL: not used) */
  int64_t workspace_bytes;
} ld_gdn_prefill_args;

#define LD_PREFILL_AUTO 0         /* the form ld_gdn_prefill_auto_chunked names, if the workspace fits */
#define LD_PREFILL_TOKEN_SERIAL 1 /* the decode recurrence token by token */
#define LD_PREFILL_CHUNKED 2      /* chunks of 64 tokens in the WY form (needs the workspace) */
#define LD_PREFILL_CHUNKED_32 3   /* chunks of 32 tokens in the WY form (needs the workspace) */

int ld_gdn_prefill(const ld_gdn_prefill_args* args, void* stream);

/* Bytes of the static device scratch of ld_gdn_prefill_static (64 MiB per GPU). */
#define LD_PREFILL_STATIC_SCRATCH_BYTES (64LL << 20)

/*
 * ld_gdn_prefill without any allocation by anyone: the chunked form's workspace is a static
 * device array of LD_PREFILL_STATIC_SCRATCH_BYTES in this library (one per GPU it runs on,
 * held until the process ends) instead of args->workspace, which must be NULL with
 * workspace_bytes 0.  Same contract and results as ld_gdn_prefill otherwise: LD_PREFILL_AUTO
 * takes the chunked form when the shape favours it and its workspace
 * (ld_gdn_prefill_workspace_bytes) fits the scratch, else the token-serial one;
 * LD_PREFILL_CHUNKED beyond the scratch is rejected with LD_ERR_INVALID_ARGUMENT.  The
 * stream must belong to the current device.  Calls on one GPU share its scratch: calls that
 * overlap in time on one GPU race (stream-order them).  The first call on a device looks the
 * scratch up (hipGetSymbolAddress); make it before a graph capture.  Calls no hipMalloc and no
 * allocating routine.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
int ld_gdn_prefill_static(const ld_gdn_prefill_args* args, void* stream);

/*
 * Workspace bytes the chunked prefill needs for num_tokens rows in num_sequences sequences
 * and num_v_heads heads: one 115,712-byte record per chunk of 64 tokens and head (chunks
 * bounded by num_tokens / 64 + num_sequences), then a chunk index of num_sequences + 1
 * int32 rounded up to 256 bytes; the 32-token form's 54,272-byte records per 32 tokens fit
 * in the same bytes.  0 for negative arguments.
 */
int64_t ld_gdn_prefill_workspace_bytes(int64_t num_tokens, int32_t num_sequences,
                                       int32_t num_v_heads);

/*
 * The tokens per chunk LD_PREFILL_AUTO runs for this shape (given a workspace), 64 or 32, or
 * 0 when it runs the token-serial form.  With L = num_tokens / num_sequences: 0 for L < 17;
 * 64 for L >= 512 in fewer than 64 (sequence, head) pairs; else 32.
 * Callers use it to decide whether to provide the workspace.  No counterpart in the
 * reference (its prefill always runs chunk_gated_delta_rule).
 */
int32_t ld_gdn_prefill_auto_chunked(int64_t num_tokens, int32_t num_sequences,
                                    int32_t num_v_heads);

/*
 * Gather pool rows into a packed buffer:
 *   out[r] = (slots[r*slot_stride] > 0 && valid[r]) ? pool[slots[r*slot_stride]] : 0
 * Byte-generic (serves the fp32 SSM pool and the bf16 conv pool).  row_bytes, both
 * row strides and both base pointers must be multiples of 16 bytes.  valid is a bool
 * (one byte per row) vector, or NULL for "all valid".
 * Replaces lightdelta::gather_state (reference include/lightdelta/ops.h:10-11,
 * csrc/state_io.cu:44-58).
 */
int ld_state_gather(const void* pool, int64_t pool_slot_stride_bytes,
                    const int32_t* slots, int64_t slot_stride, const uint8_t* valid,
                    void* out, int64_t out_row_stride_bytes, int64_t row_bytes,
                    int64_t rows, void* stream);

/*
 * Scatter packed rows into the pool, skipping padding:
 *   if slots[r*slot_stride] > 0: pool[slots[r*slot_stride]] = packed[r]
 * Same alignment rules as ld_state_gather.  Replaces lightdelta::scatter_state
 * (reference include/lightdelta/ops.h:12, csrc/state_io.cu:60-69).
 */
int ld_state_scatter(const void* packed, int64_t packed_row_stride_bytes,
                     const int32_t* slots, int64_t slot_stride, void* pool,
                     int64_t pool_slot_stride_bytes, int64_t row_bytes, int64_t rows,
                     void* stream);

/*
 * Slot-to-slot copy inside one pool for `pairs` (src, dst) pairs:
 *   if src_slots[p] > 0 && dst_slots[p] > 0: pool[dst_slots[p]] = pool[src_slots[p]]
 * A pair whose slots overlap another live pair's -- its source is another pair's
 * destination (a chain a->b, b->c), or its destination is another pair's source or
 * destination -- is rejected and writes nothing; every other pair is copied from the pool
 * as it was before the call.  Each workgroup scans the pair list for its own pair, so the
 * cost grows with pairs^2 / 256 (a few percent at 1024 pairs of 2 MiB).
 * No counterpart in the reference (which commits MTP states implicitly through the
 * next step's `accepted`, csrc/gdn_decode.cu:154-158); it is the explicit commit /
 * slot-lifecycle copy, with the reference's padding convention (slot <= 0).
 */
int ld_state_copy(void* pool, int64_t pool_slot_stride_bytes, const int32_t* src_slots,
                  const int32_t* dst_slots, int64_t pairs, int64_t slot_bytes,
                  void* stream);

/*
 * ld_state_copy that also reports which pairs it rejected: rejected[p] (device int32, one
 * entry per pair) becomes 1 for a pair rejected for overlapping another live pair, and 0 for
 * a pair that was copied or is padding.  Every entry is written on every call, so the array
 * needs no clearing (no memset node in a captured graph); sum it for a count.  slot_bytes
 * must be positive.  No counterpart in the reference: the commit copy is additive (see
 * ld_state_copy), and this variant gives callers whose pair sets may chain, swap or share a
 * destination a graph-safe signal instead of a silent skip.
 */
int ld_state_copy_checked(void* pool, int64_t pool_slot_stride_bytes, const int32_t* src_slots,
                          const int32_t* dst_slots, int64_t pairs, int64_t slot_bytes,
                          int32_t* rejected, void* stream);

/*
 * Zero-fill `count` whole slots of a pool in place:
 *   if slots[i] > 0: pool[slots[i]] = 0   (all slot_bytes bytes)
 * Same alignment rules as ld_state_gather (pool base, slot stride and slot_bytes multiples
 * of 16 bytes).  No counterpart in the reference (there a reused slot is re-initialised
 * through gather_state's zero fill of rows whose `valid` flag is false,
 * csrc/state_io.cu:17-25, python/lightdelta/backend.py:41-44); it resets slots of the pool
 * itself for a new sequence, with the padding convention (slot <= 0 skipped).
 */
int ld_state_zero(void* pool, int64_t pool_slot_stride_bytes, const int32_t* slots,
                  int64_t count, int64_t slot_bytes, void* stream);

/*
 * The packed state-access path's bookkeeping for `batch` requests with `width` slots each,
 * in one launch (all arrays device memory; slots [batch, width] contiguous, cu [batch + 1],
 * accepted [batch]; outputs source [batch], valid [batch] (0/1 bytes), indices
 * [batch, width], destinations [batch * width]):
 *   source[r]   = slots[r, clamp(accepted[r], 1, width) - 1]
 *   valid[r]    = 1 <= accepted[r] <= width and source[r] > 0
 *   indices[r, t] = valid[r] ? 1 + r * width + t : 0   (request r's rows of a scratch pool
 *                                                       whose row 0 is padding)
 *   destinations[r * width + t] = t < cu[r + 1] - cu[r] and valid[r] and slots[r, t] > 0
 *                                 ? slots[r, t] : 0
 * Then ld_state_gather(pool -> scratch[1 + r * width], source, valid), ld_gdn_decode on the
 * scratch with `indices` and accepted = 1, and ld_state_scatter(scratch[1:] ->
 * destinations) make the packed step.  Replaces the Torch index arithmetic of the
 * reference's packed path (python/lightdelta/backend.py:39-47, 87-91); no allocation, no
 * host read of device memory (graph-capturable).
 */
int ld_packed_plan(const int32_t* slots, const int32_t* cu, const int32_t* accepted,
                   int32_t batch, int32_t width, int32_t* source, uint8_t* valid,
                   int32_t* indices, int32_t* destinations, void* stream);

/* Message for the last non-zero return on the calling thread ("" if none). */
const char* ld_last_error(void);

/* LD_ABI_VERSION of the loaded library. */
int ld_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LIGHTDELTA_HIP_H */
