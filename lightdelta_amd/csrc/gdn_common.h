// Device-side definitions shared by the decode / verify / prefill kernels (gdn_decode.hip)
// and the chunked prefill (prefill_chunked.hip): the tile geometry, the kernel parameters,
// and the per-token scalar math.
#pragma once

#include "common.h"

namespace ld {

constexpr int kDim = LD_HEAD_DIM;
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kPieces = 16;        // 16-byte pieces of the tile per lane
constexpr int kMaxTokens = LD_MAX_TOKENS;

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct DecodeParams {
  const uint16_t* qkv;
  int64_t qkv_row;
  const uint16_t* a;
  int64_t a_row;
  const uint16_t* b;
  int64_t b_row;
  const float* a_log;
  const void* dt_bias;
  const int32_t* indices;
  const int32_t* cu;
  const int32_t* accepted;
  const uint8_t* has_initial;  // prefill only: per sequence, 0 = start from a zero state
  float* state;
  int64_t state_slot;
  const uint16_t* gate;
  int64_t gate_row;
  const void* norm_weight;
  uint16_t* out;
  int32_t width;
  int32_t num_k_heads;
  int32_t num_v_heads;
  int32_t group;  // num_v_heads / num_k_heads
  float scale;
  float eps;
  // Conv-fused variant only (pre-conv activations and the conv-state pool).
  const uint16_t* conv_x;
  int64_t conv_x_row;
  uint16_t* conv_state;
  int64_t conv_slot;
  int64_t conv_dim_stride;
  int64_t conv_len_stride;
  int32_t conv_len;
  const uint16_t* conv_weight;  // [conv_dim, 4]
  const uint16_t* conv_bias;    // [conv_dim] or NULL
  bool conv_packed;             // host-side: dense dim-first, 16-byte aligned conv pool
};

// ---- state-tile traffic through buffer resources -------------------------------------------
//
// Cache-policy bits of gfx950 vector memory instructions: sc0 = 1, nt = 2, sc1 = 16.  On a
// store, sc0|sc1 (system scope) writes the line through the XCD's L2 instead of leaving it
// dirty there; the Infinity Cache still keeps it.  nt marks the access as streaming.  For the
// in-place read-modify-write of 64 KiB tiles at random slots, cache-cold, non-temporal
// system-scope stores (nt|sc0|sc1) measured fastest of the combinations of these bits, for
// every decode shape (B=128 single token 90.3 -> 88.8 us against system scope alone; the
// conv-fused step 94.2 -> 90.6 us against non-temporal alone), with the load bits within
// noise of each other.
constexpr int kPolPlain = 0;
constexpr int kPolNT = 2;
constexpr int kPolSys = 1 | 16;
constexpr int kPolNTSys = kPolNT | kPolSys;  // streaming, written through to memory
constexpr int kTileBytes = kDim * kDim * 4;

// A raw (untyped) buffer resource over `bytes` bytes at `base`.  Accesses at byte offsets at
// or past `bytes` are dropped by the hardware (loads return 0, stores write nothing), so a
// resource over 0 bytes is a store sink.  Word 3 is the gfx9-family raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

template <int Pol>
__device__ __forceinline__ f32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, Pol));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int Pol>
__device__ __forceinline__ void buffer_store16(f32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t offset) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, offset, 0, Pol);
}

__device__ __forceinline__ float load_param(const void* p, int i, bool bf16) {
  return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i])
              : static_cast<const float*>(p)[i];
}

// The per-token scalars and norms below use the hardware approximations (v_exp_f32,
// v_log_f32, v_rcp_f32, v_rsq_f32; about 1 ulp): they sit between the arrival of the data
// and the first state update of every wave, where exactly rounded sequences cost ~1 us per
// step, and their error (~1e-7 relative) is four orders of magnitude below the bf16 output
// resolution.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }

__device__ __forceinline__ float sigmoid(float x) { return fast_rcp(1.0f + __expf(-x)); }

__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }

// softplus with the threshold torch's F.softplus uses (beta=1, threshold=20); log1p(y) for
// small y = e^x by its series, where log(1 + y) would lose y to the rounding of 1 + y.
__device__ __forceinline__ float softplus(float x) {
  if (x > 20.0f) return x;
  const float y = __expf(x);
  return y < 1e-4f ? y * (1.0f - 0.5f * y) : __logf(1.0f + y);
}

// Chunked prefill (prefill_chunked.hip): workspace bytes for num_tokens rows in
// num_sequences sequences and num_v_heads heads, and the launch of its three phases; the
// raw outputs go to p.out for prefill_norm_kernel.
// The form AUTO runs, from the mean prompt length L = num_tokens / num_sequences, measured
// on MI355X over 1 x 8 .. 4096 x 8 tokens at 32 v heads (ms, token-serial / 64-token
// chunks / 32-token chunks):
//   * token-serial below 17 tokens (1024 x 12: 1.30 / - / 1.51; 1024 x 16: 1.53-1.78 /
//     3.03 / 1.50-1.55, where boxes of the pool disagree on the order; 1 x 16: 0.026 /
//     0.032 / 0.030);
//   * 64-token chunks for prompts of 512 tokens or more in fewer than 64 (sequence, head)
//     pairs, where the chunk-by-chunk chain is the time and 64-token chunks halve it
//     (1 x 4096: 2.74 / 0.201 / 0.279; 1 x 512: 0.357 / 0.051 / 0.056; 1 x 256: 0.183 /
//     0.043 / 0.038; 2 x 2048, 64 pairs: 1.38 / 0.199 / 0.167);
//   * 32-token chunks otherwise (1024 x 17: 1.63 / 3.06 / 1.53; 1024 x 32: 2.66 / 3.12 /
//     1.72; 32 x 1024: 2.66 / 1.36 / 1.06; 1 x 64: 0.053 / 0.033 / 0.030).
// Returns the tokens per chunk (64 or 32), or 0 for the token-serial form.
inline int prefill_auto_chunk_tokens(int64_t num_tokens, int64_t num_sequences,
                                     int64_t num_v_heads) {
  if (num_sequences <= 0 || num_tokens <= 0) return 0;
  const int64_t mean = num_tokens / num_sequences;
  if (mean < 17) return 0;
  if (num_sequences * num_v_heads < 64 && mean >= 512) return 64;
  return 32;
}

int64_t prefill_chunked_workspace_bytes(int64_t num_tokens, int64_t num_sequences,
                                        int64_t num_v_heads);
// chunk_tokens: 64 or 32
int launch_prefill_chunked(const DecodeParams& p, int num_sequences, int64_t num_tokens,
                           bool dt_bf16, int chunk_tokens, void* workspace, hipStream_t stream);

}  // namespace ld
