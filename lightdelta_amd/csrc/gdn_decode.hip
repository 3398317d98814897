// Fused post-conv Gated DeltaNet decode / MTP-verify step for gfx950 (CDNA4).
//
// Math per (request r, v-head h, token t), following the unfused Torch contract of the
// reference (python/lightdelta/reference/gdn.py:97-120) and the slot semantics of its CUDA
// op (csrc/gdn_decode.cu:147-168, 303-316):
//   q^ = (q * rsqrt(sum q^2 + 1e-6)) * scale          k^ = k * rsqrt(sum k^2 + 1e-6)
//   alpha = exp(-exp(A_log[h]) * softplus(a + dt_bias[h]))      beta = sigmoid(b)
//   S <- alpha * S ;  delta[v] = (v[v] - sum_k S[v,k] k^[k]) * beta ;  S[v,:] += delta[v] k^
//   raw[v] = bf16(sum_k S[v,k] q^[k])
//   out[v] = bf16(raw[v] * rsqrt(mean(raw^2) + eps) * w[v] * silu(gate[v]))
//
// Work decomposition (one workgroup = one (request, v-head) 128x128 fp32 state tile):
//   * 256 threads = 4 wave64s; wave w owns V rows 32w .. 32w+31.
//   * Inside a wave, the 16 lanes of a DPP row span one 512-byte K row: lane kq holds
//     k = 4kq..4kq+3 and 64+4kq..64+4kq+3 (two 16-byte pieces); the 4 DPP rows of the wave
//     take 4 consecutive V rows.  One global_load_dwordx4 therefore reads four half rows,
//     i.e. eight whole 128-byte lines.  A lane keeps 8 V rows x 8 K values = 64 fp32
//     (16 x 128-bit loads) of the tile in VGPRs for the whole step.
//   * All 16 tile loads are issued up front, then the slice is processed in 4 chunks of
//     8 V rows in load order: each chunk waits only for its own 4 loads, runs every token
//     on its rows and stores them, so arithmetic on chunk c overlaps the loads of the later
//     chunks and the stores of the earlier ones.
//   * Row dot products S k^ and S q^ are 8 products per lane plus a 4-step DPP butterfly
//     over the 16-lane row (quad_perm, row_half_mirror, row_mirror); every lane ends with
//     the full sums, so no LDS round trip and no broadcast step is needed.
//   * T <= 4 tokens (MTP verify) reuse the registers: 1 tile read, T tile writes.
#include "gdn_common.h"

namespace ld {
namespace {

constexpr int kConvWidth = 4;
constexpr int kMaxConvLen = 8;
// Tickets of the conv-fused variant, one per (conv slot, k-head); see gdn_decode_kernel.
constexpr int kMaxConvTickets = 1 << 20;
__device__ uint32_t g_conv_ticket[kMaxConvTickets];

// Destination of the state of an MTP token that has no slot to go to (past the request's last
// token, or a padding slot) under non-temporal stores: one tile, written and never read.
__device__ __align__(256) f32x4 g_state_sink[kDim * kDim / 4];

// Sums over the 16 lanes of a DPP row; every lane of the row receives the totals.
__device__ __forceinline__ void row_sum2(float& x, float& y) {
  x += dpp<kDppQuadXor1>(x);
  y += dpp<kDppQuadXor1>(y);
  x += dpp<kDppQuadXor2>(x);
  y += dpp<kDppQuadXor2>(y);
  x += dpp<kDppRowHalfMirror>(x);
  y += dpp<kDppRowHalfMirror>(y);
  x += dpp<kDppRowMirror>(x);
  y += dpp<kDppRowMirror>(y);
}

// Byte offset of a lane's 16-byte piece j of the tile, relative to its first piece: piece j
// is V row 4*(j/2) further down (2 KiB per 4 rows) and, for odd j, 64 floats further along K.
__device__ __forceinline__ constexpr uint32_t tile_piece_bytes(int j) {
  return static_cast<uint32_t>(j >> 1) * 4u * kDim * 4u + static_cast<uint32_t>(j & 1) * 256u;
}

__device__ __forceinline__ float dot8(f32x4 s0, f32x4 s1, f32x4 x0, f32x4 x1) {
  float acc = s0.x * x0.x;
  acc = fmaf(s0.y, x0.y, acc);
  acc = fmaf(s0.z, x0.z, acc);
  acc = fmaf(s0.w, x0.w, acc);
  acc = fmaf(s1.x, x1.x, acc);
  acc = fmaf(s1.y, x1.y, acc);
  acc = fmaf(s1.z, x1.z, acc);
  acc = fmaf(s1.w, x1.w, acc);
  return acc;
}

// Normalised k^ and q^ pieces a lane multiplies with (k = 4kq.. and 64+4kq..).
struct Vectors {
  f32x4 k0, k1, q0, q1;
};

// qk[0] holds q^, qk[1] holds k^, as 32 float4 pieces each.
__device__ __forceinline__ Vectors load_vectors(const f32x4 (&qk)[2][kDim / 4], int kq) {
  Vectors x;
  x.q0 = qk[0][kq];
  x.q1 = qk[0][16 + kq];
  x.k0 = qk[1][kq];
  x.k1 = qk[1][16 + kq];
  return x;
}

// Raw bf16 activations of one token as a lane needs them: four q and four k pieces of 2
// bf16 each (k = 4kq..4kq+3 and 64+4kq..), one v value (column v_col of the row), a and b.
struct TokenIn {
  uint32_t q[4], k[4];
  uint16_t v, a, b;
};

__device__ __forceinline__ TokenIn load_token(const DecodeParams& p, int64_t token, int q_col,
                                              int k_col, int v_col, int head, int kq) {
  const uint16_t* row = p.qkv + token * p.qkv_row;
  TokenIn in;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int off = (e == 0 ? 0 : 64) + kq * 4;
    in.q[2 * e] = row[q_col + off] | (static_cast<uint32_t>(row[q_col + off + 1]) << 16);
    in.q[2 * e + 1] = row[q_col + off + 2] | (static_cast<uint32_t>(row[q_col + off + 3]) << 16);
    in.k[2 * e] = row[k_col + off] | (static_cast<uint32_t>(row[k_col + off + 1]) << 16);
    in.k[2 * e + 1] = row[k_col + off + 2] | (static_cast<uint32_t>(row[k_col + off + 3]) << 16);
  }
  in.v = row[v_col];
  in.a = p.a[token * p.a_row + head];
  in.b = p.b[token * p.b_row + head];
  return in;
}

// The q/k part of a token in the lane layout of load_token, from conv outputs in LDS
// (256 bf16 q/k channels of the k-head, then the v channels).
__device__ __forceinline__ TokenIn conv_token(const uint16_t* conv, int kq) {
  const uint32_t* c32 = reinterpret_cast<const uint32_t*>(conv);
  TokenIn in;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    in.q[2 * e] = c32[e * 32 + 2 * kq];
    in.q[2 * e + 1] = c32[e * 32 + 2 * kq + 1];
    in.k[2 * e] = c32[64 + e * 32 + 2 * kq];
    in.k[2 * e + 1] = c32[64 + e * 32 + 2 * kq + 1];
  }
  return in;
}

// A token's q^ / k^ pieces of this lane (q^ scaled by `scale`), decay and beta.
struct Staged {
  f32x4 q0, q1, k0, k1;
  float decay, beta;
};

// q/k L2 norm over the 16 lanes of the DPP row (each holds 8 of the 128 values), then the
// gates: decay = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b).
__device__ __forceinline__ Staged stage_token(const TokenIn& in, float a_log, float dt_bias,
                                              float scale) {
  float qf[8], kf[8];
  float qq = 0.0f, kk = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qf[2 * e] = bf16_to_f32(static_cast<uint16_t>(in.q[e]));
    qf[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(in.q[e] >> 16));
    kf[2 * e] = bf16_to_f32(static_cast<uint16_t>(in.k[e]));
    kf[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(in.k[e] >> 16));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    qq = fmaf(qf[e], qf[e], qq);
    kk = fmaf(kf[e], kf[e], kk);
  }
  row_sum2(qq, kk);
  const float rq = fast_rsqrt(qq + 1e-6f);
  const float rk = fast_rsqrt(kk + 1e-6f);
  Staged x;
  x.q0 = f32x4{qf[0] * rq, qf[1] * rq, qf[2] * rq, qf[3] * rq} * scale;
  x.q1 = f32x4{qf[4] * rq, qf[5] * rq, qf[6] * rq, qf[7] * rq} * scale;
  x.k0 = f32x4{kf[0] * rk, kf[1] * rk, kf[2] * rk, kf[3] * rk};
  x.k1 = f32x4{kf[4] * rk, kf[5] * rk, kf[6] * rk, kf[7] * rk};
  x.decay = __expf(-__expf(a_log) * softplus(bf16_to_f32(in.a) + dt_bias));
  x.beta = sigmoid(bf16_to_f32(in.b));
  return x;
}

// One token on chunk C of the lane's slice (pieces 4C..4C+3 = V rows row0 and row0 + 4,
// whose v values are v0 and v1):
//   S <- decay*S ; delta = (v - S k^) * beta ; S += delta k^ ; raw = bf16(S q^)
// The updated pieces are stored to `dst_tile` (NULL: padding slot, nothing stored) and the
// two rows' raw outputs go to LDS (one lane per row).
template <int C, bool Stream, bool Store = true, int N = kPieces>
__device__ __forceinline__ void chunk_step(f32x4 (&s)[N], const Vectors& x, float v0,
                                           float v1, float* o, float decay, float beta,
                                           int kq, int row0, char* dst_tile,
                                           uint32_t lane_bytes) {
  constexpr int j0 = 4 * C;
#pragma unroll
  for (int j = j0; j < j0 + 4; ++j) s[j] *= decay;
  float pred0 = dot8(s[j0], s[j0 + 1], x.k0, x.k1);
  float pred1 = dot8(s[j0 + 2], s[j0 + 3], x.k0, x.k1);
  row_sum2(pred0, pred1);
  const float d0 = (v0 - pred0) * beta;
  const float d1 = (v1 - pred1) * beta;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s[j0][e] = fmaf(d0, x.k0[e], s[j0][e]);
    s[j0 + 1][e] = fmaf(d0, x.k1[e], s[j0 + 1][e]);
    s[j0 + 2][e] = fmaf(d1, x.k0[e], s[j0 + 2][e]);
    s[j0 + 3][e] = fmaf(d1, x.k1[e], s[j0 + 3][e]);
  }
  // Stream: unconditional (a token without a destination writes the sink tile), so the
  // compiler's count of memory operations in flight is exact and later chunks wait for
  // their own loads only.  Keep: skipped for a null destination; the branch makes the
  // compiler assume the stores may not have been issued, so chunks 2 and 3 also wait for
  // the earlier chunks' stores -- measured 1.5% faster when the state is served from the
  // Infinity Cache, and 2% slower when it streams from HBM.
  if (Store && (Stream || dst_tile != nullptr)) {
#pragma unroll
    for (int j = j0; j < j0 + 4; ++j) {
      f32x4* dst = reinterpret_cast<f32x4*>(dst_tile + (lane_bytes + tile_piece_bytes(j)));
      if (Stream)
        __builtin_nontemporal_store(s[j], dst);
      else
        *dst = s[j];
    }
  }
  float out0 = dot8(s[j0], s[j0 + 1], x.q0, x.q1);
  float out1 = dot8(s[j0 + 2], s[j0 + 3], x.q0, x.q1);
  row_sum2(out0, out1);
  if (kq == 0) {
    o[row0] = round_bf16(out0);
    o[row0 + 4] = round_bf16(out1);
  }
}

// Uses a wave-uniform value (in SGPRs) at this point of the program, so its computation (a
// kernel-argument or metadata load) cannot be sunk past later branches.  Input-only: the
// value itself, and for pointers their global address space, stay visible to the compiler.
template <typename T>
__device__ __forceinline__ void pin_sgpr(const T& x) {
  asm volatile("" ::"s"(x));
}

// silu(x) rounded to the nearest bf16 (ties to even) as if computed exactly.
//
// Fast path: x * rcp(1 + exp(-x)) in fp32.  Rounding x * log2(e) inside the hardware exp
// costs a relative error of |x| * 2^-24 in exp(-x); exp, the add, rcp and the final multiply
// add at most ~3 * 2^-23 more, so the fp32 result is within |x| + 6 fp32 ulps of the exact
// value.  Its bf16 rounding is therefore the exact value's unless it lies within that
// distance of a bf16 rounding midpoint (low 16 bits near 0x8000); such lanes (window
// 64 + 4|x| ulps) and |x| > 64 recompute x / (1 + exp(-x)) in fp64 and round that to bf16
// without double rounding.  Inlined: a call would make the callee wait for every load in
// flight.
__device__ __forceinline__ uint16_t silu_bf16_exact(float x) {
  const double yd = static_cast<double>(x) / (1.0 + exp(-static_cast<double>(x)));
  const float t = static_cast<float>(yd);
  const uint32_t u = __float_as_uint(t);
  if ((u & 0xffffu) == 0x8000u && static_cast<double>(t) != yd)  // fp32 rounding hit a tie
    return static_cast<uint16_t>((u >> 16) + (fabs(yd) > fabs(static_cast<double>(t)) ? 1u : 0u));
  return f32_to_bf16(t);
}

__device__ __forceinline__ uint16_t silu_bf16(float x) {
  const float y = silu(x);
  const float ax = fabsf(x);
  const int low = static_cast<int>(__float_as_uint(y) & 0xffffu) - 0x8000;
  if (!(ax <= 64.0f) || static_cast<float>(abs(low)) <= 64.0f + 4.0f * ax)
    return silu_bf16_exact(x);
  return f32_to_bf16(y);
}

// One decode-token output of the causal depthwise conv (width 4) plus SiLU, rounded to bf16:
//   bf16(silu(bias + sum_j w[j] * [state[len-3], state[len-2], state[len-1], x][j]))
// with the fp32 accumulation running from the oldest tap to the newest (one rounding per
// fused multiply-add) and the SiLU correctly rounded to bf16.
// bf16(silu(bias + w0*t0 + w1*t1 + w2*t2 + w3*t3)): one causal conv output from its four
// taps, oldest first, with the fp32 accumulation running from the oldest tap to the newest
// (one rounding per fused multiply-add) and the SiLU correctly rounded to bf16.
__device__ __forceinline__ uint16_t conv_dot(uint16_t t0, uint16_t t1, uint16_t t2, uint16_t t3,
                                             const uint32_t (&w)[2], uint16_t bias, bool has_bias) {
  float acc = has_bias ? bf16_to_f32(bias) : 0.0f;
  acc = fmaf(bf16_to_f32(static_cast<uint16_t>(w[0])), bf16_to_f32(t0), acc);
  acc = fmaf(bf16_to_f32(static_cast<uint16_t>(w[0] >> 16)), bf16_to_f32(t1), acc);
  acc = fmaf(bf16_to_f32(static_cast<uint16_t>(w[1])), bf16_to_f32(t2), acc);
  acc = fmaf(bf16_to_f32(static_cast<uint16_t>(w[1] >> 16)), bf16_to_f32(t3), acc);
  return silu_bf16(acc);
}

// Up to 8 bf16 values of one conv channel packed in two 64-bit registers.  Element i is
// selected with a shift, for a runtime i too: a select chain over an array lets the compiler
// turn it into a dynamically indexed array, which it then places in scratch or LDS memory.
struct Packed8 {
  uint64_t lo = 0, hi = 0;
  __device__ __forceinline__ void set(int i, uint32_t v) {  // v < 2^16, i compile-time
    if (i < 4)
      lo |= static_cast<uint64_t>(v) << (16 * i);
    else
      hi |= static_cast<uint64_t>(v) << (16 * (i - 4));
  }
  __device__ __forceinline__ uint16_t get(int i) const {  // 0 <= i < 8
    return static_cast<uint16_t>((i < 4 ? lo : hi) >> (16 * (i & 3)));
  }
};

// One decode-token output of the causal depthwise conv (width 4) plus SiLU, rounded to bf16,
// with the history in the first 3 state columns (vLLM's causal_conv1d_update without
// speculative tokens reads columns 0..2 whatever the state's length):
//   bf16(silu(bias + sum_j w[j] * [state[0], state[1], state[2], x][j]))
__device__ __forceinline__ uint16_t conv_output(uint16_t x, const uint16_t (&state)[4],
                                                const uint32_t (&w)[2], uint16_t bias,
                                                bool has_bias) {
  return conv_dot(state[0], state[1], state[2], x, w, bias, has_bias);
}

// The conv of one channel over the Width tokens of a speculative-decoding step (vLLM's
// causal_conv1d_update with num_accepted_tokens): the history is the 3 state columns from
// `offset` (= accepted - 1), token t's window is the 4 inputs of history ++ x ending at x_t,
// and the new state is state[offset + 1 .. offset + len - n] followed by x_0 .. x_{n-1}
// (n = the request's tokens, len = the state's columns).  Outputs go to out[t * 3 * kDim],
// t < Width (tokens past n use copies of the last input and are discarded by the caller);
// new_state[k] holds column min(k, len - 1).  Reads nothing out of bounds: every column is
// clamped to len - 1 and every token to n - 1 when loaded.
template <int Width, int Cols>
__device__ __forceinline__ void conv_channel_tokens(const DecodeParams& p, int64_t bos, int n,
                                                    int offset, int64_t state_at, int channel,
                                                    bool has_bias, uint16_t* out,
                                                    uint16_t (&new_state)[Cols]) {
  static_assert(Cols <= 8 && Width <= 4, "packed conv registers hold 8 columns, 4 tokens");
  Packed8 st, x;
#pragma unroll
  for (int j = 0; j < Cols; ++j)
    st.set(j, p.conv_state[state_at + min(j, p.conv_len - 1) * p.conv_len_stride]);
#pragma unroll
  for (int t = 0; t < Width; ++t) x.set(t, p.conv_x[(bos + min(t, n - 1)) * p.conv_x_row + channel]);
  const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(p.conv_weight + channel * kConvWidth);
  const uint32_t w[2] = {wsrc[0], wsrc[1]};
  const uint16_t bias = (p.conv_bias != nullptr ? p.conv_bias : p.conv_weight)[channel];
  uint16_t seq[3 + Width];
#pragma unroll
  for (int m = 0; m < 3; ++m) seq[m] = st.get(offset + m);
#pragma unroll
  for (int t = 0; t < Width; ++t) seq[3 + t] = x.get(t);
#pragma unroll
  for (int t = 0; t < Width; ++t)
    out[t * 3 * kDim] = conv_dot(seq[t], seq[t + 1], seq[t + 2], seq[t + 3], w, bias, has_bias);
  const int kept = p.conv_len - n;  // state columns that survive (<= 0: none)
#pragma unroll
  for (int k = 0; k < Cols; ++k) {
    const int col = min(k, p.conv_len - 1);
    new_state[k] = col < kept ? st.get(offset + 1 + col) : x.get(col - kept);
  }
}

// Waits for this wave's LDS traffic, then joins the workgroup barrier.  Global loads that
// are still in flight stay in flight (a __syncthreads() fence would drain them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Four waves per SIMD (<= 128 VGPRs) keep four workgroups, i.e. four tiles, resident per CU.
// DtBf16 / WBf16: dt_bias / norm_weight stored as bf16 (else fp32).  Stream: non-temporal
// state loads and stores (for working sets larger than the caches).  Width: the indices
// width W (tokens per request at most); fixing it at compile time unrolls every token loop
// into straight-line code, which keeps the tile's per-piece load waits exact.
//
// Conv: the causal depthwise conv1d (width 4, SiLU) runs first on the pre-conv activations.
// Each workgroup convolves the 256 q/k channels of its k-head and the 128 v channels of its
// head from the conv state of the request's slot, rounds the outputs to bf16 (the dtype an
// unfused conv writes) and feeds them to the GDN step; one token (W = 1) while the tile
// streams in, several (speculative verify, W > 1) before the tile loads.  Its own v
// channels' conv state is updated in place.  The q/k channels are shared by the
// HV/H workgroups of a k-head group, so their shifted state is written only after all of
// them have read it: every workgroup counts itself in (relaxed atomic add on
// g_conv_ticket[slot*H + kh], returning the previous count) after its reads; the one that
// receives HV/H - 1 counted in last, writes the shifted state at its end and resets the
// count to 0.  Nothing waits on another workgroup, and every launch leaves the counts at
// zero.  ConvCols: conv-state columns held per channel (4 for states of 3..4 columns, 8 for
// up to 8; 0 = no conv).
template <bool DtBf16, bool WBf16, bool Stream, int Width, int ConvCols>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void gdn_decode_kernel(const DecodeParams args) {
  constexpr bool Conv = ConvCols > 0;
  constexpr int kCols = Conv ? ConvCols : 1;
  // Cache hints of the state traffic.  One token: the policy's (plain loads and stores keep
  // a layer's state in the Infinity Cache between steps; non-temporal ones stream it).
  // Several tokens (verify): the writes are 4 times the reads, and plain loads with
  // non-temporal stores measured fastest under either policy (B=64, T=4: 103 us against
  // 134-139 us with both hints alike), the stores being unconditional (sink tile) so that
  // load waits stay exact.
  constexpr bool kLoadNT = Stream && Width == 1;
  constexpr bool kStoreNT = Stream || Width > 1;
  // The conv runs before the tile loads for several tokens or more than 4 state columns;
  // one token with 3..4 columns keeps it in registers while the tile streams in.
  constexpr bool kConvFirst = Conv && (Width > 1 || kCols > 4);
  constexpr bool kConvLate = Conv && !kConvFirst;
  static_assert(!kConvLate || kCols == 4, "the in-flight conv holds 4 state columns");
  // Every kernel argument, then all request metadata, is loaded before the first branch:
  // two dependent scalar round trips (kernel-argument segment; cu/accepted/indices) instead
  // of the compiler's default of sinking each load to its first use behind the early exits.
  // The pins come after the metadata loads: a pin is opaque to the compiler, and scalar
  // (s_load) metadata loads must not follow anything that might have written memory.
  const DecodeParams& p = args;
  const int tile = blockIdx.x;
  const int request = tile / p.num_v_heads;
  const int head = tile - request * p.num_v_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Request metadata in one round trip: token range, accepted count and the (at most 4)
  // slots of the request, read before any state store.
  const int32_t* req_slots = p.indices + static_cast<int64_t>(request) * Width;
  const int bos = p.cu[request];
  const int eos = p.cu[request + 1];
  const int accepted = p.accepted[request];
  int slot[Width];
#pragma unroll
  for (int t = 0; t < Width; ++t) slot[t] = req_slots[t];
#pragma unroll
  for (int t = 0; t < Width; ++t) pin_sgpr(slot[t]);
  pin_sgpr(bos);
  pin_sgpr(eos);
  pin_sgpr(accepted);
  pin_sgpr(p.qkv);
  pin_sgpr(p.qkv_row);
  pin_sgpr(p.a);
  pin_sgpr(p.a_row);
  pin_sgpr(p.b);
  pin_sgpr(p.b_row);
  pin_sgpr(p.a_log);
  pin_sgpr(p.dt_bias);
  pin_sgpr(p.state);
  pin_sgpr(p.state_slot);
  pin_sgpr(p.gate);
  pin_sgpr(p.gate_row);
  pin_sgpr(p.norm_weight);
  pin_sgpr(p.out);
  pin_sgpr(p.num_k_heads);
  pin_sgpr(p.group);
  pin_sgpr(p.scale);
  pin_sgpr(p.eps);
  const int num_tokens = eos - bos;
  if (num_tokens <= 0) return;
  int source = 0;
#pragma unroll
  for (int t = 0; t < Width; ++t)
    if (accepted == t + 1) source = slot[t];
  // Conv variant: the conv state lives in slot indices[r, 0]; the history of token 0 is its
  // 3 columns from accepted - 1, and the columns kept for the next step must lie in the
  // state too (true whenever the state has 3 + W - 1 columns and accepted <= tokens).
  const int conv_offset = accepted - 1;
  const bool conv_ok = !Conv || (slot[0] > 0 && conv_offset + kConvWidth - 2 <= p.conv_len - 1 &&
                                 (p.conv_len <= num_tokens || conv_offset <= num_tokens - 1));
  if (source <= 0 || num_tokens > Width || !conv_ok) {
    // Invalid request: zero outputs, state untouched.
    for (int i = tid; i < num_tokens * kDim; i += kThreads) {
      const int64_t token = bos + (i >> 7);
      p.out[(token * p.num_v_heads + head) * kDim + (i & (kDim - 1))] = 0;
    }
    return;
  }

  // Token 0 is staged by every wave for itself (wave-private LDS, no barrier before the
  // recurrence): q^ and k^ (128 each), v of the wave's 32 rows, decay and beta.  MTP tokens
  // t >= 1 are staged once, by wave t, in the shared area (one barrier, after chunk 0's
  // token 0).  s_o collects the raw outputs of all rows for the epilogue.
  __shared__ f32x4 s_qk0[kWaves][2][kDim / 4];
  __shared__ float s_v0[kWaves][kRowsPerWave];
  __shared__ float s_db0[kWaves][2];
  __shared__ f32x4 s_qkt[Width][2][kDim / 4];
  __shared__ float s_vt[Width][kDim];
  __shared__ float s_dbt[Width][2];
  __shared__ float s_o[Width][kDim];
  // Conv variant: bf16 conv outputs of the 256 q/k channels and 128 v channels per token,
  // and the shifted q/k conv state kept for the end-of-kernel write.
  __shared__ uint16_t s_conv[Conv ? Width : 1][Conv ? 3 * kDim : 2];
  __shared__ uint16_t s_conv_new[Conv ? 2 * kDim : 1][kCols];
  __shared__ uint32_t s_arrived;

  const int key_head = head / p.group;
  const int kq = lane & 15;
  const int rsub = lane >> 4;
  const int row_base = wave * kRowsPerWave + rsub;  // V row of the lane's piece 0
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;

  // ---- small activation loads go out before the tile, so they return first: token 0 in
  // the lane layout of the tile (q, k at 4kq.. and 64+4kq..; v of the wave's 32 rows), the
  // MTP token `wave` for the shared staging, and the epilogue inputs of token `wave` ----
  TokenIn in0;
  // Conv variant: this thread convolves q/k channel `conv_qk` and (tid < 128) v channel
  // `conv_v`; it loads their input, conv-state columns (clamped to the last column past
  // conv_len, so every load is in bounds), weights and bias.
  const int conv_qk = tid < kDim ? q_col + tid : k_col + (tid - kDim);
  const int conv_v = v_col + (tid & (kDim - 1));
  const int64_t conv_slot_at = static_cast<int64_t>(slot[0]) * p.conv_slot;
  int64_t cs_qk_at = conv_slot_at + conv_qk * p.conv_dim_stride;
  int64_t cs_v_at = conv_slot_at + conv_v * p.conv_dim_stride;
  uint16_t cx_qk = 0, cx_v = 0, cb_qk = 0, cb_v = 0;
  uint16_t cs_qk_raw[kConvLate ? 4 : 1], cs_v_raw[kConvLate ? 4 : 1];
  uint32_t cw_qk[2], cw_v[2];
  uint32_t arrived = 0;  // ticket count before this workgroup's increment (thread 0)
  if constexpr (kConvFirst) {
    // Several tokens (speculative verify), or a long conv state: the conv runs to
    // completion before the tile loads, so its inputs do not compete with the tile for
    // registers.  The v channels are
    // this workgroup's alone and are shifted in place (threads 128..255 repeat the stores
    // of 0..127 with identical bytes); the q/k channels are kept for the end-of-kernel write.
    uint16_t qk_new[kCols], v_new[kCols];
    const bool has_bias = p.conv_bias != nullptr;
    conv_channel_tokens<Width, kCols>(p, bos, num_tokens, conv_offset, cs_qk_at, conv_qk, has_bias,
                                      &s_conv[0][tid], qk_new);
    conv_channel_tokens<Width, kCols>(p, bos, num_tokens, conv_offset, cs_v_at, conv_v, has_bias,
                                      &s_conv[0][2 * kDim + (tid & (kDim - 1))], v_new);
#pragma unroll
    for (int k = 0; k < kCols; ++k) s_conv_new[tid][k] = qk_new[k];
    // Every wave has consumed its conv-state reads once past the barrier, so the v channels
    // (read by two threads each) can be overwritten.
    lds_barrier();
#pragma unroll
    for (int k = 0; k < kCols; ++k)
      p.conv_state[cs_v_at + min(k, p.conv_len - 1) * p.conv_len_stride] = v_new[k];
    if (p.group > 1 && tid == 0)
      arrived = __hip_atomic_fetch_add(
          &g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head], 1u,
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    in0.a = p.a[static_cast<int64_t>(bos) * p.a_row + head];
    in0.b = p.b[static_cast<int64_t>(bos) * p.b_row + head];
  } else if constexpr (kConvLate) {
    const uint16_t* xrow = p.conv_x + static_cast<int64_t>(bos) * p.conv_x_row;
    cx_qk = xrow[conv_qk];
    cx_v = xrow[conv_v];
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      const int64_t col = min(j, p.conv_len - 1) * p.conv_len_stride;
      cs_qk_raw[j] = p.conv_state[cs_qk_at + col];
      cs_v_raw[j] = p.conv_state[cs_v_at + col];
    }
    const uint32_t* wq = reinterpret_cast<const uint32_t*>(p.conv_weight + conv_qk * kConvWidth);
    const uint32_t* wv = reinterpret_cast<const uint32_t*>(p.conv_weight + conv_v * kConvWidth);
    cw_qk[0] = wq[0];
    cw_qk[1] = wq[1];
    cw_v[0] = wv[0];
    cw_v[1] = wv[1];
    // Without a bias the weight array stands in as an always-valid source: the loads stay
    // unconditional (a load under a branch makes the compiler drain every earlier load at
    // the branch's end) and conv_output ignores the value.
    const uint16_t* bias_src = p.conv_bias != nullptr ? p.conv_bias : p.conv_weight;
    cb_qk = bias_src[conv_qk];
    cb_v = bias_src[conv_v];
    in0.a = p.a[static_cast<int64_t>(bos) * p.a_row + head];
    in0.b = p.b[static_cast<int64_t>(bos) * p.b_row + head];
  } else {
    in0 = load_token(p, bos, q_col, k_col, v_col + wave * kRowsPerWave + (lane & 31), head, kq);
  }
  // Every MTP token slot t < W is staged and stepped, past the request's last token too
  // (with a copy of that token), so the token loops have no branches; such tokens' states
  // go to the sink tile (non-temporal stores) or are not stored, and their outputs are not
  // written.
  const bool stages_mtp = Width > 1 && wave >= 1 && wave < Width;
  const int64_t token_w = bos + min(wave, num_tokens - 1);
  TokenIn inw;
  uint16_t vw_hi = 0;
  if constexpr (Conv && Width > 1) {  // post-conv token from LDS (ready: barrier above)
    const uint16_t* conv_w = s_conv[min(wave, num_tokens - 1)];
    inw = conv_token(conv_w, kq);
    inw.v = conv_w[2 * kDim + 2 * lane];
    vw_hi = conv_w[2 * kDim + 2 * lane + 1];
    inw.a = p.a[token_w * p.a_row + head];
    inw.b = p.b[token_w * p.b_row + head];
  } else if (Width > 1) {
    inw = load_token(p, token_w, q_col, k_col, v_col + 2 * lane, head, kq);
    vw_hi = p.qkv[token_w * p.qkv_row + v_col + 2 * lane + 1];
  }
  uint16_t gh[2];
  float w[2];
  {
    const uint16_t* grow = p.gate + token_w * p.gate_row + head * kDim;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      gh[e] = grow[2 * lane + e];
      w[e] = load_param(p.norm_weight, 2 * lane + e, WBf16);
    }
  }
  const float dt_bias = load_param(p.dt_bias, head, DtBf16);
  const float a_log = p.a_log[head];
  __builtin_amdgcn_sched_barrier(0);

  // ---- the whole 64 KiB source tile: 16 x 128-bit loads per lane (uniform base address,
  // 32-bit per-lane byte offsets), issued in chunk order ----
  const int64_t head_offset = static_cast<int64_t>(head) * kDim * kDim;
  const uint32_t lane_bytes = static_cast<uint32_t>(row_base * kDim + kq * 4) * 4u;
  const char* src_tile = reinterpret_cast<const char*>(
      p.state + static_cast<int64_t>(source) * p.state_slot + head_offset);
  f32x4 s[kPieces];
#pragma unroll
  for (int j = 0; j < kPieces; ++j) {
    const f32x4* src =
        reinterpret_cast<const f32x4*>(src_tile + (lane_bytes + tile_piece_bytes(j)));
    s[j] = kLoadNT ? __builtin_nontemporal_load(src) : *src;
    __builtin_amdgcn_sched_barrier(0);  // keep program order: chunk c's loads issue first
  }

  // ---- staging, while the tile streams in ----
  if constexpr (kConvLate) {
    const int len = p.conv_len;
    const bool has_bias = p.conv_bias != nullptr;
    s_conv[0][tid] = conv_output(cx_qk, cs_qk_raw, cw_qk, cb_qk, has_bias);
    if (tid < kDim) s_conv[0][2 * kDim + tid] = conv_output(cx_v, cs_v_raw, cw_v, cb_v, has_bias);
    // Shifted state: columns 1..len-1, then the new input.  The q/k channels are kept for
    // the end-of-kernel write.
    uint16_t v_new[kCols];
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      s_conv_new[tid][j] = j + 1 < len ? cs_qk_raw[j + 1 < kCols ? j + 1 : j] : cx_qk;
      v_new[j] = j + 1 < len ? cs_v_raw[j + 1 < kCols ? j + 1 : j] : cx_v;
    }
    // Conv outputs visible to every wave; every conv-state read of this workgroup consumed.
    lds_barrier();
    // The v channels (this workgroup's alone) are shifted in place; threads 128..255 repeat
    // the stores of threads 0..127 with identical bytes (both read the channel before the
    // barrier), and columns past len-1 repeat column len-1, so the stores need no branch (a
    // store under a branch makes later load waits conservative).
#pragma unroll
    for (int j = 0; j < kCols; ++j)
      p.conv_state[cs_v_at + min(j, len - 1) * p.conv_len_stride] = v_new[j];
    // Relaxed: every conv-state value this workgroup read has already been consumed (the
    // barrier above follows the conv arithmetic), so the increment cannot overtake a read.
    // The returned count is first used at the kernel's end, by which time it has long
    // arrived: no wait on the tile stream here, and no extra round trip there.
    if (p.group > 1 && tid == 0)
      arrived = __hip_atomic_fetch_add(
          &g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head], 1u,
          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (Conv) {  // token 0 after the conv, from LDS
    const TokenIn c = conv_token(s_conv[0], kq);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      in0.q[e] = c.q[e];
      in0.k[e] = c.k[e];
    }
    in0.v = s_conv[0][2 * kDim + wave * kRowsPerWave + (lane & 31)];
  }
  {
    const Staged x = stage_token(in0, a_log, dt_bias, p.scale);
    if (rsub == 0) {
      s_qk0[wave][0][kq] = x.q0;
      s_qk0[wave][0][16 + kq] = x.q1;
      s_qk0[wave][1][kq] = x.k0;
      s_qk0[wave][1][16 + kq] = x.k1;
    }
    if (lane < kRowsPerWave) s_v0[wave][lane] = bf16_to_f32(in0.v);
    if (lane == 0) {
      s_db0[wave][0] = x.decay;
      s_db0[wave][1] = x.beta;
    }
  }
  if (stages_mtp) {
    const Staged x = stage_token(inw, a_log, dt_bias, p.scale);
    if (rsub == 0) {
      s_qkt[wave][0][kq] = x.q0;
      s_qkt[wave][0][16 + kq] = x.q1;
      s_qkt[wave][1][kq] = x.k0;
      s_qkt[wave][1][16 + kq] = x.k1;
    }
    s_vt[wave][2 * lane] = bf16_to_f32(inw.v);
    s_vt[wave][2 * lane + 1] = bf16_to_f32(vw_hi);
    if (lane == 0) {
      s_dbt[wave][0] = x.decay;
      s_dbt[wave][1] = x.beta;
    }
  }

  // The token-0 staging above is read back by other lanes of the same wave.  A wave executes
  // its LDS instructions in program order, so only the compiler must not move the reads
  // above the writes.
  asm volatile("" ::: "memory");

  // ---- recurrence, chunk by chunk in load order (each chunk's first use of a piece waits
  // for that piece alone: s_waitcnt vmcnt(N)); every token of a chunk before the next ----
  char* const state_bytes = reinterpret_cast<char*>(p.state + head_offset);
  const int64_t slot_bytes = p.state_slot * 4;
  char* dst[Width];
#pragma unroll
  for (int t = 0; t < Width; ++t)
    dst[t] = (t < num_tokens && slot[t] > 0) ? state_bytes + slot[t] * slot_bytes
             : kStoreNT                       ? reinterpret_cast<char*>(g_state_sink)
                                              : nullptr;

#define LD_CHUNK(C)                                                                         \
  {                                                                                         \
    const int r = row_base + 8 * (C);                                                       \
    chunk_step<C, kStoreNT>(s, load_vectors(s_qk0[wave], kq), s_v0[wave][8 * (C) + rsub],     \
                          s_v0[wave][8 * (C) + 4 + rsub], s_o[0], s_db0[wave][0],           \
                          s_db0[wave][1], kq, r, dst[0], lane_bytes);                       \
    if ((C) == 0 && Width > 1) lds_barrier();                                               \
    _Pragma("unroll") for (int t = 1; t < Width; ++t) {                                     \
      chunk_step<C, kStoreNT>(s, load_vectors(s_qkt[t], kq), s_vt[t][r], s_vt[t][r + 4],      \
                            s_o[t], s_dbt[t][0], s_dbt[t][1], kq, r, dst[t], lane_bytes);   \
    }                                                                                       \
  }
  LD_CHUNK(0)
  LD_CHUNK(1)
  LD_CHUNK(2)
  LD_CHUNK(3)
#undef LD_CHUNK
  if constexpr (Conv) {
    if (tid == 0) s_arrived = arrived;
  }
  lds_barrier();

  // ---- gated RMSNorm epilogue for token `wave` ----
  if (wave < num_tokens) {
    const int64_t token = bos + wave;
    float raw[2];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      raw[e] = s_o[wave][2 * lane + e];
      ss = fmaf(raw[e], raw[e], ss);
    }
    ss = wave_sum(ss);
    const float rstd = fast_rsqrt(ss / static_cast<float>(kDim) + p.eps);
    uint16_t* orow = p.out + (token * p.num_v_heads + head) * kDim;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = 2 * lane + e;
      const float gate = bf16_to_f32(gh[e]);
      orow[v] = f32_to_bf16(((raw[e] * rstd) * w[e]) * silu(gate));
    }
  }

  // ---- conv variant: the only workgroup of its k-head (HV == H), or the one that counted
  // in last (all HV/H of the k-head group had read the q/k conv state before it), writes the
  // shifted q/k conv state and returns the count to zero for the next launch ----
  if constexpr (Conv) {
    if (p.group == 1 || s_arrived == static_cast<uint32_t>(p.group - 1)) {
      const int64_t slot_at = static_cast<int64_t>(slot[0]) * p.conv_slot;
      for (int c = tid; c < 2 * kDim; c += kThreads) {
        const int ch = c < kDim ? q_col + c : k_col + (c - kDim);
        const int64_t at = slot_at + ch * p.conv_dim_stride;
        for (int j = 0; j < p.conv_len; ++j) p.conv_state[at + j * p.conv_len_stride] = s_conv_new[c][j];
      }
      if (p.group > 1 && tid == 0)
        __hip_atomic_store(&g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head],
                           0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}


// Prefill: the sequence's tokens run in order with a block of state rows in registers for
// the whole prompt (read once, from the slot or as zeros; written once, to the slot).  The
// per-token arithmetic is the decode kernel's (stage_token, chunk_step), so a prefill of n
// tokens gives bit for bit the states and outputs of n single-token decode steps.  Rows of
// the state evolve independently (row v needs only v[v], k, q and the gates), so a head's
// 128 rows may be split over 4 / Chunks workgroups of 4 waves, each wave holding 8 * Chunks
// rows: fewer rows per wave shorten the per-token chain and spread a few long prompts over
// more of the GPU, at the price of staging q and k in every workgroup.
//   Chunks == 4 (one workgroup per head): the raw outputs of a group of 4 tokens collect in
//   LDS (double-buffered); after one barrier per group, wave w runs the gated-RMSNorm
//   epilogue of the group's token w.
//   Chunks < 4: every wave writes its rows' raw outputs (rounded to bf16, the reference's
//   rounding point before the norm) to `out`; prefill_norm_kernel applies the gated RMSNorm
//   in place afterwards, with the epilogue's arithmetic.
// The next token's inputs are prefetched.  Three to four waves per SIMD: the token loop
// keeps them in flight on top of the tile, which does not fit 128 VGPRs without spills.
constexpr int kPrefillGroup = 4;

template <bool DtBf16, bool WBf16, int Chunks>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 4)))
void gdn_prefill_kernel(const DecodeParams args) {
  static_assert(Chunks == 1 || Chunks == 2 || Chunks == 4, "8, 16 or 32 rows per wave");
  constexpr int kBlocks = 4 / Chunks;         // workgroups per (sequence, head)
  constexpr int kWaveRows = 8 * Chunks;       // state rows per wave
  constexpr int kTilePieces = 4 * Chunks;     // 16-byte pieces per lane
  const DecodeParams& p = args;
  const int tile = blockIdx.x;
  const int sequence = tile / (p.num_v_heads * kBlocks);
  const int rest = tile - sequence * p.num_v_heads * kBlocks;
  const int head = rest / kBlocks;
  const int block = rest - head * kBlocks;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int bos = p.cu[sequence];
  const int eos = p.cu[sequence + 1];
  const int slot = p.indices[sequence];
  const bool from_slot = slot > 0 && p.has_initial[sequence] != 0;

  const int key_head = head / p.group;
  const int kq = lane & 15;
  const int rsub = lane >> 4;
  const int wave_row0 = block * kWaves * kWaveRows + wave * kWaveRows;  // first row of the wave
  const int row_base = wave_row0 + rsub;
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;
  const int v_lane = v_col + wave_row0 + (lane & (kWaveRows - 1));

  __shared__ float s_v[kWaves][kWaveRows];
  __shared__ float s_o[Chunks == 4 ? 2 : 1][Chunks == 4 ? kPrefillGroup : kWaves]
                      [Chunks == 4 ? kDim : kWaveRows];

  const float dt_bias = load_param(p.dt_bias, head, DtBf16);
  const float a_log = p.a_log[head];
  float w[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) w[e] = Chunks == 4 ? load_param(p.norm_weight, 2 * lane + e, WBf16) : 0.0f;

  const int64_t head_offset = static_cast<int64_t>(head) * kDim * kDim;
  const uint32_t lane_bytes = static_cast<uint32_t>(row_base * kDim + kq * 4) * 4u;
  f32x4 s[kTilePieces];
  if (from_slot) {
    const char* src_tile = reinterpret_cast<const char*>(
        p.state + static_cast<int64_t>(slot) * p.state_slot + head_offset);
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j)
      s[j] = *reinterpret_cast<const f32x4*>(src_tile + (lane_bytes + tile_piece_bytes(j)));
  } else {
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j) s[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  TokenIn next;  // inputs of the next token
  if (bos < eos) next = load_token(p, bos, q_col, k_col, v_lane, head, kq);
  int buf = 0;
  for (int g0 = bos; g0 < eos; g0 += kPrefillGroup, buf ^= 1) {
    // gate of the token whose epilogue this wave runs after the group (one workgroup per head)
    uint16_t gh[2] = {0, 0};
    if constexpr (Chunks == 4) {
      const int64_t etoken = min(g0 + wave, eos - 1);
#pragma unroll
      for (int e = 0; e < 2; ++e) gh[e] = p.gate[etoken * p.gate_row + head * kDim + 2 * lane + e];
    }
    for (int i = 0; i < kPrefillGroup && g0 + i < eos; ++i) {
      const int t = g0 + i;
      const TokenIn in = next;
      if (t + 1 < eos) next = load_token(p, t + 1, q_col, k_col, v_lane, head, kq);
      const Staged x = stage_token(in, a_log, dt_bias, p.scale);
      if (lane < kWaveRows) s_v[wave][lane] = bf16_to_f32(in.v);
      // s_v (and s_o below) are read back by other lanes of this wave: a wave's LDS
      // operations run in program order, so only the compiler must not reorder them.
      asm volatile("" ::: "memory");
      Vectors vec;
      vec.q0 = x.q0;
      vec.q1 = x.q1;
      vec.k0 = x.k0;
      vec.k1 = x.k1;
      // output rows: absolute in the per-group buffer, wave-relative in the per-wave one
      float* o = Chunks == 4 ? s_o[buf][i] : s_o[0][wave];
      const int orow = Chunks == 4 ? row_base : rsub;
#define LD_PREFILL_CHUNK(C)                                                                    \
  if constexpr ((C) < Chunks)                                                                  \
    chunk_step<C, false, false, kTilePieces>(s, vec, s_v[wave][8 * (C) + rsub],                \
                                             s_v[wave][8 * (C) + 4 + rsub], o, x.decay,        \
                                             x.beta, kq, orow + 8 * (C), nullptr, lane_bytes);
      LD_PREFILL_CHUNK(0)
      LD_PREFILL_CHUNK(1)
      LD_PREFILL_CHUNK(2)
      LD_PREFILL_CHUNK(3)
#undef LD_PREFILL_CHUNK
      asm volatile("" ::: "memory");
      if constexpr (Chunks < 4) {  // raw outputs of the wave's rows (bf16-exact values)
        if (lane < kWaveRows)
          p.out[(static_cast<int64_t>(t) * p.num_v_heads + head) * kDim + wave_row0 + lane] =
              f32_to_bf16(s_o[0][wave][lane]);
      }
    }
    if constexpr (Chunks == 4) {
      lds_barrier();  // the group's raw outputs are complete
      if (g0 + wave < eos) {  // gated RMSNorm epilogue of the group's token `wave`
        float raw[2];
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          raw[e] = s_o[buf][wave][2 * lane + e];
          ss = fmaf(raw[e], raw[e], ss);
        }
        ss = wave_sum(ss);
        const float rstd = fast_rsqrt(ss / static_cast<float>(kDim) + p.eps);
        uint16_t* orow_ptr = p.out + (static_cast<int64_t>(g0 + wave) * p.num_v_heads + head) * kDim;
#pragma unroll
        for (int e = 0; e < 2; ++e)
          orow_ptr[2 * lane + e] =
              f32_to_bf16(((raw[e] * rstd) * w[e]) * silu(bf16_to_f32(gh[e])));
      }
    }
  }

  if (slot > 0) {  // the state after the last token (the initial one for an empty sequence)
    char* dst_tile = reinterpret_cast<char*>(p.state + static_cast<int64_t>(slot) * p.state_slot +
                                             head_offset);
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j)
      *reinterpret_cast<f32x4*>(dst_tile + (lane_bytes + tile_piece_bytes(j))) = s[j];
  }
}

// Prefill with a head's rows split over 4 / Chunks workgroups (Chunks = 1 or 2): for a few
// prompts, where one workgroup per (sequence, head) leaves most of the GPU idle and every
// token's latency chain is exposed.  Same arithmetic as gdn_prefill_kernel; the loop is
// arranged for latency: token inputs are prefetched kDepth tokens ahead, token t + 1 is
// staged (norms, gates) while token t's rows update, and every lane loads the v values of
// its own rows directly.  Raw outputs go to `out` for prefill_norm_kernel.
template <bool DtBf16, bool WBf16, int Chunks>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 4)))
void gdn_prefill_rows_kernel(const DecodeParams args) {
  static_assert(Chunks == 1 || Chunks == 2, "8 or 16 rows per wave");
  constexpr int kBlocks = 4 / Chunks;
  constexpr int kWaveRows = 8 * Chunks;
  constexpr int kTilePieces = 4 * Chunks;
  constexpr int kDepth = 3;  // tokens in flight ahead of the one being stepped
  const DecodeParams& p = args;
  const int tile = blockIdx.x;
  const int sequence = tile / (p.num_v_heads * kBlocks);
  const int rest = tile - sequence * p.num_v_heads * kBlocks;
  const int head = rest / kBlocks;
  const int block = rest - head * kBlocks;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int bos = p.cu[sequence];
  const int eos = p.cu[sequence + 1];
  const int slot = p.indices[sequence];
  const bool from_slot = slot > 0 && p.has_initial[sequence] != 0;

  const int key_head = head / p.group;
  const int kq = lane & 15;
  const int rsub = lane >> 4;
  const int wave_row0 = block * kWaves * kWaveRows + wave * kWaveRows;
  const int row_base = wave_row0 + rsub;
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;

  __shared__ float s_o[kWaves][kWaveRows];

  const float dt_bias = load_param(p.dt_bias, head, DtBf16);
  const float a_log = p.a_log[head];
  const int64_t head_offset = static_cast<int64_t>(head) * kDim * kDim;
  const uint32_t lane_bytes = static_cast<uint32_t>(row_base * kDim + kq * 4) * 4u;
  f32x4 s[kTilePieces];
  if (from_slot) {
    const char* src_tile = reinterpret_cast<const char*>(
        p.state + static_cast<int64_t>(slot) * p.state_slot + head_offset);
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j)
      s[j] = *reinterpret_cast<const f32x4*>(src_tile + (lane_bytes + tile_piece_bytes(j)));
  } else {
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j) s[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // A token's inputs: q/k/a/b as load_token lays them out, and v of the lane's 2 * Chunks rows
  // (rows row_base + 4 i, i < 2 * Chunks).  Tokens past the sequence's end load its last one.
  struct Pending {
    TokenIn in;
    uint16_t v[2 * Chunks];
  };
  auto fetch = [&](int t) {
    Pending f;
    const int64_t token = min(t, eos - 1);
    f.in = load_token(p, token, q_col, k_col, v_col + row_base, head, kq);
    const uint16_t* vrow = p.qkv + token * p.qkv_row + v_col + row_base;
#pragma unroll
    for (int i = 0; i < 2 * Chunks; ++i) f.v[i] = vrow[4 * i];
    return f;
  };
  if (bos >= eos) {  // empty sequence: the initial state goes back to the slot
    if (slot > 0) {
      char* dst_tile = reinterpret_cast<char*>(p.state + static_cast<int64_t>(slot) * p.state_slot +
                                               head_offset);
#pragma unroll
      for (int j = 0; j < kTilePieces; ++j)
        *reinterpret_cast<f32x4*>(dst_tile + (lane_bytes + tile_piece_bytes(j))) = s[j];
    }
    return;
  }
  Pending pf[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) pf[d] = fetch(bos + 1 + d);
  Pending cur = fetch(bos);
  Staged x = stage_token(cur.in, a_log, dt_bias, p.scale);
  for (int t = bos; t < eos; ++t) {
    float vv[2 * Chunks];
#pragma unroll
    for (int i = 0; i < 2 * Chunks; ++i) vv[i] = bf16_to_f32(cur.v[i]);
    const Staged now = x;
    // next token: stage it now (its inputs arrived kDepth tokens ago) and refill the queue
    cur = pf[0];
#pragma unroll
    for (int d = 0; d + 1 < kDepth; ++d) pf[d] = pf[d + 1];
    pf[kDepth - 1] = fetch(t + 1 + kDepth);
    x = stage_token(cur.in, a_log, dt_bias, p.scale);
    Vectors vec;
    vec.q0 = now.q0;
    vec.q1 = now.q1;
    vec.k0 = now.k0;
    vec.k1 = now.k1;
    float* o = s_o[wave];
    chunk_step<0, false, false, kTilePieces>(s, vec, vv[0], vv[1], o, now.decay, now.beta, kq,
                                             rsub, nullptr, lane_bytes);
    if constexpr (Chunks == 2)
      chunk_step<1, false, false, kTilePieces>(s, vec, vv[2], vv[3], o, now.decay, now.beta, kq,
                                               rsub + 8, nullptr, lane_bytes);
    // s_o is read back by other lanes of this wave: a wave's LDS operations run in program
    // order, so only the compiler must not reorder them.
    asm volatile("" ::: "memory");
    if (lane < kWaveRows)
      p.out[(static_cast<int64_t>(t) * p.num_v_heads + head) * kDim + wave_row0 + lane] =
          f32_to_bf16(s_o[wave][lane]);
    asm volatile("" ::: "memory");
  }
  if (slot > 0) {
    char* dst_tile = reinterpret_cast<char*>(p.state + static_cast<int64_t>(slot) * p.state_slot +
                                             head_offset);
#pragma unroll
    for (int j = 0; j < kTilePieces; ++j)
      *reinterpret_cast<f32x4*>(dst_tile + (lane_bytes + tile_piece_bytes(j))) = s[j];
  }
}

// The gated RMSNorm of prefill rows whose raw outputs (bf16) are already in `out`, in place,
// with the arithmetic of gdn_prefill_kernel's epilogue (same products in the same order, so
// both give the same bits).  Rows are items (token, head) over cu[0] .. cu[num_sequences] - 1;
// each wave takes kNormItems consecutive items and has all their loads in flight before the
// first sum.  Pairs: a lane's two elements as one 32-bit load or store (needs `gate` rows at
// 4-byte alignment; `out` is contiguous).
constexpr int kNormItems = 8;

template <bool WBf16, bool Pairs>
__global__ __launch_bounds__(kThreads) void prefill_norm_kernel(const DecodeParams p,
                                                                int num_sequences) {
  const int lane = threadIdx.x & 63;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6)) *
                        kNormItems;
  const int64_t lo = static_cast<int64_t>(p.cu[0]) * p.num_v_heads;
  const int64_t hi = static_cast<int64_t>(p.cu[num_sequences]) * p.num_v_heads;
  if (first >= hi || first + kNormItems <= lo) return;  // no row of this wave (or none at all)
  float w[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) w[e] = load_param(p.norm_weight, 2 * lane + e, WBf16);
  uint32_t raw_bits[kNormItems], gate_bits[kNormItems];
#pragma unroll
  for (int n = 0; n < kNormItems; ++n) {
    const int64_t item = min(max(first + n, lo), hi - 1);  // in range; unused ones not stored
    const int64_t token = item / p.num_v_heads;
    const int head = static_cast<int>(item - token * p.num_v_heads);
    const uint16_t* row = p.out + item * kDim + 2 * lane;
    const uint16_t* grow = p.gate + token * p.gate_row + head * kDim + 2 * lane;
    if (Pairs) {
      raw_bits[n] = *reinterpret_cast<const uint32_t*>(row);
      gate_bits[n] = *reinterpret_cast<const uint32_t*>(grow);
    } else {
      raw_bits[n] = row[0] | (static_cast<uint32_t>(row[1]) << 16);
      gate_bits[n] = grow[0] | (static_cast<uint32_t>(grow[1]) << 16);
    }
  }
#pragma unroll
  for (int n = 0; n < kNormItems; ++n) {
    const int64_t item = first + n;
    float raw[2], gate[2];
    raw[0] = bf16_to_f32(static_cast<uint16_t>(raw_bits[n]));
    raw[1] = bf16_to_f32(static_cast<uint16_t>(raw_bits[n] >> 16));
    gate[0] = bf16_to_f32(static_cast<uint16_t>(gate_bits[n]));
    gate[1] = bf16_to_f32(static_cast<uint16_t>(gate_bits[n] >> 16));
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) ss = fmaf(raw[e], raw[e], ss);
    ss = wave_sum(ss);
    const float rstd = fast_rsqrt(ss / static_cast<float>(kDim) + p.eps);
    uint16_t y[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) y[e] = f32_to_bf16(((raw[e] * rstd) * w[e]) * silu(gate[e]));
    if (item >= lo && item < hi) {
      uint16_t* row = p.out + item * kDim + 2 * lane;
      if (Pairs) {
        *reinterpret_cast<uint32_t*>(row) = y[0] | (static_cast<uint32_t>(y[1]) << 16);
      } else {
        row[0] = y[0];
        row[1] = y[1];
      }
    }
  }
}

template <bool Stream, int Width, int ConvCols>
void launch_decode(const DecodeParams& p, bool dt_bf16, bool w_bf16, uint32_t blocks,
                   hipStream_t stream) {
  auto kernel = dt_bf16 ? (w_bf16 ? gdn_decode_kernel<true, true, Stream, Width, ConvCols>
                                  : gdn_decode_kernel<true, false, Stream, Width, ConvCols>)
                        : (w_bf16 ? gdn_decode_kernel<false, true, Stream, Width, ConvCols>
                                  : gdn_decode_kernel<false, false, Stream, Width, ConvCols>);
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kThreads), 0, stream, p);
}

template <bool Stream>
void launch_decode(const DecodeParams& p, bool conv, bool dt_bf16, bool w_bf16,
                   uint32_t blocks, hipStream_t stream) {
  if (conv) {
    switch (p.width) {
      case 1:  // conv state of 3..4 columns (the usual width - 1 = 3), or up to 8
        if (p.conv_len <= 4)
          launch_decode<Stream, 1, 4>(p, dt_bf16, w_bf16, blocks, stream);
        else
          launch_decode<Stream, 1, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream);
        break;
      case 2: launch_decode<Stream, 2, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream); break;
      case 3: launch_decode<Stream, 3, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream); break;
      default: launch_decode<Stream, 4, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream); break;
    }
    return;
  }
  switch (p.width) {
    case 1: launch_decode<Stream, 1, 0>(p, dt_bf16, w_bf16, blocks, stream); break;
    case 2: launch_decode<Stream, 2, 0>(p, dt_bf16, w_bf16, blocks, stream); break;
    case 3: launch_decode<Stream, 3, 0>(p, dt_bf16, w_bf16, blocks, stream); break;
    default: launch_decode<Stream, 4, 0>(p, dt_bf16, w_bf16, blocks, stream); break;
  }
}

// Validates the step arguments and fills the kernel parameters; returns LD_OK, or an error
// code with the message recorded.  *blocks = 0 means there is nothing to launch.
int prepare(const ld_gdn_decode_args* args, DecodeParams& p, int64_t& blocks) {
  if (args == nullptr) return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode: args is NULL");
  const ld_gdn_decode_args& a = *args;
  blocks = 0;
  if (a.num_requests < 0) return fail(LD_ERR_INVALID_ARGUMENT, "num_requests must be >= 0");
  if (a.width < 1 || a.width > LD_MAX_TOKENS)
    return fail(LD_ERR_INVALID_ARGUMENT, "decode/MTP supports 1 through 4 tokens per request");
  if (a.num_k_heads <= 0 || a.num_v_heads <= 0 || a.num_v_heads % a.num_k_heads != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "num_v_heads must be a positive multiple of num_k_heads");
  if (!(a.eps > 0.0f)) return fail(LD_ERR_INVALID_ARGUMENT, "norm epsilon must be positive");
  if ((a.dt_bias_dtype != LD_DTYPE_F32 && a.dt_bias_dtype != LD_DTYPE_BF16) ||
      (a.norm_weight_dtype != LD_DTYPE_F32 && a.norm_weight_dtype != LD_DTYPE_BF16))
    return fail(LD_ERR_INVALID_ARGUMENT, "weights must be FP32/BF16");
  if (a.cache_policy != LD_CACHE_KEEP && a.cache_policy != LD_CACHE_STREAM)
    return fail(LD_ERR_INVALID_ARGUMENT, "cache_policy must be LD_CACHE_KEEP or LD_CACHE_STREAM");
  if (a.num_requests == 0) return LD_OK;
  if (!a.a || !a.b || !a.a_log || !a.dt_bias || !a.indices || !a.cu || !a.accepted ||
      !a.state || !a.gate || !a.norm_weight || !a.out)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode: NULL tensor pointer");
  if (!aligned16(a.state) || (a.state_slot_stride & 3) != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "state slots must be 16-byte aligned");
  blocks = static_cast<int64_t>(a.num_requests) * a.num_v_heads;
  if (blocks > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "too many (request, head) tiles");

  p = DecodeParams{};
  p.qkv = static_cast<const uint16_t*>(a.qkv);
  p.qkv_row = a.qkv_row_stride;
  p.a = static_cast<const uint16_t*>(a.a);
  p.a_row = a.a_row_stride;
  p.b = static_cast<const uint16_t*>(a.b);
  p.b_row = a.b_row_stride;
  p.a_log = a.a_log;
  p.dt_bias = a.dt_bias;
  p.indices = a.indices;
  p.cu = a.cu;
  p.accepted = a.accepted;
  p.state = a.state;
  p.state_slot = a.state_slot_stride;
  p.gate = static_cast<const uint16_t*>(a.gate);
  p.gate_row = a.gate_row_stride;
  p.norm_weight = a.norm_weight;
  p.out = static_cast<uint16_t*>(a.out);
  p.width = a.width;
  p.num_k_heads = a.num_k_heads;
  p.num_v_heads = a.num_v_heads;
  p.group = a.num_v_heads / a.num_k_heads;
  p.scale = a.scale;
  p.eps = a.eps;
  return LD_OK;
}

int launch(const ld_gdn_decode_args& a, const DecodeParams& p, int64_t blocks, bool conv,
           void* stream) {
  const bool dt_bf16 = a.dt_bias_dtype == LD_DTYPE_BF16;
  const bool w_bf16 = a.norm_weight_dtype == LD_DTYPE_BF16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.cache_policy == LD_CACHE_STREAM)
    launch_decode<true>(p, conv, dt_bf16, w_bf16, static_cast<uint32_t>(blocks), s);
  else
    launch_decode<false>(p, conv, dt_bf16, w_bf16, static_cast<uint32_t>(blocks), s);
  return check_launch(conv ? "ld_gdn_decode_conv" : "ld_gdn_decode");
}

}  // namespace
}  // namespace ld

extern "C" int ld_gdn_decode(const ld_gdn_decode_args* args, void* stream) {
  using namespace ld;
  DecodeParams p;
  int64_t blocks = 0;
  const int rc = prepare(args, p, blocks);
  if (rc != LD_OK || blocks == 0) return rc;
  if (!args->qkv) return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode: NULL tensor pointer");
  return launch(*args, p, blocks, false, stream);
}

extern "C" int ld_gdn_decode_conv(const ld_gdn_decode_args* args, const ld_conv_args* conv,
                                  void* stream) {
  using namespace ld;
  if (args == nullptr || conv == nullptr)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode_conv: args or conv is NULL");
  if (conv->width != kConvWidth) return fail(LD_ERR_INVALID_ARGUMENT, "conv width must be 4");
  if (conv->state_len < kConvWidth - 1 || conv->state_len > kMaxConvLen)
    return fail(LD_ERR_INVALID_ARGUMENT, "conv state length must be 3 through 8");
  if (conv->weight_dtype != LD_DTYPE_BF16 ||
      (conv->bias != nullptr && conv->bias_dtype != LD_DTYPE_BF16))
    return fail(LD_ERR_INVALID_ARGUMENT, "conv weight and bias must be BF16");
  if (conv->state_slots < 0 ||
      conv->state_slots * static_cast<int64_t>(args->num_k_heads) > kMaxConvTickets)
    return fail(LD_ERR_INVALID_ARGUMENT, "conv state pool too large (slots x k-heads > 2^20)");
  DecodeParams p;
  int64_t blocks = 0;
  const int rc = prepare(args, p, blocks);
  if (rc != LD_OK || blocks == 0) return rc;
  if (!conv->x || !conv->state || !conv->weight)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode_conv: NULL tensor pointer");
  if ((reinterpret_cast<uintptr_t>(conv->weight) & 7) != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "conv weight must be 8-byte aligned");
  p.conv_x = static_cast<const uint16_t*>(conv->x);
  p.conv_x_row = conv->x_row_stride;
  p.conv_state = static_cast<uint16_t*>(conv->state);
  p.conv_slot = conv->state_slot_stride;
  p.conv_dim_stride = conv->state_dim_stride;
  p.conv_len_stride = conv->state_len_stride;
  p.conv_len = conv->state_len;
  p.conv_weight = static_cast<const uint16_t*>(conv->weight);
  p.conv_bias = static_cast<const uint16_t*>(conv->bias);
  return launch(*args, p, blocks, true, stream);
}

extern "C" int ld_gdn_prefill(const ld_gdn_prefill_args* args, void* stream) {
  using namespace ld;
  if (args == nullptr) return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_prefill: args is NULL");
  const ld_gdn_prefill_args& a = *args;
  if (a.num_sequences < 0) return fail(LD_ERR_INVALID_ARGUMENT, "num_sequences must be >= 0");
  if (a.algorithm < LD_PREFILL_AUTO || a.algorithm > LD_PREFILL_CHUNKED)
    return fail(LD_ERR_INVALID_ARGUMENT, "unknown prefill algorithm");
  if (a.num_k_heads <= 0 || a.num_v_heads <= 0 || a.num_v_heads % a.num_k_heads != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "num_v_heads must be a positive multiple of num_k_heads");
  if (!(a.eps > 0.0f)) return fail(LD_ERR_INVALID_ARGUMENT, "norm epsilon must be positive");
  if ((a.dt_bias_dtype != LD_DTYPE_F32 && a.dt_bias_dtype != LD_DTYPE_BF16) ||
      (a.norm_weight_dtype != LD_DTYPE_F32 && a.norm_weight_dtype != LD_DTYPE_BF16))
    return fail(LD_ERR_INVALID_ARGUMENT, "weights must be FP32/BF16");
  if (a.num_sequences == 0) return LD_OK;
  if (!a.qkv || !a.a || !a.b || !a.a_log || !a.dt_bias || !a.slots || !a.has_initial ||
      !a.cu_seqlens || !a.state || !a.gate || !a.norm_weight || !a.out)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_prefill: NULL tensor pointer");
  if (!aligned16(a.state) || (a.state_slot_stride & 3) != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "state slots must be 16-byte aligned");
  if (a.num_tokens < 0) return fail(LD_ERR_INVALID_ARGUMENT, "num_tokens must be >= 0");
  const int64_t blocks = static_cast<int64_t>(a.num_sequences) * a.num_v_heads;
  if (blocks * 4 > 0x7fffffff || a.num_tokens * static_cast<int64_t>(a.num_v_heads) > 0x1ffffffffLL)
    return fail(LD_ERR_INVALID_ARGUMENT, "too many (sequence, head) tiles");
  DecodeParams p{};
  p.qkv = static_cast<const uint16_t*>(a.qkv);
  p.qkv_row = a.qkv_row_stride;
  p.a = static_cast<const uint16_t*>(a.a);
  p.a_row = a.a_row_stride;
  p.b = static_cast<const uint16_t*>(a.b);
  p.b_row = a.b_row_stride;
  p.a_log = a.a_log;
  p.dt_bias = a.dt_bias;
  p.indices = a.slots;
  p.has_initial = a.has_initial;
  p.cu = a.cu_seqlens;
  p.state = a.state;
  p.state_slot = a.state_slot_stride;
  p.gate = static_cast<const uint16_t*>(a.gate);
  p.gate_row = a.gate_row_stride;
  p.norm_weight = a.norm_weight;
  p.out = static_cast<uint16_t*>(a.out);
  p.width = 1;
  p.num_k_heads = a.num_k_heads;
  p.num_v_heads = a.num_v_heads;
  p.group = a.num_v_heads / a.num_k_heads;
  p.scale = a.scale;
  p.eps = a.eps;
  const bool dt_bf16 = a.dt_bias_dtype == LD_DTYPE_BF16;
  const bool w_bf16 = a.norm_weight_dtype == LD_DTYPE_BF16;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles = blocks;
  const int64_t ws_need = prefill_chunked_workspace_bytes(a.num_tokens, a.num_sequences,
                                                          a.num_v_heads);
  const bool ws_fits = a.workspace != nullptr && a.workspace_bytes >= ws_need;
  if (a.algorithm == LD_PREFILL_CHUNKED && !ws_fits)
    return fail(LD_ERR_INVALID_ARGUMENT, "chunked prefill: workspace missing or too small");
  const bool chunked =
      a.algorithm == LD_PREFILL_CHUNKED ||
      (a.algorithm == LD_PREFILL_AUTO && ws_fits &&
       prefill_auto_chunked(a.num_tokens, a.num_sequences, a.num_v_heads));
  if (chunked) {
    const int rc = launch_prefill_chunked(p, a.num_sequences, a.num_tokens, dt_bf16,
                                          a.workspace, s);
    if (rc != LD_OK) return rc;
  }
  // Token-serial: split a head's rows over more workgroups when (sequence, head) tiles alone
  // would leave the GPU short of work (1024 tiles fill 256 CUs at 4 per CU).
  const int chunks = chunked ? 0 : (tiles >= 256 ? 4 : (tiles >= 128 ? 2 : 1));
  const uint32_t grid = chunks > 0 ? static_cast<uint32_t>(tiles * (4 / chunks)) : 0u;
#define LD_PREFILL_LAUNCH(C)                                                                 \
  hipLaunchKernelGGL(dt_bf16 ? (w_bf16 ? gdn_prefill_kernel<true, true, C>                   \
                                       : gdn_prefill_kernel<true, false, C>)                 \
                             : (w_bf16 ? gdn_prefill_kernel<false, true, C>                  \
                                       : gdn_prefill_kernel<false, false, C>),               \
                     dim3(grid), dim3(kThreads), 0, s, p)
#define LD_PREFILL_ROWS_LAUNCH(C)                                                            \
  hipLaunchKernelGGL(dt_bf16 ? (w_bf16 ? gdn_prefill_rows_kernel<true, true, C>              \
                                       : gdn_prefill_rows_kernel<true, false, C>)            \
                             : (w_bf16 ? gdn_prefill_rows_kernel<false, true, C>             \
                                       : gdn_prefill_rows_kernel<false, false, C>),          \
                     dim3(grid), dim3(kThreads), 0, s, p)
  if (chunks == 4) {
    LD_PREFILL_LAUNCH(4);
  } else {
    if (chunks == 2)
      LD_PREFILL_ROWS_LAUNCH(2);
    else if (chunks == 1)
      LD_PREFILL_ROWS_LAUNCH(1);
    if (check_launch("ld_gdn_prefill") != LD_OK) return LD_ERR_LAUNCH;
    const int64_t items = a.num_tokens * static_cast<int64_t>(a.num_v_heads);
    if (items > 0) {
      const int64_t per_block = static_cast<int64_t>(kWaves) * kNormItems;
      const uint32_t norm_grid = static_cast<uint32_t>((items + per_block - 1) / per_block);
      const bool pairs = (reinterpret_cast<uintptr_t>(a.gate) & 3) == 0 && (a.gate_row_stride & 1) == 0;
#define LD_NORM_LAUNCH(W, P)                                                                  \
  hipLaunchKernelGGL((prefill_norm_kernel<W, P>), dim3(norm_grid), dim3(kThreads), 0, s, p,  \
                     a.num_sequences)
      if (w_bf16) {
        if (pairs) LD_NORM_LAUNCH(true, true); else LD_NORM_LAUNCH(true, false);
      } else {
        if (pairs) LD_NORM_LAUNCH(false, true); else LD_NORM_LAUNCH(false, false);
      }
#undef LD_NORM_LAUNCH
    }
  }
#undef LD_PREFILL_LAUNCH
#undef LD_PREFILL_ROWS_LAUNCH
  return check_launch("ld_gdn_prefill");
}

extern "C" int64_t ld_gdn_prefill_workspace_bytes(int64_t num_tokens, int32_t num_sequences,
                                                  int32_t num_v_heads) {
  if (num_tokens < 0 || num_sequences < 0 || num_v_heads < 0) return 0;
  return ld::prefill_chunked_workspace_bytes(num_tokens, num_sequences, num_v_heads);
}

extern "C" int32_t ld_gdn_prefill_auto_chunked(int64_t num_tokens, int32_t num_sequences,
                                               int32_t num_v_heads) {
  return ld::prefill_auto_chunked(num_tokens, num_sequences, num_v_heads) ? 1 : 0;
}
