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
//   * 256 threads = 4 wave64s (16 wave64s for the single-token step under the stream
//     policy and for the verify steps).  Inside a wave, the 16 lanes of a
//     DPP row span one 512-byte K row: lane kq holds k = 4kq..4kq+3 and 64+4kq..64+4kq+3 (two 16-byte pieces); the 4 DPP rows of the
//     wave take 4 consecutive V rows.  Wave w's rows are 4w..4w+3 plus multiples of 4 * waves:
//     a piece pair of all waves covers one contiguous block of the tile (16 rows = 8 KiB with
//     4 waves, the whole 32 KiB half tile with 16).  A cold in-place read-modify-write of
//     64 KiB tiles at random slots runs 13% faster laid out that way than with each wave
//     owning contiguous rows, whose first piece pairs spread over the whole tile (B=128, 16
//     waves: 85.7 against 98.0 us).  With 4 waves a lane keeps 8 V rows x 8 K values = 64 fp32
//     (16 x 128-bit loads) of the tile in VGPRs for the whole step.
//   * All tile loads are issued up front, then the slice is processed in chunks of 2 rows per
//     lane in load order: each chunk waits only for its own 4 loads, runs every token on its
//     rows and stores them, so arithmetic on chunk c overlaps the loads of the later chunks
//     and the stores of the earlier ones.
//   * Row dot products S k^ and S q^ are 8 products per lane plus a 4-step DPP butterfly
//     over the 16-lane row (quad_perm, row_half_mirror, row_mirror); every lane ends with
//     the full sums, so no LDS round trip and no broadcast step is needed.
//   * T <= 4 tokens (MTP verify) reuse the registers: 1 tile read, T tile writes.
#include "gdn_step.h"

namespace ld {
namespace {

constexpr int kConvWidth = 4;
constexpr int kMaxConvLen = 8;
// Tickets of the conv-fused variant, one per (conv slot, k-head); see gdn_decode_kernel.
constexpr int kMaxConvTickets = 1 << 20;
__device__ uint32_t g_conv_ticket[kMaxConvTickets];

// Destination of the state of a token that has no slot to go to (past the request's last
// token, or a padding slot) under pointer stores: one tile, written and never read.
__device__ __align__(256) f32x4 g_state_sink[kDim * kDim / 4];

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

// Counts a workgroup in on a conv ticket of a k-head group of `group` workgroups: a wrapping
// increment (global_atomic_inc: the ticket becomes 0 when it held group - 1, else its value
// + 1) that returns the previous count, so the workgroup that counts in last receives
// group - 1 and leaves the ticket at 0 for the next launch, with no store of its own.  Any
// sequence of arrivals whose number is a multiple of `group` (every launch: each valid
// request counts its group in once per k-head, a repeated conv slot in one batch twice)
// returns the ticket to where it was.  Relaxed, agent scope: the count orders nothing; the
// conv-state reads it follows were consumed before it is issued.
__device__ __forceinline__ uint32_t count_in(uint32_t* ticket, int group) {
  return __builtin_amdgcn_atomic_inc32(ticket, static_cast<uint32_t>(group - 1), __ATOMIC_RELAXED,
                                       "agent");
}

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
// The inputs of one channel's conv over a verify step: its state columns, the tokens'
// inputs, weights and bias (the weight array stands in for a missing bias).
struct ConvIn {
  Packed8 st, x;
  uint32_t w[2];
  uint16_t bias;
};

// Fills `in` in place: a ConvIn returned by value was left as a private aggregate, which the
// backend then placed in LDS (48 bytes a thread per channel).
template <int Width, int Cols>
__device__ __forceinline__ void conv_load(const DecodeParams& p, int64_t bos, int n,
                                          int64_t state_at, int channel, ConvIn& in) {
  static_assert(Cols <= 8 && Width <= 4, "packed conv registers hold 8 columns, 4 tokens");
#pragma unroll
  for (int j = 0; j < Cols; ++j)
    in.st.set(j, p.conv_state[state_at + min(j, p.conv_len - 1) * p.conv_len_stride]);
#pragma unroll
  for (int t = 0; t < Width; ++t)
    in.x.set(t, p.conv_x[(bos + min(t, n - 1)) * p.conv_x_row + channel]);
  const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(p.conv_weight + channel * kConvWidth);
  in.w[0] = wsrc[0];
  in.w[1] = wsrc[1];
  in.bias = (p.conv_bias != nullptr ? p.conv_bias : p.conv_weight)[channel];
}

// `in` by value, its weights copied into a local array for conv_dot: a reference into the
// caller's ConvIn kept that aggregate in memory.
template <int Width, int Cols>
__device__ __forceinline__ void conv_compute(const ConvIn in, int len, int n, int offset,
                                             bool has_bias, uint16_t* out,
                                             uint16_t (&new_state)[Cols]) {
  const uint32_t w[2] = {in.w[0], in.w[1]};
  uint16_t seq[3 + Width];
#pragma unroll
  for (int m = 0; m < 3; ++m) seq[m] = in.st.get(offset + m);
#pragma unroll
  for (int t = 0; t < Width; ++t) seq[3 + t] = in.x.get(t);
#pragma unroll
  for (int t = 0; t < Width; ++t)
    out[t * 3 * kDim] = conv_dot(seq[t], seq[t + 1], seq[t + 2], seq[t + 3], w, in.bias,
                                 has_bias);
  const int kept = len - n;  // state columns that survive (<= 0: none)
#pragma unroll
  for (int k = 0; k < Cols; ++k) {
    const int col = min(k, len - 1);
    new_state[k] = col < kept ? in.st.get(offset + 1 + col) : in.x.get(col - kept);
  }
}

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


// The LDS arrays of one gdn_decode_kernel workgroup, as types, so that the kernel declares
// them from here and the launch can bound their total at compile time (kBytes: every array
// rounded up to 16 bytes; arrays a kernel does not use are dropped by the compiler, so its
// static LDS is at most this).  Token 0 staged per wave (or, for verify steps with 16 waves,
// once), MTP tokens 1..W-1, the raw outputs of every row for the epilogue.
template <int Width, int ConvCols, int Waves, bool Packed>
struct DecodeLds {
  static constexpr bool kShared0 = Width > 1 && Waves == 16;
  static constexpr bool kConv = ConvCols > 0;
  static constexpr int kCols = kConv ? ConvCols : 1;
  using Qk0 = f32x4[kShared0 ? 1 : Waves][2][kDim / 4];  // token 0: q^, k^ in the lane layout
  using V0 = float[kShared0 ? 1 : Waves][kDim / Waves];  // token 0: v of the wave's rows
  using Db0 = float[kShared0 ? 1 : Waves][2];            // token 0: decay, beta
  using Qkt = f32x4[Width][2][kDim / 4];                 // token t (shared staging)
  using Vt = float[Width][kDim];
  using Dbt = float[Width][2];
  using O = float[Width][kDim];                          // raw outputs of token t
  // Epilogue inputs, parked here once they arrive so that no register holds them through the
  // recurrence: silu(gate) of token t (written by wave t) and the norm weight (wave 0).
  using Sg = float[Width][kDim];
  using W = float[kDim];
  // Conv variant: bf16 conv outputs of the 256 q/k channels and 128 v channels per token,
  // and the shifted q/k conv state kept for the end-of-kernel write.
  using Conv = uint16_t[kConv ? Width : 1][kConv ? 3 * kDim : 2];
  using ConvNew = uint16_t[kConv && !Packed ? 2 * kDim : 1][kCols];
  // Packed conv state: per wave, the 16-byte pieces of its q/k ([0]) and v ([1]) channels'
  // columns (4 waves), or of its one run of 64 channels (16 waves: waves 0..5), then their
  // shifted columns.
  using Cpk = u32x4[Packed ? (Waves == 16 ? 6 : Waves) : 1][Waves == 16 ? 1 : 2][32];
  static constexpr size_t up16(size_t n) { return (n + 15) / 16 * 16; }
  static constexpr size_t kBytes =
      up16(sizeof(Qk0)) + up16(sizeof(V0)) + up16(sizeof(Db0)) + up16(sizeof(Qkt)) +
      up16(sizeof(Vt)) + up16(sizeof(Dbt)) + up16(sizeof(O)) + up16(sizeof(Sg)) +
      up16(sizeof(W)) + up16(sizeof(Conv)) + up16(sizeof(ConvNew)) + up16(sizeof(uint32_t)) +
      up16(sizeof(Cpk));
};

// Four waves per SIMD (<= 128 VGPRs) keep four workgroups, i.e. four tiles, resident per CU.
// DtBf16 / WBf16: dt_bias / norm_weight stored as bf16 (else fp32).  LoadPol / StorePol: cache
// policy bits of the state loads and stores (kPolPlain, kPolNT, kPolSys; never a change of
// results).  Width: the indices width W (tokens per request at most); fixing it at compile
// time unrolls every token loop into straight-line code, which keeps the tile's per-piece load
// waits exact.
//
// Conv: the causal depthwise conv1d (width 4, SiLU) runs first on the pre-conv activations.
// Each workgroup convolves the 256 q/k channels of its k-head and the 128 v channels of its
// head from the conv state of the request's slot, rounds the outputs to bf16 (the dtype an
// unfused conv writes) and feeds them to the GDN step; one token (W = 1) while the tile
// streams in, several (speculative verify, W > 1) before the tile loads.  Its own v
// channels' conv state is updated in place.  The q/k channels are shared by the
// HV/H workgroups of a k-head group, so their shifted state is written only after all of
// them have read it: every workgroup counts itself in (count_in, a wrapping increment of
// g_conv_ticket[slot*H + kh] that returns the previous count) after its reads; the one that
// receives HV/H - 1 counted in last and writes the shifted state at its end; its increment
// returned the ticket to 0.  Nothing waits on another workgroup, and every launch leaves the
// tickets as it found them.  ConvCols: conv-state columns held per channel (4 for states of
// 3..4 columns, 8 for up to 8; 0 = no conv).
//
// Packed (one token, ConvCols 4): the conv pool is dim-first and dense (a slot's channels
// consecutive, each channel's columns consecutive) and 16-byte aligned, so the 64 channels of
// a wave's q/k (or v) conv state are one run of 128 * len bytes: the wave reads it with one
// 16-byte load per lane, redistributes it through wave-private LDS, and writes the shifted
// state back the same way (16-byte stores), instead of one 2-byte access per channel and
// column (B=32, 3 columns: 22.04 -> 21.41 us, bit-identical results).  With 16 waves, waves
// 0..5 each own one run, the 64 channels they convolve (B=32 cache-cold: 27.35 -> 26.84 us;
// B=128: 94.05 -> 93.71 us; bit-identical).
//
// Waves: 4 (32 V rows and 16 tile pieces per wave), or 16 (8 rows, 4 pieces) for the
// single-token step under the stream policy and for every verify step.  A
// cold in-place read-modify-write of 64 KiB per workgroup in this layout runs at 6.26 TB/s
// as 1024 threads x 4 pieces against 5.63 as 256 x 16 (B=128 tiles at random slots,
// non-temporal loads, system-scope stores).
// Waves per SIMD the register allocation aims at: 4 (four 4-wave workgroups per CU, or one
// 16-wave workgroup for the conv-fused verify: at 8, two per CU, it spilled 1-6 VGPRs and
// ran 131.2 against 123.5 us cold at B=64, T=4) or 8 (two 16-wave workgroups, the
// conv-fused single token included).
constexpr int waves_per_simd(int waves, int conv_cols, int width) {
  return waves == kWaves || (conv_cols > 0 && width > 1) ? 4 : 8;
}

template <bool DtBf16, bool WBf16, int LoadPol, int StorePol, int Width, int ConvCols,
          int Waves = kWaves, bool Packed = false>
__global__ __launch_bounds__(64 * Waves)
__attribute__((amdgpu_waves_per_eu(waves_per_simd(Waves, ConvCols, Width),
                                   waves_per_simd(Waves, ConvCols, Width))))
void gdn_decode_kernel(const int32_t* md_indices, const int32_t* md_cu,
                       const int32_t* md_accepted, int md_num_v_heads, const DecodeParams args) {
  // The request metadata pointers and the head count are kernel arguments of their own, ahead
  // of the parameter block: the build preloads the first 7 argument dwords into SGPRs
  // (-amdgpu-kernarg-preload-count=7), so the metadata loads go out at once instead of after
  // the argument segment's round trip (19.97 -> 19.82 us at B=32, back-to-back A/B runs on
  // one MI355X).
  constexpr bool Conv = ConvCols > 0;
  constexpr int kCols = Conv ? ConvCols : 1;
  constexpr int kBlock = 64 * Waves;           // threads
  constexpr int kRows = kDim / Waves;          // V rows per wave
  constexpr int kPc = kRows / 2;               // 16-byte tile pieces per lane
  // A piece pair of every wave (4 rows per wave) covers one contiguous block of 4 * Waves
  // rows: lane (rsub, kq) of wave w holds rows 4w + rsub + kPair * i, i < kPc / 2.
  constexpr int kPair = 4 * Waves;
  // Token 0 staged by every wave for itself (no barrier before the recurrence), or -- verify
  // steps with 16 waves, whose registers (<= 64 for 8 waves per SIMD) do not hold two tokens'
  // inputs at once -- by wave 0 once, like tokens 1..W-1, behind one barrier.
  constexpr bool kShared0 = Width > 1 && Waves == 16;
  constexpr int kChunks = kPc / 4;             // chunks of 2 rows per lane (8 per wave)
  static_assert(Waves == kWaves || Waves == 16, "4 or 16 waves");
  // The conv runs before the tile loads for several tokens or more than 4 state columns;
  // one token with 3..4 columns keeps it in registers while the tile streams in.
  // The conv of a verify step with 16 waves: one channel per thread (0..255 q/k, 256..383
  // v), its inputs loaded before the tile and convolved while the tile streams in.
  constexpr bool kConvSplit = Conv && Width > 1 && Waves == 16;
  // One token, 3..4 state columns, 16 waves: one channel per thread (0..255 q/k, 256..383
  // v), its inputs loaded ahead of the tile and convolved while the tile streams in, in 6
  // registers, so that two workgroups fit a CU; Packed: each of waves 0..5 moves its 64
  // channels' columns as one run of 16-byte pieces.
  constexpr bool kConvOne16 = Conv && Width == 1 && kCols <= 4 && Waves == 16;
  constexpr bool kConvFirst = Conv && (Width > 1 || kCols > 4) && !kConvSplit;
  constexpr bool kConvLate = Conv && !kConvFirst && !kConvSplit && !kConvOne16;
  static_assert(!kConvLate || kCols == 4, "the in-flight conv holds 4 state columns");
  static_assert(!kConvLate || Waves == kWaves, "the in-flight conv runs with 4 waves");
  static_assert(!Packed || (kConvLate && Waves == 4) || kConvOne16,
                "the packed conv state: one token with 3..4 columns");
  // Every kernel argument, then all request metadata, is loaded before the first branch:
  // two dependent scalar round trips (kernel-argument segment; cu/accepted/indices) instead
  // of the compiler's default of sinking each load to its first use behind the early exits.
  // The pins come after the metadata loads: a pin is opaque to the compiler, and scalar
  // (s_load) metadata loads must not follow anything that might have written memory.
  const DecodeParams& p = args;
  const int tile = blockIdx.x;
  const int request = tile / md_num_v_heads;
  const int head = tile - request * md_num_v_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // The same as a scalar the compiler knows to be wave-uniform, for branches on the wave's
  // role (a per-lane compare of tid kept its 64-bit mask alive across the conv, which spilled
  // SGPRs in the 16-wave single-token conv).
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);

  // Request metadata in one round trip: token range, accepted count and the (at most 4)
  // slots of the request, read before any state store.
  const int32_t* req_slots = md_indices + static_cast<int64_t>(request) * Width;
  const int bos = md_cu[request];
  const int eos = md_cu[request + 1];
  const int accepted = md_accepted[request];
  int slot[Width];
#pragma unroll
  for (int t = 0; t < Width; ++t) slot[t] = req_slots[t];
#pragma unroll
  for (int t = 0; t < Width; ++t) pin_sgpr(slot[t]);
  pin_sgpr(bos);
  pin_sgpr(eos);
  pin_sgpr(accepted);
  // The step's arguments too -- except where the conv runs to completion before the tile
  // loads (several tokens, or a long conv state): those have no loads to get ahead of, and
  // holding every argument through the conv would exceed the 102 SGPRs.
  if constexpr (!kConvFirst && !kConvSplit) {
    if constexpr (!Conv) {  // the conv variant reads its activations from conv_x
      pin_sgpr(p.qkv);
      pin_sgpr(p.qkv_row);
    }
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
  }
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
    for (int i = tid; i < num_tokens * kDim; i += kBlock) {
      const int64_t token = bos + (i >> 7);
      p.out[(token * p.num_v_heads + head) * kDim + (i & (kDim - 1))] = 0;
    }
    return;
  }

  // Token 0 is staged by every wave for itself (wave-private LDS, no barrier before the
  // recurrence): q^ and k^ (128 each), v of the wave's 32 rows, decay and beta.  MTP tokens
  // t >= 1 are staged once, by wave t, in the shared area (one barrier, after chunk 0's
  // token 0).  s_o collects the raw outputs of all rows for the epilogue.
  // (the array types, and what each holds, are DecodeLds')
  using Lds = DecodeLds<Width, ConvCols, Waves, Packed>;
  __shared__ typename Lds::Qk0 s_qk0;
  __shared__ typename Lds::V0 s_v0;
  __shared__ typename Lds::Db0 s_db0;
  __shared__ typename Lds::Qkt s_qkt;
  __shared__ typename Lds::Vt s_vt;
  __shared__ typename Lds::Dbt s_dbt;
  __shared__ typename Lds::O s_o;
  __shared__ typename Lds::Sg s_sg;
  __shared__ typename Lds::W s_w;
  __shared__ typename Lds::Conv s_conv;
  __shared__ typename Lds::ConvNew s_conv_new;
  __shared__ uint32_t s_arrived;
  __shared__ typename Lds::Cpk s_cpk;

  const int key_head = head / p.group;
  const int kq = lane & 15;
  const int rsub = lane >> 4;
  const int row_base = 4 * wave + rsub;  // V row of the lane's piece 0
  // Row of the wave's i-th staged v value (i < kRows): the rows of its lanes, in the order
  // chunk_step reads them (s_v0[wave][8C + rsub] and [8C + 4 + rsub] for chunk C).
  const int v_row = 4 * wave + (lane & 3) + kPair * ((lane & (kRows - 1)) >> 2);
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;

  // ---- small activation loads go out before the tile, so they return first: token 0 in
  // the lane layout of the tile (q, k at 4kq.. and 64+4kq..; v of the wave's 32 rows), the
  // MTP token `wave` for the shared staging, and the epilogue inputs of token `wave` ----
  TokenIn in0;
  // Conv variant with 4 waves: this thread convolves q/k channel `conv_qk` and (tid < 128)
  // v channel `conv_v`; it loads their input, conv-state columns (clamped to the last
  // column past conv_len, so every load is in bounds), weights and bias.
  const int ctid = tid & (2 * kDim - 1);
  const int conv_qk = ctid < kDim ? q_col + ctid : k_col + (ctid - kDim);
  const int conv_v = v_col + (ctid & (kDim - 1));
  const int64_t conv_slot_at = static_cast<int64_t>(slot[0]) * p.conv_slot;
  int64_t cs_qk_at = conv_slot_at + conv_qk * p.conv_dim_stride;
  int64_t cs_v_at = conv_slot_at + conv_v * p.conv_dim_stride;
  // kConvSplit: thread tid < 384 convolves one channel, q/k channel tid or v channel
  // tid - 256 (waves 6..15 load no conv inputs; one channel per thread instead of a q/k and
  // a v channel on every thread: 128.5 -> 123.5 us cold, 107.8 -> 104.5 hot at B=64, T=4,
  // 94 -> 69 VGPRs, identical bits)
  const int conv_ch3 = tid < 2 * kDim ? conv_qk : v_col + ((tid - 2 * kDim) & (kDim - 1));
  const int64_t cs3_at = conv_slot_at + conv_ch3 * p.conv_dim_stride;
  uint16_t cx_qk = 0, cx_v = 0, cb_qk = 0, cb_v = 0;
  uint16_t cs_qk_raw[kConvLate ? 4 : 1], cs_v_raw[kConvLate ? 4 : 1];
  uint32_t cw_qk[2], cw_v[2];
  uint32_t arrived = 0;  // ticket count before this workgroup's increment (thread 0)
  ConvIn ci;             // kConvSplit: the channel's conv inputs, loaded ahead of the tile
  // kConvOne16: the thread's channel (state columns as bf16 pairs, input, weights, bias)
  uint32_t c1_st[2] = {0u, 0u}, c1_w[2] = {0u, 0u};
  uint16_t c1_x = 0, c1_bias = 0;
  int64_t c1_at = 0;
  // Packed: the wave's first q/k and v channel (waves 0, 1: q channels 0..63, 64..127;
  // waves 2, 3: the k channels; the v channels of waves 2, 3 repeat those of 0, 1), and the
  // lane's 16-byte piece of a 128 * len-byte run (lanes past its 8 * len pieces repeat the
  // last one; lanes 0..31 read the q/k run, 32..63 the v run).
  // 16 waves (kConvOne16): wave w < 6 owns one run, the 64 channels it convolves (waves 0, 1
  // the q channels, 2, 3 the k channels, 4, 5 the v channels): pk_qk0 is its first channel
  // for w < 4, pk_v0 for w = 4, 5; lane l holds piece min(l, 8 * len - 1) of the run.
  const int pk_qk0 = wave < 2 ? q_col + 64 * wave : k_col + 64 * ((wave - 2) & 1);
  const int pk_v0 = v_col + 64 * (wave & 1);
  const int pk_piece = min(Waves == 16 ? lane : lane & 31, 8 * p.conv_len - 1);
  u32x4 pk_raw = {0u, 0u, 0u, 0u};
  if constexpr (kConvFirst) {
    // Several tokens (speculative verify), or a long conv state: the conv runs to
    // completion before the tile loads, so its inputs do not compete with the tile for
    // registers.  Threads 0..255 convolve (with 16 waves, waves 4..15 only wait at the
    // barrier).  The v channels are this workgroup's alone and are shifted in place
    // (threads 128..255 repeat the stores of 0..127 with identical bytes); the q/k channels
    // are kept for the end-of-kernel write.
    const bool convolves = Waves == kWaves || tid < 2 * kDim;   // wave-uniform
    uint16_t qk_new[kCols], v_new[kCols];
    if (convolves) {
      const bool has_bias = p.conv_bias != nullptr;
      conv_channel_tokens<Width, kCols>(p, bos, num_tokens, conv_offset, cs_qk_at, conv_qk,
                                        has_bias, &s_conv[0][tid], qk_new);
      conv_channel_tokens<Width, kCols>(p, bos, num_tokens, conv_offset, cs_v_at, conv_v,
                                        has_bias, &s_conv[0][2 * kDim + (tid & (kDim - 1))],
                                        v_new);
#pragma unroll
      for (int k = 0; k < kCols; ++k) s_conv_new[tid][k] = qk_new[k];
    }
    // Every wave has consumed its conv-state reads once past the barrier, so the v channels
    // (read by two threads each) can be overwritten.
    lds_barrier();
    if (convolves) {
#pragma unroll
      for (int k = 0; k < kCols; ++k)
        p.conv_state[cs_v_at + min(k, p.conv_len - 1) * p.conv_len_stride] = v_new[k];
    }
    if (p.group > 1 && tid == 0)
      arrived = count_in(&g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head],
                         p.group);
    in0.a = p.a[static_cast<int64_t>(bos) * p.a_row + head];
    in0.b = p.b[static_cast<int64_t>(bos) * p.b_row + head];
  } else if constexpr (kConvSplit) {
    if (tid < 3 * kDim) conv_load<Width, kCols>(p, bos, num_tokens, cs3_at, conv_ch3, ci);
  } else if constexpr (kConvOne16) {
    if (wave_s < 6) {  // every column clamped to the state's last
      const int ch = tid < kDim ? q_col + tid
                                : (tid < 2 * kDim ? k_col + (tid - kDim) : v_col + (tid - 2 * kDim));
      c1_at = conv_slot_at + ch * p.conv_dim_stride;
      c1_x = p.conv_x[static_cast<int64_t>(bos) * p.conv_x_row + ch];
      if constexpr (Packed) {  // the wave's run, one 16-byte piece per lane
        pk_raw = *reinterpret_cast<const u32x4*>(
            p.conv_state + conv_slot_at + static_cast<int64_t>(wave < 4 ? pk_qk0 : pk_v0) *
                                              p.conv_len + 8 * pk_piece);
      } else {
        uint32_t st[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st[j] = p.conv_state[c1_at + min(j, p.conv_len - 1) * p.conv_len_stride];
        c1_st[0] = st[0] | (st[1] << 16);
        c1_st[1] = st[2] | (st[3] << 16);
      }
      const uint32_t* wsrc = reinterpret_cast<const uint32_t*>(p.conv_weight + ch * kConvWidth);
      c1_w[0] = wsrc[0];
      c1_w[1] = wsrc[1];
      c1_bias = (p.conv_bias != nullptr ? p.conv_bias : p.conv_weight)[ch];
    }
    in0.a = p.a[static_cast<int64_t>(bos) * p.a_row + head];
    in0.b = p.b[static_cast<int64_t>(bos) * p.b_row + head];
  } else if constexpr (kConvLate) {
    const uint16_t* xrow = p.conv_x + static_cast<int64_t>(bos) * p.conv_x_row;
    cx_qk = xrow[conv_qk];
    cx_v = xrow[conv_v];
    if constexpr (Packed) {
      pk_raw = *reinterpret_cast<const u32x4*>(
          p.conv_state + conv_slot_at + static_cast<int64_t>(lane < 32 ? pk_qk0 : pk_v0) * p.conv_len +
          8 * pk_piece);
    } else {
#pragma unroll
      for (int j = 0; j < kCols; ++j) {
        const int64_t col = min(j, p.conv_len - 1) * p.conv_len_stride;
        cs_qk_raw[j] = p.conv_state[cs_qk_at + col];
        cs_v_raw[j] = p.conv_state[cs_v_at + col];
      }
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
  } else if constexpr (!kShared0) {
    in0 = load_token(p, bos, q_col, k_col, v_col + v_row, head, kq);
  }
  // Every MTP token slot t < W is staged and stepped, past the request's last token too
  // (with a copy of that token), so the token loops have no branches; such tokens' states
  // go to the sink tile (non-temporal stores) or are not stored, and their outputs are not
  // written.
  const bool stages_mtp = Width > 1 && wave >= (kShared0 ? 0 : 1) && wave < Width;
  const int64_t token_w = bos + min(wave, num_tokens - 1);
  TokenIn inw;
  uint16_t vw_hi = 0;
  // post-conv token from LDS, for the split conv (in the staging below, after its barrier)
  auto conv_token_w = [&]() {
    const uint16_t* conv_w = s_conv[min(wave, num_tokens - 1)];
    const TokenIn t = conv_token(conv_w, kq);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      inw.q[e] = t.q[e];
      inw.k[e] = t.k[e];
    }
    inw.v = conv_w[2 * kDim + 2 * lane];
    vw_hi = conv_w[2 * kDim + 2 * lane + 1];
  };
  if constexpr (Conv && Width > 1 && !kConvSplit) {  // post-conv token from LDS (barrier above)
    const uint16_t* conv_w = s_conv[min(wave, num_tokens - 1)];
    inw = conv_token(conv_w, kq);
    inw.v = conv_w[2 * kDim + 2 * lane];
    vw_hi = conv_w[2 * kDim + 2 * lane + 1];
    inw.a = p.a[token_w * p.a_row + head];
    inw.b = p.b[token_w * p.b_row + head];
  } else if constexpr (kConvSplit) {
    inw.a = p.a[token_w * p.a_row + head];
    inw.b = p.b[token_w * p.b_row + head];
  } else if (Width > 1) {
    inw = load_token(p, token_w, q_col, k_col, v_col + 2 * lane, head, kq);
    vw_hi = p.qkv[token_w * p.qkv_row + v_col + 2 * lane + 1];
  }
  // The epilogue's inputs (gate row of token `wave`, norm weight).  Without a conv and with
  // one token they are loaded behind the tile and parked in LDS after the chunks, so that
  // nothing but the token's own inputs stands in front of the tile's loads (B=32 hot
  // 19.76 -> 19.38 us, cold 24.65 -> 24.57 us, bit-identical); the conv-fused and verify
  // kernels load them ahead, as they stage them before the recurrence (the conv-fused
  // single token measured 21.36 -> 21.52 us the other way).
  uint16_t gh[2];
  float w[2];
  constexpr bool kLate = Width == 1 && !Conv;
  auto load_epi = [&]() {
    const uint16_t* grow = p.gate + token_w * p.gate_row + head * kDim;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      gh[e] = grow[2 * lane + e];
      w[e] = load_param(p.norm_weight, 2 * lane + e, WBf16);
    }
  };
  if constexpr (!kLate) load_epi();
  const float dt_bias = load_param(p.dt_bias, head, DtBf16);
  const float a_log = p.a_log[head];
  __builtin_amdgcn_sched_barrier(0);

  // ---- the whole 64 KiB source tile: 16 x 128-bit loads per lane (uniform base address,
  // 32-bit per-lane byte offsets), issued in chunk order ----
  const int64_t head_offset = static_cast<int64_t>(head) * kDim * kDim;
  const uint32_t lane_bytes = static_cast<uint32_t>(row_base * kDim + kq * 4) * 4u;
  const char* src_tile = reinterpret_cast<const char*>(
      p.state + static_cast<int64_t>(source) * p.state_slot + head_offset);
  f32x4 s[kPc];
#pragma unroll
  for (int j = 0; j < kPc; ++j) {
    s[j] = load_tile_piece<LoadPol>(src_tile, lane_bytes + tile_piece_bytes<kPair>(j));
    __builtin_amdgcn_sched_barrier(0);  // keep program order: chunk c's loads issue first
  }
  if constexpr (kLate) load_epi();  // after the tile's loads
  __builtin_amdgcn_sched_barrier(0);

  // ---- staging, while the tile streams in ----
  uint16_t v_new_split[kConvSplit ? kCols : 1];
  if constexpr (kConvSplit) {
    const bool convolves = tid < 3 * kDim;   // wave-uniform
    if (convolves) {
      const bool has_bias = p.conv_bias != nullptr;
      uint16_t new_st[kCols];
      conv_compute<Width, kCols>(ci, p.conv_len, num_tokens, conv_offset, has_bias,
                                 &s_conv[0][tid], new_st);
      if (tid < 2 * kDim) {
#pragma unroll
        for (int k = 0; k < kCols; ++k) s_conv_new[tid][k] = new_st[k];
      } else {
#pragma unroll
        for (int k = 0; k < kCols; ++k) v_new_split[k] = new_st[k];
      }
    }
    // conv outputs visible to every wave; every conv-state read of the workgroup consumed
    // (the shifted v state and the ticket follow the tokens' staging, off its path)
    lds_barrier();
    conv_token_w();
  }
  if constexpr (kConvOne16) {
    if (wave_s < 6) {
      const int len = p.conv_len;
      uint16_t st[4];
      if constexpr (Packed) {  // the lane's channel's columns out of the wave's run
        // lanes with the same piece index hold the same piece: their writes agree
        s_cpk[wave][0][pk_piece] = pk_raw;
        lds_order();
        const uint16_t* run = reinterpret_cast<const uint16_t*>(s_cpk[wave][0]) + lane * len;
#pragma unroll
        for (int j = 0; j < 4; ++j) st[j] = run[min(j, len - 1)];
      } else {
        st[0] = static_cast<uint16_t>(c1_st[0]);
        st[1] = static_cast<uint16_t>(c1_st[0] >> 16);
        st[2] = static_cast<uint16_t>(c1_st[1]);
        st[3] = static_cast<uint16_t>(c1_st[1] >> 16);
      }
      s_conv[0][tid] = conv_output(c1_x, st, c1_w, c1_bias, p.conv_bias != nullptr);
      // shifted state: columns 1..len-1, then the new input; q/k kept for the end-of-kernel
      // write, the thread's own v channel shifted in place (only it reads that channel)
      uint16_t shifted[kCols];
#pragma unroll
      for (int j = 0; j < kCols; ++j) shifted[j] = j + 1 < len ? st[j + 1 < kCols ? j + 1 : j] : c1_x;
      if constexpr (Packed) {  // shifted columns into the run (its old values were read above)
        uint16_t* run = reinterpret_cast<uint16_t*>(s_cpk[wave][0]) + lane * len;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j < len) run[j] = shifted[j];
        lds_order();
        // waves 4, 5: the v run back to the pool, one 16-byte piece per lane (lanes past the
        // run's last piece repeat it with the same bytes)
        if (wave_s >= 4)
          *reinterpret_cast<u32x4*>(p.conv_state + conv_slot_at +
                                    static_cast<int64_t>(pk_v0) * len + 8 * pk_piece) =
              s_cpk[wave][0][pk_piece];
      } else if (wave_s < 4) {
#pragma unroll
        for (int j = 0; j < kCols; ++j) s_conv_new[tid][j] = shifted[j];
      } else {
#pragma unroll
        for (int j = 0; j < kCols; ++j)
          p.conv_state[c1_at + min(j, len - 1) * p.conv_len_stride] = shifted[j];
      }
    }
    // conv outputs visible to every wave; every q/k conv-state read of the workgroup consumed
    lds_barrier();
    if (p.group > 1 && tid == 0)
      arrived = count_in(&g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head],
                         p.group);
  }
  if constexpr (kConvLate) {
    const int len = p.conv_len;
    const bool has_bias = p.conv_bias != nullptr;
    if constexpr (Packed) {  // the lane's channels' columns out of the wave's runs
      s_cpk[wave][lane >> 5][lane & 31] = pk_raw;
      lds_order();
      const uint16_t* run_qk = reinterpret_cast<const uint16_t*>(s_cpk[wave][0]) + lane * len;
      const uint16_t* run_v = reinterpret_cast<const uint16_t*>(s_cpk[wave][1]) + lane * len;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cs_qk_raw[j] = run_qk[min(j, len - 1)];
        cs_v_raw[j] = run_v[min(j, len - 1)];
      }
    }
    s_conv[0][tid] = conv_output(cx_qk, cs_qk_raw, cw_qk, cb_qk, has_bias);
    if (tid < kDim) s_conv[0][2 * kDim + tid] = conv_output(cx_v, cs_v_raw, cw_v, cb_v, has_bias);
    // Shifted state: columns 1..len-1, then the new input.  The q/k channels are kept for
    // the end-of-kernel write.
    uint16_t qk_new[kCols], v_new[kCols];
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      qk_new[j] = j + 1 < len ? cs_qk_raw[j + 1 < kCols ? j + 1 : j] : cx_qk;
      v_new[j] = j + 1 < len ? cs_v_raw[j + 1 < kCols ? j + 1 : j] : cx_v;
    }
    if constexpr (Packed) {  // shifted columns into the runs (their old values were read above)
      uint16_t* run_qk = reinterpret_cast<uint16_t*>(s_cpk[wave][0]) + lane * len;
      uint16_t* run_v = reinterpret_cast<uint16_t*>(s_cpk[wave][1]) + lane * len;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < len) {
          run_qk[j] = qk_new[j];
          run_v[j] = v_new[j];
        }
      lds_order();
    } else {
#pragma unroll
      for (int j = 0; j < kCols; ++j) s_conv_new[tid][j] = qk_new[j];
    }
    // Conv outputs visible to every wave; every conv-state read of this workgroup consumed.
    lds_barrier();
    // The v channels (this workgroup's alone) are shifted in place; threads 128..255 repeat
    // the stores of threads 0..127 with identical bytes (both read the channel before the
    // barrier), and columns past len-1 repeat column len-1, so the stores need no branch (a
    // store under a branch makes later load waits conservative).
    if constexpr (Packed) {
      *reinterpret_cast<u32x4*>(p.conv_state + conv_slot_at + static_cast<int64_t>(pk_v0) * len +
                                8 * pk_piece) = s_cpk[wave][1][pk_piece];
    } else {
#pragma unroll
      for (int j = 0; j < kCols; ++j)
        p.conv_state[cs_v_at + min(j, len - 1) * p.conv_len_stride] = v_new[j];
    }
    // Relaxed: every conv-state value this workgroup read has already been consumed (the
    // barrier above follows the conv arithmetic), so the increment cannot overtake a read.
    // The returned count is first used at the kernel's end, by which time it has long
    // arrived: no wait on the tile stream here, and no extra round trip there.
    if (p.group > 1 && tid == 0)
      arrived = count_in(&g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head],
                         p.group);
  }
  if constexpr (Conv) {  // token 0 after the conv, from LDS
    const TokenIn c = conv_token(s_conv[0], kq);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      in0.q[e] = c.q[e];
      in0.k[e] = c.k[e];
    }
    in0.v = s_conv[0][2 * kDim + v_row];
  }
  if constexpr (!kShared0) {
    const Staged x = stage_token(in0, a_log, dt_bias, p.scale);
    if (rsub == 0) {
      s_qk0[wave][0][kq] = x.q0;
      s_qk0[wave][0][16 + kq] = x.q1;
      s_qk0[wave][1][kq] = x.k0;
      s_qk0[wave][1][16 + kq] = x.k1;
    }
    if (lane < kRows) s_v0[wave][lane] = bf16_to_f32(in0.v);
    if (lane == 0) {
      s_db0[wave][0] = x.decay;
      s_db0[wave][1] = x.beta;
    }
  }
  auto stage_epi = [&]() {
    if (wave < Width) {
#pragma unroll
      for (int e = 0; e < 2; ++e) s_sg[wave][2 * lane + e] = silu(bf16_to_f32(gh[e]));
    }
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < 2; ++e) s_w[2 * lane + e] = w[e];
    }
  };
  if constexpr (!kLate) stage_epi();
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
  // Token t's state goes to slot indices[r, t]; past the request's last token or to a padding
  // slot it goes nowhere (TileStore: sink tile or empty resource, no branch).
  TileStore<StorePol> dst[Width];
#pragma unroll
  for (int t = 0; t < Width; ++t) {
    const bool stored = t < num_tokens && slot[t] > 0;
    dst[t].set(reinterpret_cast<char*>(p.state + static_cast<int64_t>(stored ? slot[t] : 0) *
                                                     p.state_slot + head_offset),
               stored, reinterpret_cast<char*>(g_state_sink));
  }

#define LD_CHUNK(C)                                                                         \
  {                                                                                         \
    const int r = row_base + 2 * kPair * (C);                                               \
    if constexpr (!kShared0) {                                                              \
      chunk_step<C, kPair>(s, load_vectors(s_qk0[wave], kq), s_v0[wave][8 * (C) + rsub],      \
                           s_v0[wave][8 * (C) + 4 + rsub], s_o[0], s_db0[wave][0],            \
                           s_db0[wave][1], kq, r, dst[0], lane_bytes);                      \
      if ((C) == 0 && Width > 1) lds_barrier();                                             \
    }                                                                                       \
    _Pragma("unroll") for (int t = kShared0 ? 0 : 1; t < Width; ++t) {                      \
      chunk_step<C, kPair>(s, load_vectors(s_qkt[t], kq), s_vt[t][r], s_vt[t][r + kPair],     \
                           s_o[t], s_dbt[t][0], s_dbt[t][1], kq, r, dst[t], lane_bytes);    \
    }                                                                                       \
  }
  if constexpr (kShared0) lds_barrier();  // every token staged
  if constexpr (kConvSplit) {
    if (tid >= 2 * kDim && tid < 3 * kDim) {
#pragma unroll
      for (int k = 0; k < kCols; ++k)
        p.conv_state[cs3_at + min(k, p.conv_len - 1) * p.conv_len_stride] = v_new_split[k];
    }
    if (p.group > 1 && tid == 0)
      arrived = count_in(&g_conv_ticket[static_cast<int64_t>(slot[0]) * p.num_k_heads + key_head],
                         p.group);
  }
  LD_CHUNK(0)
  if constexpr (kChunks > 1) LD_CHUNK(1)
  if constexpr (kChunks > 2) {
    LD_CHUNK(2)
    LD_CHUNK(3)
  }
#undef LD_CHUNK
  if constexpr (kLate) stage_epi();  // read after the barrier below
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
      orow[v] = f32_to_bf16(((raw[e] * rstd) * s_w[v]) * s_sg[wave][v]);
    }
  }

  // ---- conv variant: the only workgroup of its k-head (HV == H), or the one that counted
  // in last (all HV/H of the k-head group had read the q/k conv state before it), writes the
  // shifted q/k conv state (its count_in already returned the count to zero) ----
  if constexpr (Conv) {
    if (p.group == 1 || s_arrived == static_cast<uint32_t>(p.group - 1)) {
      const int64_t slot_at = static_cast<int64_t>(slot[0]) * p.conv_slot;
      if constexpr (Packed) {  // each wave its 64 q or k channels, one 16-byte piece per lane
        if (Waves == kWaves || wave_s < 4)
          *reinterpret_cast<u32x4*>(p.conv_state + slot_at +
                                    static_cast<int64_t>(pk_qk0) * p.conv_len + 8 * pk_piece) =
              s_cpk[wave][0][pk_piece];
      } else {
        for (int c = tid; c < 2 * kDim; c += kBlock) {
          const int ch = c < kDim ? q_col + c : k_col + (c - kDim);
          const int64_t at = slot_at + ch * p.conv_dim_stride;
          for (int j = 0; j < p.conv_len; ++j)
            p.conv_state[at + j * p.conv_len_stride] = s_conv_new[c][j];
        }
      }
    }
  }
}


// Launch shape of one kernel family: cache policy bits of the state loads and stores, waves
// per workgroup, and whether a workgroup runs alone on its CU.  Solo workgroups ask for
// kSoloLds bytes of dynamic LDS (they use none of it): more than half of the CU's 160 KiB,
// so a second workgroup never fits beside one, plus the kernel's static LDS (under 16 KiB),
// within the 160 KiB a workgroup may hold.
template <int LoadPol, int StorePol, int Waves, bool Solo = false>
struct Shape {
  static constexpr int kLoad = LoadPol;
  static constexpr int kStore = StorePol;
  static constexpr int kWaveCount = Waves;
  static constexpr bool kSolo = Solo;
};
#ifndef LD_SOLO_LDS_BYTES
#define LD_SOLO_LDS_BYTES (96 * 1024)
#endif
constexpr size_t kSoloLds = LD_SOLO_LDS_BYTES;
constexpr size_t kLdsPerWorkgroup = 160 * 1024;

// Whether `kernel`'s static LDS plus `dynamic` bytes fit a workgroup (checked once per kernel
// on the host: an oversized request is not a launch error but a queue abort).
template <typename Kernel>
bool lds_fits(Kernel kernel, size_t dynamic) {
  hipFuncAttributes attr{};
  return hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel)) == hipSuccess &&
         attr.sharedSizeBytes + dynamic <= kLdsPerWorkgroup;
}

template <typename S, int Width, int ConvCols, bool Packed, bool DtBf16, bool WBf16>
int launch_one(const DecodeParams& p, uint32_t blocks, hipStream_t stream) {
  constexpr int LP = S::kLoad, SP = S::kStore, W = S::kWaveCount;
  const auto kernel = gdn_decode_kernel<DtBf16, WBf16, LP, SP, Width, ConvCols, W, Packed>;
  // The declared LDS plus the one-workgroup-per-CU request must fit a workgroup: checked for
  // every solo shape the library instantiates when it is built.
  static_assert(!S::kSolo ||
                    DecodeLds<Width, ConvCols, W, Packed>::kBytes + kSoloLds <= kLdsPerWorkgroup,
                "decode kernel: its LDS plus the one-workgroup-per-CU request exceed a "
                "workgroup's 160 KiB");
  if constexpr (S::kSolo) {
    // Backstop for LDS the compiler adds beyond the declared struct (a private aggregate it
    // places in LDS): read from the built kernel once.
    static const bool fits = lds_fits(kernel, kSoloLds);
    if (!fits)
      return fail(LD_ERR_LAUNCH, "decode kernel: static LDS plus the one-workgroup-per-CU "
                                 "request exceed a workgroup's 160 KiB");
  }
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(64 * W), S::kSolo ? kSoloLds : 0, stream,
                     p.indices, p.cu, p.accepted, p.num_v_heads, p);
  return LD_OK;
}

template <typename S, int Width, int ConvCols, bool Packed = false>
int launch_kernel(const DecodeParams& p, bool dt_bf16, bool w_bf16, uint32_t blocks,
                  hipStream_t stream) {
  return dt_bf16 ? (w_bf16 ? launch_one<S, Width, ConvCols, Packed, true, true>(p, blocks, stream)
                           : launch_one<S, Width, ConvCols, Packed, true, false>(p, blocks, stream))
                 : (w_bf16 ? launch_one<S, Width, ConvCols, Packed, false, true>(p, blocks, stream)
                           : launch_one<S, Width, ConvCols, Packed, false, false>(p, blocks, stream));
}

// One cache policy: the shapes of the single-token step (One), of verify steps (Verify), and
// of the conv-fused single-token (ConvOne) and verify (ConvVerify) steps.  A conv-fused
// verify keeps one workgroup per CU: at the register budget of two (64 VGPRs) it spills
// 108-128 bytes per lane to scratch.
template <typename One, typename Verify, typename ConvOne, typename ConvVerify>
int launch_decode(const DecodeParams& p, bool conv, bool dt_bf16, bool w_bf16,
                  uint32_t blocks, hipStream_t stream) {
  // a state of more than 4 columns runs its conv before the tile loads, with 4 waves
  using ConvLong = Shape<ConvOne::kLoad, ConvOne::kStore, kWaves>;
  if (conv) {
    switch (p.width) {
      case 1:  // conv state of 3..4 columns (the usual width - 1 = 3), or up to 8
        if (p.conv_len <= 4 && p.conv_packed)  // dense dim-first pool: 16-byte pieces
          return launch_kernel<ConvOne, 1, 4, true>(p, dt_bf16, w_bf16, blocks, stream);
        if (p.conv_len <= 4) return launch_kernel<ConvOne, 1, 4>(p, dt_bf16, w_bf16, blocks, stream);
        return launch_kernel<ConvLong, 1, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream);
      case 2: return launch_kernel<ConvVerify, 2, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream);
      case 3: return launch_kernel<ConvVerify, 3, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream);
      default: return launch_kernel<ConvVerify, 4, kMaxConvLen>(p, dt_bf16, w_bf16, blocks, stream);
    }
  }
  switch (p.width) {
    case 1: return launch_kernel<One, 1, 0>(p, dt_bf16, w_bf16, blocks, stream);
    case 2: return launch_kernel<Verify, 2, 0>(p, dt_bf16, w_bf16, blocks, stream);
    case 3: return launch_kernel<Verify, 3, 0>(p, dt_bf16, w_bf16, blocks, stream);
    default: return launch_kernel<Verify, 4, 0>(p, dt_bf16, w_bf16, blocks, stream);
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
  // Measured on MI355X (B=32 and B=128 single-token steps, B=64 4-token verify, B=32 and
  // B=128 conv-fused steps; hot = the same slots every step, cold = slot sets rotated
  // through a pool far beyond the 256 MB Infinity Cache):
  //   one token, keep:   4 waves, plain loads and stores (B=32 hot 19.9 us; 16 waves with
  //                      the same hints 20.2, the stream kernel 20.9).
  //   verify, keep:      16 waves, plain loads, non-temporal stores, one workgroup per CU
  //                      (B=64, T=4: 98.7-101 us hot, 120.8 cold; two per CU 98.8 and
  //                      124.4; 4 waves 105.1 and 138.9).
  //   conv-fused, keep:  one token 4 waves, plain loads and stores (21.3 us hot); verify as
  //                      the verify above (102-105 us hot).
  //   stream, all:       16 waves (verify steps one workgroup per CU), non-temporal
  //                      system-scope loads and stores (cold: B=128 single token 88.8 us =
  //                      6.04 TB/s, B=32 24.6; conv-fused 90.6 and 25.3; verify 112.4,
  //                      conv-fused verify 114.7; 4-wave forms 10-20% slower).
  const uint32_t n = static_cast<uint32_t>(blocks);
  int rc;
  if (a.cache_policy == LD_CACHE_STREAM)
    rc = launch_decode<Shape<kPolNTSys, kPolNTSys, 16>, Shape<kPolNTSys, kPolNTSys, 16, true>,
                       Shape<kPolNTSys, kPolNTSys, 16>, Shape<kPolNTSys, kPolNTSys, 16, true>>(
        p, conv, dt_bf16, w_bf16, n, s);
  else
    rc = launch_decode<Shape<kPolPlain, kPolPlain, kWaves>, Shape<kPolPlain, kPolNT, 16, true>,
                       Shape<kPolPlain, kPolPlain, kWaves>, Shape<kPolPlain, kPolNT, 16, true>>(
        p, conv, dt_bf16, w_bf16, n, s);
  if (rc != LD_OK) return rc;
  return check_launch(conv ? "ld_gdn_decode_conv" : "ld_gdn_decode");
}

}  // namespace
}  // namespace ld

extern "C" int ld_gdn_decode(const ld_gdn_decode_args* args, void* stream) {
  using namespace ld;
  DecodeParams p{};
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
  DecodeParams p{};
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
  // Packed conv-state access: dim-first dense channels and columns, every 64-channel run of
  // every slot 16-byte aligned (a run starts 128 * len bytes after the slot's start).
  p.conv_packed = conv->state_len_stride == 1 && conv->state_dim_stride == conv->state_len &&
                  (reinterpret_cast<uintptr_t>(conv->state) & 15) == 0 &&
                  (conv->state_slot_stride * 2) % 16 == 0;
  return launch(*args, p, blocks, true, stream);
}
