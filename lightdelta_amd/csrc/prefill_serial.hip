// Token-serial prefill for gfx950: the sequence's tokens run in order with a block of state
// rows in registers for the whole prompt (read once, from the slot or as zeros; written
// once, to the slot).  The per-token arithmetic is the decode kernel's (stage_token,
// chunk_step), so a prefill of n tokens gives bit for bit the states and outputs of n
// single-token decode steps.  Rows of the state evolve independently (row v needs only
// v[v], k, q and the gates), so a head's 128 rows may be split over several workgroups.
//   gdn_prefill_kernel: one workgroup per (sequence, head), 32 rows per wave; each token is
//   staged once per workgroup (by one wave, a group of 4 tokens ahead, through LDS), and
//   the raw outputs of a group of 4 tokens collect in LDS; after one barrier per group,
//   wave w runs the gated-RMSNorm epilogue of the group's token w.  Four waves per SIMD:
//   the tile and a token's vectors fit 128 VGPRs.
//   gdn_prefill_rows_kernel (few sequences): a head's rows over 2 or 4 workgroups, 8 or 16
//   rows per wave, for a shorter per-token chain and more of the GPU; every wave writes its
//   rows' raw outputs (rounded to bf16, the reference's rounding point before the norm) to
//   `out`, and prefill_norm_kernel applies the gated RMSNorm in place afterwards, with the
//   epilogue's arithmetic.
//
// Also here: the gated-RMSNorm pass over raw outputs (prefill_norm_kernel, or with 16-byte
// accesses prefill_norm_wide_kernel; used by the row-split kernels and the chunked form) and
// the prefill entry points of the C ABI, which choose between this form and the chunked one
// (prefill_chunked.hip).
#include <mutex>

#include "gdn_step.h"

namespace ld {
namespace {

constexpr int kPrefillGroup = 4;

// One workgroup per (sequence, v-head), wave w holding rows 32w .. 32w + 31.  Tokens go in
// groups of 4: before the group's barrier, wave w stages token w of the next group (q^ and
// k^ in the lane layout, decay, beta: stage_token) into double-buffered LDS, and every wave
// reads a token's staging from there, so each token is staged once per workgroup and off
// the per-token chain.  A wave's v values come one token ahead.
template <bool DtBf16, bool WBf16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void gdn_prefill_kernel(const DecodeParams args) {
  constexpr int kWaveRows = 32;    // state rows per wave
  constexpr int kTilePieces = 16;  // 16-byte pieces per lane
  const DecodeParams& p = args;
  const int tile = blockIdx.x;
  const int sequence = tile / p.num_v_heads;
  const int head = tile - sequence * p.num_v_heads;
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
  const int wave_row0 = wave * kWaveRows;  // first row of the wave
  const int row_base = wave_row0 + rsub;
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;

  __shared__ float s_v[kWaves][kWaveRows];
  __shared__ float s_o[2][kPrefillGroup][kDim];
  __shared__ f32x4 s_qk[2][kPrefillGroup][2][kDim / 4];  // [buffer][token][q^ | k^][piece]
  __shared__ float s_db[2][kPrefillGroup][2];             // [buffer][token][decay | beta]
  __shared__ float s_w[kDim];                              // the norm weight

  // uniform: kept in an SGPR (a bf16 load would leave it in a VGPR)
  const float dt_bias = __int_as_float(
      __builtin_amdgcn_readfirstlane(__float_as_int(load_param(p.dt_bias, head, DtBf16))));
  const float a_log = p.a_log[head];
  if (wave == 0) {  // read by every wave's epilogue, after the first barrier
#pragma unroll
    for (int e = 0; e < 2; ++e) s_w[2 * lane + e] = load_param(p.norm_weight, 2 * lane + e, WBf16);
  }

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

  // Inputs, addressed from the uniform row start with 32-bit lane offsets; tokens past the
  // end read the last one (an unconditional fetch needs no merge of old and new values).
  const int last = eos - 1;
  const uint32_t q_bytes = static_cast<uint32_t>(q_col + kq * 4) * 2u;
  const uint32_t k_bytes = static_cast<uint32_t>(k_col + kq * 4) * 2u;
  const uint32_t v_bytes = static_cast<uint32_t>(v_col + wave_row0 + (lane & (kWaveRows - 1))) * 2u;
  auto row_of = [&](int64_t token) __attribute__((always_inline)) {
    return reinterpret_cast<const char*>(p.qkv + token * p.qkv_row);
  };
  auto u16 = [](const char* row, uint32_t offset) __attribute__((always_inline)) {
    return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(row + offset));
  };
  // load_token's values of a token to stage (its v is not needed there)
  auto fetch = [&](int64_t token) __attribute__((always_inline)) {
    const char* row = row_of(token);
    TokenIn in;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t off = e * 128u;
      in.q[2 * e] = u16(row, q_bytes + off) | (u16(row, q_bytes + off + 2) << 16);
      in.q[2 * e + 1] = u16(row, q_bytes + off + 4) | (u16(row, q_bytes + off + 6) << 16);
      in.k[2 * e] = u16(row, k_bytes + off) | (u16(row, k_bytes + off + 2) << 16);
      in.k[2 * e + 1] = u16(row, k_bytes + off + 4) | (u16(row, k_bytes + off + 6) << 16);
    }
    in.v = 0;
    in.a = p.a[token * p.a_row + head];
    in.b = p.b[token * p.b_row + head];
    return in;
  };
  // stage_token's results into buffer b, token i (lanes of DPP row 0 write the pieces)
  auto stage = [&](const TokenIn& in, int b, int i) __attribute__((always_inline)) {
    const Staged x = stage_token(in, a_log, dt_bias, p.scale);
    if (rsub == 0) {
      s_qk[b][i][0][kq] = x.q0;
      s_qk[b][i][0][16 + kq] = x.q1;
      s_qk[b][i][1][kq] = x.k0;
      s_qk[b][i][1][16 + kq] = x.k1;
    }
    if (lane == 0) {
      s_db[b][i][0] = x.decay;
      s_db[b][i][1] = x.beta;
    }
  };

  // the first group's staging (wave w: token bos + w) and the first token's v
  int buf = 0;
  uint16_t v_next = 0;
  if (bos < eos) {
    stage(fetch(min(bos + wave, last)), 0, wave);
    v_next = static_cast<uint16_t>(u16(row_of(bos), v_bytes));
  }
  lds_barrier();

  // One token: its v values to the wave's LDS row (read back by other lanes of the wave:
  // a wave's LDS operations run in program order, so only the compiler must not reorder
  // them), the next token's v fetched, the staged vectors read, the tile updated; its raw
  // outputs (unrounded) go to the group's slot i.
  auto token_step = [&](int t, int i) __attribute__((always_inline)) {
    if (lane < kWaveRows) s_v[wave][lane] = bf16_to_f32(v_next);
    v_next = static_cast<uint16_t>(u16(row_of(min(t + 1, last)), v_bytes));
    asm volatile("" ::: "memory");
    const Vectors vec = load_vectors(s_qk[buf][i], kq);
    const float decay = s_db[buf][i][0];
    const float beta = s_db[buf][i][1];
#define LD_PREFILL_CHUNK(C)                                                                    \
  chunk_step<C, 4, kTilePieces, false>(s, vec, s_v[wave][8 * (C) + rsub],                     \
                                       s_v[wave][8 * (C) + 4 + rsub], s_o[buf][i], decay,    \
                                       beta, kq, row_base + 8 * (C), NoStore{}, lane_bytes);
    LD_PREFILL_CHUNK(0)
    LD_PREFILL_CHUNK(1)
    LD_PREFILL_CHUNK(2)
    LD_PREFILL_CHUNK(3)
#undef LD_PREFILL_CHUNK
    asm volatile("" ::: "memory");
  };
  // A group of tokens: the next group's token `wave` fetched first, the tokens, this
  // group's gate of token `wave` fetched, the staging of that next token (into the other
  // buffer, last read before the previous barrier), one barrier, then the gated RMSNorm
  // epilogue of the group's token `wave`.
  auto group = [&](int g0, auto&& tokens) __attribute__((always_inline)) {
    const TokenIn next_in = fetch(min(g0 + kPrefillGroup + wave, last));
    tokens();
    uint16_t gh[2];
    {
      const int64_t etoken = min(g0 + wave, last);
#pragma unroll
      for (int e = 0; e < 2; ++e) gh[e] = p.gate[etoken * p.gate_row + head * kDim + 2 * lane + e];
    }
    stage(next_in, buf ^ 1, wave);
    lds_barrier();  // the group's raw outputs and the next group's staging are complete
    if (g0 + wave < eos) {
      float raw[2];
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        raw[e] = round_bf16(s_o[buf][wave][2 * lane + e]);
        ss = fmaf(raw[e], raw[e], ss);
      }
      ss = wave_sum(ss);
      const float rstd = fast_rsqrt(ss / static_cast<float>(kDim) + p.eps);
      uint16_t* orow_ptr = p.out + (static_cast<int64_t>(g0 + wave) * p.num_v_heads + head) * kDim;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        orow_ptr[2 * lane + e] =
            f32_to_bf16(((raw[e] * rstd) * s_w[2 * lane + e]) * silu(bf16_to_f32(gh[e])));
    }
    buf ^= 1;
  };
  // Whole groups first, then the partial last group (as alternatives inside one loop the two
  // paths would need different register assignments of the tile).
  int g0 = bos;
  for (; g0 + kPrefillGroup <= eos; g0 += kPrefillGroup)
    group(g0, [&]() __attribute__((always_inline)) {
#pragma unroll 1  // unrolled, the tokens' fetches move up and spill registers
      for (int i = 0; i < kPrefillGroup; ++i) token_step(g0 + i, i);
    });
  if (g0 < eos)
    group(g0, [&]() __attribute__((always_inline)) {
      for (int i = 0; g0 + i < eos; ++i) token_step(g0 + i, i);
    });

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
    chunk_step<0, 4, kTilePieces, false>(s, vec, vv[0], vv[1], o, now.decay, now.beta, kq, rsub,
                                         NoStore{}, lane_bytes);
    if constexpr (Chunks == 2)
      chunk_step<1, 4, kTilePieces, false>(s, vec, vv[2], vv[3], o, now.decay, now.beta, kq,
                                           rsub + 8, NoStore{}, lane_bytes);
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

// The same norm with 16-byte accesses, for `gate` rows at 16-byte boundaries (the usual
// layout; `out` is contiguous): lane (r, c) of a wave holds elements 8c .. 8c + 7 of item
// 4j + r, j < kNormItems / 4.  The sum of squares runs in wave_sum's order (a lane's four
// pairs as the four lanes of a quad would sum them, then the 16 lanes of the DPP row as
// wave_sum's remaining levels), so the results are those of prefill_norm_kernel, bit for bit.
template <bool WBf16>
__global__ __launch_bounds__(kThreads) void prefill_norm_wide_kernel(const DecodeParams p,
                                                                     int num_sequences) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4;
  const int c = lane & 15;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6)) *
                        kNormItems;
  const int64_t lo = static_cast<int64_t>(p.cu[0]) * p.num_v_heads;
  const int64_t hi = static_cast<int64_t>(p.cu[num_sequences]) * p.num_v_heads;
  if (first >= hi || first + kNormItems <= lo) return;  // no row of this wave (or none at all)
  constexpr int kLoads = kNormItems / 4;
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = load_param(p.norm_weight, 8 * c + e, WBf16);
  u32x4 raw_bits[kLoads], gate_bits[kLoads];
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int64_t item = min(max(first + 4 * j + r, lo), hi - 1);  // in range; unused ones not stored
    const int64_t token = item / p.num_v_heads;
    const int head = static_cast<int>(item - token * p.num_v_heads);
    raw_bits[j] = *reinterpret_cast<const u32x4*>(p.out + item * kDim + 8 * c);
    gate_bits[j] = *reinterpret_cast<const u32x4*>(p.gate + token * p.gate_row + head * kDim + 8 * c);
  }
#pragma unroll
  for (int j = 0; j < kLoads; ++j) {
    const int64_t item = first + 4 * j + r;
    float raw[8], gate[8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      raw[2 * m] = __builtin_bit_cast(float, raw_bits[j][m] << 16);
      raw[2 * m + 1] = __builtin_bit_cast(float, raw_bits[j][m] & 0xffff0000u);
      gate[2 * m] = __builtin_bit_cast(float, gate_bits[j][m] << 16);
      gate[2 * m + 1] = __builtin_bit_cast(float, gate_bits[j][m] & 0xffff0000u);
    }
    float pq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) pq[m] = fmaf(raw[2 * m + 1], raw[2 * m + 1], raw[2 * m] * raw[2 * m]);
    float ss = (pq[0] + pq[1]) + (pq[2] + pq[3]);
    ss += dpp<kDppQuadXor1>(ss);
    ss += dpp<kDppQuadXor2>(ss);
    ss += dpp<kDppRowHalfMirror>(ss);
    ss += dpp<kDppRowMirror>(ss);
    const float rstd = fast_rsqrt(ss / static_cast<float>(kDim) + p.eps);
    uint32_t y[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint16_t y0 = f32_to_bf16(((raw[2 * m] * rstd) * w[2 * m]) * silu(gate[2 * m]));
      const uint16_t y1 = f32_to_bf16(((raw[2 * m + 1] * rstd) * w[2 * m + 1]) * silu(gate[2 * m + 1]));
      y[m] = y0 | (static_cast<uint32_t>(y1) << 16);
    }
    if (item >= lo && item < hi)
      *reinterpret_cast<u32x4*>(p.out + item * kDim + 8 * c) = u32x4{y[0], y[1], y[2], y[3]};
  }
}

// The prefill of ld_gdn_prefill, with the chunked form's workspace passed separately
// (`workspace`, `workspace_bytes`: the caller's, or the static scratch below).
int prefill(const ld_gdn_prefill_args& a, void* workspace, int64_t workspace_bytes,
            void* stream) {
  if (a.num_sequences < 0) return fail(LD_ERR_INVALID_ARGUMENT, "num_sequences must be >= 0");
  if (a.algorithm < LD_PREFILL_AUTO || a.algorithm > LD_PREFILL_CHUNKED_32)
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
  const bool ws_fits = workspace != nullptr && workspace_bytes >= ws_need;
  const bool named_chunked =
      a.algorithm == LD_PREFILL_CHUNKED || a.algorithm == LD_PREFILL_CHUNKED_32;
  if (named_chunked && !ws_fits)
    return fail(LD_ERR_INVALID_ARGUMENT, "chunked prefill: workspace missing or too small");
  // tokens per chunk of the chunked form, 0 for the token-serial one
  const int chunk_tokens =
      a.algorithm == LD_PREFILL_CHUNKED      ? 64
      : a.algorithm == LD_PREFILL_CHUNKED_32 ? 32
      : a.algorithm == LD_PREFILL_AUTO && ws_fits
          ? prefill_auto_chunk_tokens(a.num_tokens, a.num_sequences, a.num_v_heads)
          : 0;
  const bool chunked = chunk_tokens != 0;
  if (chunked) {
    const int rc = launch_prefill_chunked(p, a.num_sequences, a.num_tokens, dt_bf16,
                                          chunk_tokens, workspace, s);
    if (rc != LD_OK) return rc;
  }
  // Token-serial: split a head's rows over more workgroups when (sequence, head) tiles alone
  // would leave the GPU short of work (1024 tiles fill 256 CUs at 4 per CU).
  const int chunks = chunked ? 0 : (tiles >= 256 ? 4 : (tiles >= 128 ? 2 : 1));
  const uint32_t grid = chunks > 0 ? static_cast<uint32_t>(tiles * (4 / chunks)) : 0u;
#define LD_PREFILL_LAUNCH()                                                                  \
  hipLaunchKernelGGL(dt_bf16 ? (w_bf16 ? gdn_prefill_kernel<true, true>                      \
                                       : gdn_prefill_kernel<true, false>)                    \
                             : (w_bf16 ? gdn_prefill_kernel<false, true>                     \
                                       : gdn_prefill_kernel<false, false>),                  \
                     dim3(grid), dim3(kThreads), 0, s, p)
#define LD_PREFILL_ROWS_LAUNCH(C)                                                            \
  hipLaunchKernelGGL(dt_bf16 ? (w_bf16 ? gdn_prefill_rows_kernel<true, true, C>              \
                                       : gdn_prefill_rows_kernel<true, false, C>)            \
                             : (w_bf16 ? gdn_prefill_rows_kernel<false, true, C>             \
                                       : gdn_prefill_rows_kernel<false, false, C>),          \
                     dim3(grid), dim3(kThreads), 0, s, p)
  if (chunks == 4) {
    LD_PREFILL_LAUNCH();
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
      const bool wide = (reinterpret_cast<uintptr_t>(a.gate) & 15) == 0 && (a.gate_row_stride & 7) == 0 &&
                        (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
#define LD_NORM_LAUNCH(W, P)                                                                  \
  hipLaunchKernelGGL((prefill_norm_kernel<W, P>), dim3(norm_grid), dim3(kThreads), 0, s, p,  \
                     a.num_sequences)
      if (wide) {
        hipLaunchKernelGGL(w_bf16 ? prefill_norm_wide_kernel<true> : prefill_norm_wide_kernel<false>,
                           dim3(norm_grid), dim3(kThreads), 0, s, p, a.num_sequences);
      } else if (w_bf16) {
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

// ---- the allocation-free prefill: the chunked workspace in a static device array ----------
//
// `scratch` is this library's copy of the chunked form's workspace for ld_gdn_prefill_static,
// one per GPU the library is loaded on, held until the process ends.  In host code its name
// stands for a host-side shadow, not device memory: kernels get the address that
// hipGetSymbolAddress returns for the current device (static_scratch), never `scratch`
// itself.  The chunked form writes every byte of the workspace it reads later in the same
// call (chunk index, then the per-chunk records), so nothing in it has to start at zero and
// the previous call's contents do no harm; two calls that overlap in time on one GPU share it
// and race.
constexpr int64_t kStaticScratchBytes = int64_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices];  // per device ordinal, set on the device's first call

// Device address of the current device's `scratch`, looked up once per device (with that
// device current) and kept.  The stream must belong to the current device.
int static_scratch(void* stream, void** address) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return launch_failed("ld_gdn_prefill_static: hipGetDevice", err);
  if (device < 0 || device >= kMaxDevices)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_prefill_static: device ordinal out of range");
  hipDevice_t stream_device = -1;
  err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_device);
  if (err != hipSuccess) return launch_failed("ld_gdn_prefill_static: hipStreamGetDevice", err);
  if (stream_device != device)
    return fail(LD_ERR_INVALID_ARGUMENT,
                "ld_gdn_prefill_static: the stream belongs to another device than the current "
                "one");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* found = nullptr;
    err = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (err != hipSuccess || found == nullptr)
      return launch_failed("ld_gdn_prefill_static: hipGetSymbolAddress(scratch)", err);
    g_scratch_address[device] = found;
  }
  *address = g_scratch_address[device];
  return LD_OK;
}

}  // namespace
}  // namespace ld

extern "C" int ld_gdn_prefill(const ld_gdn_prefill_args* args, void* stream) {
  using namespace ld;
  if (args == nullptr) return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_prefill: args is NULL");
  return prefill(*args, args->workspace, args->workspace_bytes, stream);
}

extern "C" int ld_gdn_prefill_static(const ld_gdn_prefill_args* args, void* stream) {
  using namespace ld;
  if (args == nullptr)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_prefill_static: args is NULL");
  const ld_gdn_prefill_args& a = *args;
  if (a.workspace != nullptr || a.workspace_bytes != 0)
    return fail(LD_ERR_INVALID_ARGUMENT,
                "ld_gdn_prefill_static: workspace must be NULL (the static scratch is used)");
  if (a.num_tokens < 0 || a.num_sequences < 0 || a.num_v_heads <= 0)
    return prefill(a, nullptr, 0, stream);  // rejected there with its message
  const int64_t need = prefill_chunked_workspace_bytes(a.num_tokens, a.num_sequences,
                                                       a.num_v_heads);
  const bool named_chunked =
      a.algorithm == LD_PREFILL_CHUNKED || a.algorithm == LD_PREFILL_CHUNKED_32;
  const bool wants_chunked =
      named_chunked ||
      (a.algorithm == LD_PREFILL_AUTO &&
       prefill_auto_chunk_tokens(a.num_tokens, a.num_sequences, a.num_v_heads) != 0);
  if (named_chunked && need > kStaticScratchBytes)
    return fail(LD_ERR_INVALID_ARGUMENT,
                "ld_gdn_prefill_static: the chunked form needs more workspace than the static "
                "scratch holds (LD_PREFILL_STATIC_SCRATCH_BYTES); use LD_PREFILL_TOKEN_SERIAL, "
                "fewer tokens, or ld_gdn_prefill with a workspace");
  if (a.num_sequences == 0 || !wants_chunked || need > kStaticScratchBytes)
    return prefill(a, nullptr, 0, stream);  // token-serial: no scratch
  void* address = nullptr;
  const int rc = static_scratch(stream, &address);
  if (rc != LD_OK) return rc;
  return prefill(a, address, kStaticScratchBytes, stream);
}

extern "C" int64_t ld_gdn_prefill_workspace_bytes(int64_t num_tokens, int32_t num_sequences,
                                                  int32_t num_v_heads) {
  if (num_tokens < 0 || num_sequences < 0 || num_v_heads < 0) return 0;
  return ld::prefill_chunked_workspace_bytes(num_tokens, num_sequences, num_v_heads);
}

extern "C" int32_t ld_gdn_prefill_auto_chunked(int64_t num_tokens, int32_t num_sequences,
                                               int32_t num_v_heads) {
  return ld::prefill_auto_chunk_tokens(num_tokens, num_sequences, num_v_heads);
}
