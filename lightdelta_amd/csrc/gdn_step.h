// The per-token step shared by the decode / verify kernel (gdn_decode.hip) and the
// token-serial prefill (prefill_serial.hip).
//
// Lane layout of a 128 x 128 fp32 state tile: the 16 lanes of a DPP row span one 512-byte K
// row, lane kq holding k = 4kq .. 4kq+3 and 64+4kq .. 64+4kq+3 (pieces 2i and 2i+1, 16 bytes
// each); the 4 DPP rows of a wave take 4 consecutive V rows; a lane's pieces 2i, 2i+1 lie
// PairRows rows below its pieces 2i-2, 2i-1.  The token-serial prefill uses PairRows = 4
// (wave w owning the contiguous rows of its share); the decode uses PairRows = 4 * waves, so
// that a piece pair of all waves of the workgroup covers one contiguous block of the tile
// (see gdn_decode.hip).  A token is staged once (q^, k^ in the lane layout, v of the lane's
// rows, decay and beta) and applied to the tile chunk by chunk (chunk_step), with the row
// sums S k^ and S q^ by a 4-step DPP butterfly, so every lane holds the full sums.  Which lane
// holds which row does not change any row's arithmetic.
#pragma once

#include "gdn_common.h"

namespace ld {
namespace {

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
// is V row PairRows*(j/2) further down (512 bytes per row) and, for odd j, 64 floats further
// along K.
template <int PairRows = 4>
__device__ __forceinline__ constexpr uint32_t tile_piece_bytes(int j) {
  return static_cast<uint32_t>(j >> 1) * PairRows * kDim * 4u + static_cast<uint32_t>(j & 1) * 256u;
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

// Where chunk_step puts a chunk's updated pieces: nowhere (the prefill keeps the tile in
// registers), or a 64 KiB tile with cache policy Pol.  Plain and non-temporal stores go
// through the tile's address; policies with scope bits through a buffer resource over it.
// The store is unconditional, so the compiler's count of memory operations in flight stays
// exact and later chunks wait for their own loads only: a token without a destination (a
// padding slot, a token past the request's last) writes the sink tile (pointer stores), or a
// resource over 0 bytes, whose stores the hardware drops.
struct NoStore {
  __device__ __forceinline__ void store(uint32_t, f32x4) const {}
};

template <int Pol>
struct TileStore {
  static constexpr bool kBuffer = (Pol & ~kPolNT) != 0;
  char* tile;                    // pointer stores
  __amdgpu_buffer_rsrc_t rsrc;   // buffer stores
  __device__ __forceinline__ void set(char* destination, bool stored, char* sink) {
    if constexpr (kBuffer)
      rsrc = buffer_rsrc(destination, stored ? kTileBytes : 0);
    else
      tile = stored ? destination : sink;
  }
  __device__ __forceinline__ void store(uint32_t offset, f32x4 v) const {
    if constexpr (kBuffer)
      buffer_store16<Pol>(v, rsrc, offset);
    else if constexpr (Pol == kPolNT)
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(tile + offset));
    else
      *reinterpret_cast<f32x4*>(tile + offset) = v;
  }
};

// Piece of a source tile at `offset`, loaded with cache policy Pol (as TileStore).
template <int Pol>
__device__ __forceinline__ f32x4 load_tile_piece(const char* tile, uint32_t offset) {
  if constexpr ((Pol & ~kPolNT) != 0)
    return buffer_load16<Pol>(buffer_rsrc(tile, kTileBytes), offset);
  else if constexpr (Pol == kPolNT)
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(tile + offset));
  else
    return *reinterpret_cast<const f32x4*>(tile + offset);
}

// One token on chunk C of the lane's slice (pieces 4C..4C+3 = V rows row0 and
// row0 + PairRows, whose v values are v0 and v1):
//   S <- decay*S ; delta = (v - S k^) * beta ; S += delta k^ ; raw = bf16(S q^)
// The updated pieces go to `dst` and the two rows' raw outputs to LDS (one lane per row).
// RoundOut = false leaves S q^ unrounded there, for a reader that rounds it to bf16 itself
// (the same bits, and no rounding in the token's chain).
template <int C, int PairRows = 4, int N = kPieces, bool RoundOut = true, typename Dst>
__device__ __forceinline__ void chunk_step(f32x4 (&s)[N], const Vectors& x, float v0,
                                           float v1, float* o, float decay, float beta,
                                           int kq, int row0, const Dst& dst,
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
#pragma unroll
  for (int j = j0; j < j0 + 4; ++j) dst.store(lane_bytes + tile_piece_bytes<PairRows>(j), s[j]);
  float out0 = dot8(s[j0], s[j0 + 1], x.q0, x.q1);
  float out1 = dot8(s[j0 + 2], s[j0 + 3], x.q0, x.q1);
  row_sum2(out0, out1);
  if (kq == 0) {
    o[row0] = RoundOut ? round_bf16(out0) : out0;
    o[row0 + PairRows] = RoundOut ? round_bf16(out1) : out1;
  }
}

// Uses a wave-uniform value (in SGPRs) at this point of the program, so its computation (a
// kernel-argument or metadata load) cannot be sunk past later branches.  Input-only: the
// value itself, and for pointers their global address space, stay visible to the compiler.

// Keeps the compiler from moving LDS accesses across this point: a wave's packed conv runs are
// written as 16-byte pieces and read back as 2-byte columns (or the reverse), which type-based
// alias analysis would otherwise let it reorder.  The hardware runs a wave's LDS operations in
// program order, so no wait is needed.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// Waits for this wave's LDS traffic, then joins the workgroup barrier.  Global loads that
// are still in flight stay in flight (a __syncthreads() fence would drain them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace
}  // namespace ld
