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
//     i.e. eight whole 128-byte lines, and a lane keeps 8 V rows x 8 K values = 64 fp32
//     (16 x 128-bit loads) of the tile in VGPRs for the whole step.
//   * All 16 tile loads are issued before any arithmetic; the per-row dot products
//     S k^ and S q^ are 8 products per lane followed by a DPP reduce-scatter inside the
//     16-lane row (row_mirror, row_half_mirror, quad_perm), so no LDS round trip and no
//     cross-row lane traffic is needed for the contractions.
//   * T <= 4 tokens (MTP verify) reuse the registers: 1 tile read, T tile writes.
#include "common.h"

namespace ld {
namespace {

constexpr int kDim = LD_HEAD_DIM;
constexpr int kThreads = 256;
constexpr int kRowsPerWave = 32;
constexpr int kRowGroups = 8;  // V rows per lane
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
};

__device__ __forceinline__ float load_param(const void* p, int i, bool bf16) {
  return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i])
              : static_cast<const float*>(p)[i];
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// softplus with the threshold torch's F.softplus uses (beta=1, threshold=20).
__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// Reduce-scatter of 8 per-row partial sums over the 16 lanes of a DPP row: each step pairs
// lanes that differ in one bit of kq (bit 3 via row_mirror, bit 2 via row_half_mirror,
// bits 1 and 0 via quad_perm); the lane with the bit clear keeps the lower half of its list,
// the partner the upper half.  Lane kq ends with the full sum for row group kq >> 1.
__device__ __forceinline__ float reduce_scatter8(const float (&p)[kRowGroups], int kq) {
  const bool b3 = kq & 8, b2 = kq & 4, b1 = kq & 2;
  float q4[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float keep = b3 ? p[m + 4] : p[m];
    const float send = b3 ? p[m] : p[m + 4];
    q4[m] = keep + dpp<kDppRowMirror>(send);
  }
  float q2[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const float keep = b2 ? q4[m + 2] : q4[m];
    const float send = b2 ? q4[m] : q4[m + 2];
    q2[m] = keep + dpp<kDppRowHalfMirror>(send);
  }
  const float keep = b1 ? q2[1] : q2[0];
  const float send = b1 ? q2[0] : q2[1];
  const float s = keep + dpp<kDppQuadXor2>(send);
  return s + dpp<kDppQuadXor1>(s);
}

// Inverse of reduce_scatter8's placement: lane kq holds the value of row group kq >> 1;
// afterwards every lane holds all 8 row-group values of its DPP row, in row-group order.
__device__ __forceinline__ void all_gather8(float x, int kq, float (&out)[kRowGroups]) {
  const bool b3 = kq & 8, b2 = kq & 4, b1 = kq & 2;
  const float o1 = dpp<kDppQuadXor2>(x);
  const float g2[2] = {b1 ? o1 : x, b1 ? x : o1};
  const float h0 = dpp<kDppRowHalfMirror>(g2[0]);
  const float h1 = dpp<kDppRowHalfMirror>(g2[1]);
  const float g4[4] = {b2 ? h0 : g2[0], b2 ? h1 : g2[1], b2 ? g2[0] : h0, b2 ? g2[1] : h1};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float o = dpp<kDppRowMirror>(g4[m]);
    out[m] = b3 ? o : g4[m];
    out[m + 4] = b3 ? g4[m] : o;
  }
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

// One token of the recurrence on the lane's 8x8 slice of the tile:
//   S <- decay*S ; delta = (v - S k^) * beta ; S += delta k^ ; raw = bf16(S q^)
// then the updated slice is stored to `dst_tile` (skipped for a padding slot, NULL).
__device__ __forceinline__ void token_step(f32x4 (&s)[2 * kRowGroups], const float* q,
                                           const float* k, float v_row, float* o,
                                           float decay, float beta, int kq, int my_row,
                                           char* dst_tile, uint32_t lane_bytes) {
  const f32x4 k0 = *reinterpret_cast<const f32x4*>(k + kq * 4);
  const f32x4 k1 = *reinterpret_cast<const f32x4*>(k + 64 + kq * 4);
  const f32x4 q0 = *reinterpret_cast<const f32x4*>(q + kq * 4);
  const f32x4 q1 = *reinterpret_cast<const f32x4*>(q + 64 + kq * 4);

  float part[kRowGroups];
#pragma unroll
  for (int g = 0; g < kRowGroups; ++g) {
    s[2 * g] *= decay;
    s[2 * g + 1] *= decay;
    part[g] = dot8(s[2 * g], s[2 * g + 1], k0, k1);
  }
  const float pred = reduce_scatter8(part, kq);
  const float delta = (v_row - pred) * beta;
  float d[kRowGroups];
  all_gather8(delta, kq, d);
#pragma unroll
  for (int g = 0; g < kRowGroups; ++g) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[2 * g][e] = fmaf(d[g], k0[e], s[2 * g][e]);
      s[2 * g + 1][e] = fmaf(d[g], k1[e], s[2 * g + 1][e]);
    }
    part[g] = dot8(s[2 * g], s[2 * g + 1], q0, q1);
  }
  const float out = reduce_scatter8(part, kq);
  if ((kq & 1) == 0) o[my_row] = round_bf16(out);

  if (dst_tile != nullptr) {
#pragma unroll
    for (int j = 0; j < 2 * kRowGroups; ++j) {
      __builtin_nontemporal_store(
          s[j], reinterpret_cast<f32x4*>(dst_tile + (lane_bytes + tile_piece_bytes(j))));
    }
  }
}

// Waits for this wave's LDS traffic, then joins the workgroup barrier.  Global loads that
// are still in flight stay in flight (a __syncthreads() fence would drain them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Four waves per SIMD (<= 128 VGPRs) keep four workgroups, i.e. four tiles, resident per CU.
// DtBf16 / WBf16: dt_bias / norm_weight stored as bf16 (else fp32).
template <bool DtBf16, bool WBf16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void gdn_decode_kernel(const DecodeParams p) {
  const int tile = blockIdx.x;
  const int request = tile / p.num_v_heads;
  const int head = tile - request * p.num_v_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  const int bos = p.cu[request];
  const int num_tokens = p.cu[request + 1] - bos;
  if (num_tokens <= 0) return;
  const int accepted = p.accepted[request];
  const int32_t* req_slots = p.indices + static_cast<int64_t>(request) * p.width;
  const int source = (accepted >= 1 && accepted <= p.width) ? req_slots[accepted - 1] : 0;
  if (source <= 0 || num_tokens > p.width) {
    // Invalid request: zero outputs, state untouched.
    for (int i = tid; i < num_tokens * kDim; i += kThreads) {
      const int64_t token = bos + (i >> 7);
      p.out[(token * p.num_v_heads + head) * kDim + (i & (kDim - 1))] = 0;
    }
    return;
  }

  __shared__ float s_q[kMaxTokens][kDim];
  __shared__ float s_k[kMaxTokens][kDim];
  __shared__ float s_v[kMaxTokens][kDim];
  __shared__ float s_o[kMaxTokens][kDim];
  __shared__ float s_silu[kMaxTokens][kDim];  // silu(gate)
  __shared__ float s_w[kDim];                  // norm weight
  __shared__ float s_decay[kMaxTokens];
  __shared__ float s_beta[kMaxTokens];

  const int key_head = head / p.group;
  const bool has_token = wave < num_tokens;  // wave t prepares token t
  // Destination slots of the (at most 4) tokens, read before any state store.
  int dest_slot[kMaxTokens];
#pragma unroll
  for (int t = 0; t < kMaxTokens; ++t) dest_slot[t] = t < p.width ? req_slots[t] : 0;

  // ---- small activation loads first, so the tile loads below do not delay them.  Every
  // wave loads (waves past the request's last token re-read that token) so the loads stay
  // in one basic block with the tile loads and their waits sink to the first use. ----
  const int64_t token_w = bos + min(wave, num_tokens - 1);
  uint16_t qh[2], kh[2], vh[2], gh[2];
  float w[2];
  {
    const uint16_t* row = p.qkv + token_w * p.qkv_row;
    const uint16_t* qrow = row + key_head * kDim;
    const uint16_t* krow = row + (p.num_k_heads + key_head) * kDim;
    const uint16_t* vrow = row + (2 * p.num_k_heads + head) * kDim;
    const uint16_t* grow = p.gate + token_w * p.gate_row + head * kDim;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      qh[e] = qrow[2 * lane + e];
      kh[e] = krow[2 * lane + e];
      vh[e] = vrow[2 * lane + e];
      gh[e] = grow[2 * lane + e];
      w[e] = load_param(p.norm_weight, 2 * lane + e, WBf16);
    }
  }
  const uint16_t a_bits = p.a[token_w * p.a_row + head];
  const uint16_t b_bits = p.b[token_w * p.b_row + head];
  const float dt_bias = load_param(p.dt_bias, head, DtBf16);
  const float a_log = p.a_log[head];
  __builtin_amdgcn_sched_barrier(0);

  // ---- the whole 64 KiB source tile: 16 x 128-bit loads per lane (uniform base address,
  // 32-bit per-lane byte offsets) ----
  const int kq = lane & 15;
  const int rsub = lane >> 4;
  const int64_t head_offset = static_cast<int64_t>(head) * kDim * kDim;
  const uint32_t lane_bytes = static_cast<uint32_t>((wave * kRowsPerWave + rsub) * kDim + kq * 4) * 4u;
  const char* src_tile = reinterpret_cast<const char*>(
      p.state + static_cast<int64_t>(source) * p.state_slot + head_offset);
  f32x4 s[2 * kRowGroups];
#pragma unroll
  for (int j = 0; j < 2 * kRowGroups; ++j) {
    s[j] = *reinterpret_cast<const f32x4*>(src_tile + (lane_bytes + tile_piece_bytes(j)));
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue: q/k L2 norm, decay and beta for token `wave`.  Waves past the last token
  // compute on a copy of it and their LDS rows are never read. ----
  {
    float q[2], k[2];
    float qq = 0.0f, kk = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      q[e] = bf16_to_f32(qh[e]);
      k[e] = bf16_to_f32(kh[e]);
      qq = fmaf(q[e], q[e], qq);
      kk = fmaf(k[e], k[e], kk);
    }
    qq = wave_sum(qq);
    kk = wave_sum(kk);
    const float rq = 1.0f / sqrtf(qq + 1e-6f);
    const float rk = 1.0f / sqrtf(kk + 1e-6f);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      s_q[wave][2 * lane + e] = (q[e] * rq) * p.scale;
      s_k[wave][2 * lane + e] = k[e] * rk;
      s_v[wave][2 * lane + e] = bf16_to_f32(vh[e]);
      const float gate = bf16_to_f32(gh[e]);
      s_silu[wave][2 * lane + e] = gate / (1.0f + expf(-gate));
      if (wave == 0) s_w[2 * lane + e] = w[e];
    }
    const float g = -expf(a_log) * softplus(bf16_to_f32(a_bits) + dt_bias);
    const float decay = expf(g);
    const float beta = sigmoid(bf16_to_f32(b_bits));
    if (lane == 0) {
      s_decay[wave] = decay;
      s_beta[wave] = beta;
    }
  }
  lds_barrier();

  // ---- recurrence: 1 tile read, one tile write per token.  Token 0 is peeled off the loop
  // so its first uses of the tile wait for each 16-byte piece separately (s_waitcnt vmcnt(N)
  // per piece) instead of for the whole tile. ----
  const int my_row = wave * kRowsPerWave + (kq >> 1) * 4 + rsub;  // row of reduce results
  char* const state_bytes = reinterpret_cast<char*>(p.state + head_offset);
  const int64_t slot_bytes = p.state_slot * 4;
  token_step(s, s_q[0], s_k[0], s_v[0][my_row], s_o[0], s_decay[0], s_beta[0], kq, my_row,
             dest_slot[0] > 0 ? state_bytes + dest_slot[0] * slot_bytes : nullptr, lane_bytes);
  for (int t = 1; t < num_tokens; ++t) {
    const int dest = t == 1 ? dest_slot[1] : t == 2 ? dest_slot[2] : dest_slot[3];
    token_step(s, s_q[t], s_k[t], s_v[t][my_row], s_o[t], s_decay[t], s_beta[t], kq, my_row,
               dest > 0 ? state_bytes + dest * slot_bytes : nullptr, lane_bytes);
  }
  lds_barrier();

  // ---- gated RMSNorm epilogue for token `wave` ----
  if (has_token) {
    const int64_t token = bos + wave;
    float raw[2];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      raw[e] = s_o[wave][2 * lane + e];
      ss = fmaf(raw[e], raw[e], ss);
    }
    ss = wave_sum(ss);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(kDim) + p.eps);
    uint16_t* orow = p.out + (token * p.num_v_heads + head) * kDim;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int v = 2 * lane + e;
      orow[v] = f32_to_bf16(((raw[e] * rstd) * s_w[v]) * s_silu[wave][v]);
    }
  }
}

}  // namespace
}  // namespace ld

extern "C" int ld_gdn_decode(const ld_gdn_decode_args* args, void* stream) {
  using namespace ld;
  if (args == nullptr) return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode: args is NULL");
  const ld_gdn_decode_args& a = *args;
  if (a.num_requests < 0) return fail(LD_ERR_INVALID_ARGUMENT, "num_requests must be >= 0");
  if (a.width < 1 || a.width > LD_MAX_TOKENS)
    return fail(LD_ERR_INVALID_ARGUMENT, "decode/MTP supports 1 through 4 tokens per request");
  if (a.num_k_heads <= 0 || a.num_v_heads <= 0 || a.num_v_heads % a.num_k_heads != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "num_v_heads must be a positive multiple of num_k_heads");
  if (!(a.eps > 0.0f)) return fail(LD_ERR_INVALID_ARGUMENT, "norm epsilon must be positive");
  if ((a.dt_bias_dtype != LD_DTYPE_F32 && a.dt_bias_dtype != LD_DTYPE_BF16) ||
      (a.norm_weight_dtype != LD_DTYPE_F32 && a.norm_weight_dtype != LD_DTYPE_BF16))
    return fail(LD_ERR_INVALID_ARGUMENT, "weights must be FP32/BF16");
  if (a.num_requests == 0) return LD_OK;
  if (!a.qkv || !a.a || !a.b || !a.a_log || !a.dt_bias || !a.indices || !a.cu || !a.accepted ||
      !a.state || !a.gate || !a.norm_weight || !a.out)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_gdn_decode: NULL tensor pointer");
  if (!aligned16(a.state) || (a.state_slot_stride & 3) != 0)
    return fail(LD_ERR_INVALID_ARGUMENT, "state slots must be 16-byte aligned");
  const int64_t blocks = static_cast<int64_t>(a.num_requests) * a.num_v_heads;
  if (blocks > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "too many (request, head) tiles");

  DecodeParams p;
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
  const bool dt_bf16 = a.dt_bias_dtype == LD_DTYPE_BF16;
  const bool w_bf16 = a.norm_weight_dtype == LD_DTYPE_BF16;
  auto kernel = dt_bf16 ? (w_bf16 ? gdn_decode_kernel<true, true> : gdn_decode_kernel<true, false>)
                        : (w_bf16 ? gdn_decode_kernel<false, true> : gdn_decode_kernel<false, false>);
  hipLaunchKernelGGL(kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  return check_launch("ld_gdn_decode");
}
