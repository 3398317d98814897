// Chunked prefill for gfx950: the delta rule over chunks of 64 or 32 tokens in the WY form,
// with every product on the matrix cores: products with an fp32 operand on the fp32 ones
// (v_mfma_f32_16x16x4_f32: fp32 operands, fp32 accumulation, so the arithmetic is the
// vector ALUs' up to summation order), the dot products of the bf16 inputs q . k and k . k
// on the bf16 ones (v_mfma_f32_16x16x32_bf16: the inputs as they are, exact products, fp32
// sums; the norms are applied to the sums), and in the scans a product of q or k as stored
// (exact bf16) with fp32 data as three bf16 products against the data's exact three-way
// bf16 split (the same exact terms, fp32 sums).
//
// Per chunk (tokens i = 0 .. n-1, n <= C, C = 64 or 32), with g_i the log decay,
// G_i = g_0 + .. + g_i, Gam_ij = exp(G_i - G_j), beta_i, normalised q^_i (scaled) and k^_i,
// and S the state at the chunk's start ([V, K], row v):
//   A_im = beta_i Gam_im (k^_i . k^_m) for m < i            (strictly lower, C x C)
//   (I + A) W = rows beta_i exp(G_i) k^_i,  (I + A) U = rows beta_i v_i   (forward subst.)
//   V_new = U - W S^T                                        (C x 128)
//   O     = (q^_i exp(G_i)) S^T + P V_new,  P_ij = Gam_ij (q^_i . k^_j) for j <= i
//   S'    = exp(G_{n-1}) S + V_new^T (k^_j exp(G_{n-1} - G_j))
// which equals the token-by-token recurrence of the decode kernel (checked against it in
// float64: 7e-8 relative on the state).  After chunk_index_kernel (where each sequence's
// chunks start), two launches:
//   chunk_prep_kernel  one workgroup per (chunk, k-head), all chunks in parallel, running
//                      the group's v-heads in turn: norms, gates, A and P, the blocked
//                      forward substitution for W and U, and q and k with their per-token
//                      scales; everything to workspace records.
//   chunk_scan_kernel  one workgroup per (sequence, v-head, block of 16 or 32 state rows),
//   (64-token chunks)  the only sequential part: chunk by chunk, V_new, the raw outputs of
//                      its columns (rounded to bf16 into `out`, the reference's rounding
//                      point before the gated RMSNorm, which prefill_norm_kernel applies
//                      afterwards) and the state update.  Rows evolve independently, so a
//                      head's 128 rows spread over 8 or 4 workgroups.
//   chunk_scan32_kernel  the same for 32-token chunks, 32 state rows per workgroup.
// A 64-token chunk costs the same whether it holds 64 tokens or 20, so prompts shorter than
// a chunk waste the difference; 32-token chunks halve that waste (and the scan's products
// per token: P V_new grows with the square of the chunk), at twice the sequential steps.
//
// MFMA fragments (16 x 16 x 4, wave64): for lane l, li = l % 16 and lg = l / 16.  One
// instruction takes a = A[li][kk = lg] and b = B[kk = lg][li] from every lane and adds
// sum over kk of A[i][kk] B[kk][j] to D[i][j], held as d[r] = D[4 lg + r][li].  Summation
// indices are assigned to (step, lg) freely as long as both operands agree; in the forward
// substitution k = 4 lg + step, so a result's d[r] is directly the b operand of step r.
#include "gdn_common.h"

namespace ld {
namespace {

constexpr int kC = 64;                          // tokens per chunk (64-token form)

// Workspace record of one (chunk, v-head) of the 64-token form, offsets in floats.  Every
// operand of the scan is stored in the order its loads read it -- [scan wave or tile][step
// group][lane][16 bytes] -- so that one 16-byte-per-lane load of a wave reads 1 KiB of
// consecutive memory.  q and k go as the bf16 inputs themselves (exact), their norms and
// decays as per-token scales applied by the scan.  With li, lg the lane's fragment
// coordinates:
//   W    [w][q < 8][lane][e]  = W[16 w + li][32 lg + 4 q + e]       (W: 64 token x 128 k)
//   U    [b][w][lane][r]      = U[16 w + 4 lg + r][16 b + li]        (b: block of 16 v rows)
//   P    [w][q < 4][lane][e]  = P[16 w + li][16 lg + 4 q + e]
//   Qr   [w][qq < 4][lane][e < 8] = q_i[32 lg + 8 qq + e] (bf16), i = 16 w + li
//   Kr   [t][qq < 2][lane][e < 8] = k_j[16 t + li] (bf16), j = 16 lg + 8 qq + e
//   misc [0] exp(G_n-1); [64 + i] sq_i = rq_i scale exp(G_i); [128 + j] ck_j = rk_j exp(G_n-1 - G_j)
// with w a token tile, rq, rk the inverse L2 norms; rows past the chunk's end hold zeros.
// So the scan's operands are Qg = diag(sq) Qr (applied to the product's rows) and
// Kd = diag(ck) Kr (applied to V_new's rows in the update).  Qr and Kr depend on the k-head
// alone: only the record of a group's first v-head holds them (the others leave that space
// unwritten), and the scans of all the group's v-heads read them there.
constexpr int64_t kOffW = 0;
constexpr int64_t kOffU = kOffW + kC * kDim;
constexpr int64_t kOffP = kOffU + kDim * kC;
constexpr int64_t kOffQr = kOffP + kC * kC;          // bf16 pairs: kC * kDim / 2 floats
constexpr int64_t kOffKr = kOffQr + kC * kDim / 2;
constexpr int64_t kOffMisc = kOffKr + kC * kDim / 2;
constexpr int64_t kMiscSq = 64;
constexpr int64_t kMiscCk = 128;
constexpr int64_t kRecord = kOffMisc + 256;          // floats (a multiple of 64: 256 B)

// The 32-token form keeps (I + A)^-1 itself instead of W and U: with T = (I + A)^-1,
//   V_new = U - W S^T = T (diag(beta) V - diag(ws) K S^T),  ws_i = beta_i exp(G_i) rk_i,
// where the scan forms K S^T from the bf16 keys and reads V from qkv, so a record carries
// 4 KiB of T where W and U took 32 KiB.  Record of one (chunk, v-head), offsets in floats:
//   T    [w][q < 2][lane][e]  = T[16 w + li][8 lg + 4 q + e]         (32 x 32, lower)
//   P    [w][q < 2][lane][e]  = P[16 w + li][8 lg + 4 q + e]
//   Qr   [w][qq < 4][lane][e < 8] = q_i[32 lg + 8 qq + e] (bf16), i = 16 w + li
//   Kq   [w][qq < 4][lane][e < 8] = k_i[32 lg + 8 qq + e] (bf16), i = 16 w + li
//   Kr   [t][lane][e < 8]     = k_j[16 t + li] (bf16), j = 8 lg + e
//   misc as above, and [160 + i] beta_i, [192 + i] ws_i
// Qr, Kq and Kr, as in the 64-token record, only in the record of a group's first v-head.
struct Rec32 {
  static constexpr int kC = 32;
  static constexpr int64_t kOffT = 0;
  static constexpr int64_t kOffP = kOffT + kC * kC;
  static constexpr int64_t kOffQr = kOffP + kC * kC;
  static constexpr int64_t kOffKq = kOffQr + kC * kDim / 2;
  static constexpr int64_t kOffKr = kOffKq + kC * kDim / 2;
  static constexpr int64_t kOffMisc = kOffKr + kC * kDim / 2;
  static constexpr int64_t kSize = kOffMisc + 256;
};
constexpr int64_t kMiscBeta = 160;
constexpr int64_t kMiscWs = 192;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


__device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// chunk_start[n] = sum over m < n of ceil(L_m / C) for n = 0 .. num_sequences: where the
// chunks of sequence n begin in the global chunk order.  One workgroup, a block-wide scan per
// 256 sequences.
template <int C>
__global__ __launch_bounds__(kThreads) void chunk_index_kernel(const int32_t* cu,
                                                               int num_sequences,
                                                               int32_t* chunk_start) {
  __shared__ int32_t wave_total[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid == 0) chunk_start[0] = 0;
  int carry = 0;
  for (int base = 0; base < num_sequences; base += kThreads) {
    const int n = base + tid;
    int c = n < num_sequences ? (cu[n + 1] - cu[n] + C - 1) / C : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int up = __shfl_up(c, d);
      if (lane >= d) c += up;
    }
    if (lane == 63) wave_total[wave] = c;
    __syncthreads();
    int before = carry;
    int total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      before += w < wave ? wave_total[w] : 0;
      total += wave_total[w];
    }
    if (n < num_sequences) chunk_start[n + 1] = before + c;
    carry += total;
    __syncthreads();  // wave_total is rewritten by the next round
  }
}

// Global chunk g -> (sequence, first row, tokens): the last n with chunk_start[n] <= g
// (empty sequences come before it), by a 64-way search with one wave-wide load per level
// (one level up to 64 sequences, two up to 4096; a binary search took one dependent load per
// halving); false past the last chunk.  Called by every lane of a wave; the results are
// uniform.  C: tokens per chunk.
template <int C>
__device__ bool find_chunk(const int32_t* cu, const int32_t* chunk_start, int num_sequences,
                           int g, int& seq, int& t0, int& len) {
  if (g >= chunk_start[num_sequences]) return false;
  const int lane = threadIdx.x & 63;
  int lo = 0;              // chunk_start[lo] <= g throughout
  int count = num_sequences;
  for (;;) {
    const int step = (count + 63) >> 6;   // entries per lane at this level
    const bool in = lane * step < count;
    const int idx = lo + (in ? lane * step : 0);
    const int start = chunk_start[idx];
    int row0 = 0, row1 = 0;
    if (step == 1) {   // the last level: the rows of every candidate in the same round trip
      row0 = cu[idx];
      row1 = cu[idx + 1];
    }
    const int k = 63 - __clzll(static_cast<long long>(__ballot(in && start <= g)));
    if (step == 1) {
      seq = lo + k;
      t0 = __builtin_amdgcn_readlane(row0, k) + (g - __builtin_amdgcn_readlane(start, k)) * C;
      len = min(C, __builtin_amdgcn_readlane(row1, k) - t0);
      return true;
    }
    lo += k * step;
    count = min(step, count - k * step);
  }
}

// The 20 tiles of A (K K^T) and P (Q K^T) on or below the diagonal over the prep's 8 waves:
// 3 each for waves 0-3 and 2 each for waves 4-7 (so 5 per SIMD, waves w and w + 4 sharing
// one), 5 bits a tile, (is_p << 4) | (row tile << 2) | column tile.
constexpr uint32_t tile_code(int is_p, int mt, int nt) { return (is_p << 4) | (mt << 2) | nt; }
constexpr uint32_t tiles3(uint32_t a, uint32_t b, uint32_t c = 0) {
  return a | (b << 5) | (c << 10);
}
__device__ __forceinline__ uint32_t prep_tiles(int wave) {
  switch (wave) {
    case 0: return tiles3(tile_code(0, 0, 0), tile_code(1, 0, 0), tile_code(0, 3, 0));
    case 1: return tiles3(tile_code(0, 1, 0), tile_code(0, 1, 1), tile_code(1, 1, 0));
    case 2: return tiles3(tile_code(0, 2, 0), tile_code(0, 2, 1), tile_code(0, 2, 2));
    case 3: return tiles3(tile_code(1, 2, 0), tile_code(1, 2, 1), tile_code(1, 2, 2));
    case 4: return tiles3(tile_code(1, 3, 0), tile_code(0, 3, 1));
    case 5: return tiles3(tile_code(1, 1, 1), tile_code(1, 3, 1));
    case 6: return tiles3(tile_code(0, 3, 2), tile_code(0, 3, 3));
    default: return tiles3(tile_code(1, 3, 2), tile_code(1, 3, 3));
  }
}

constexpr int kPrepThreads = 512;
constexpr int kPrepWaves = kPrepThreads / 64;
constexpr int kPrepTokens = kC / kPrepWaves;   // tokens normalised per wave

// ---- phase 1: per (chunk, k-head), then per v-head of its group -----------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16v4 __attribute__((ext_vector_type(4)));

// One workgroup per (chunk, k-head).  What depends on q and k alone -- their loads, inverse
// norms, the raw q.k and k.k tiles on the bf16 matrix cores -- is done once; then the
// workgroup runs the group's HV/H v-heads in turn: gates, the scaled A and P, the inverses of
// I + A's diagonal blocks, the substitution for W and U, and the v-head's record.  (One
// workgroup per (chunk, v-head) recomputed the q/k part for every v-head of a group: with
// 16 qk / 32 v heads, about a third of each workgroup's lifetime.)
// Wide: qkv rows at 16-byte alignment, so q, k and v come in 16-byte pieces (8 bf16 of one
// row) instead of one or two bf16 per load: a quarter of the q / k loads and an eighth of
// the v loads, v then transposed through LDS.  Same values, same arithmetic.
template <bool DtBf16, bool Wide>
__global__ __launch_bounds__(kPrepThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void chunk_prep_kernel(const DecodeParams p, int num_sequences, float* ws,
                       const int32_t* chunk_start, int records) {
  const int64_t unit = blockIdx.x;   // chunk * H + k-head
  const int g = static_cast<int>(unit / p.num_k_heads);   // global chunk
  if (g >= records) return;
  const int key_head = static_cast<int>(unit - static_cast<int64_t>(g) * p.num_k_heads);
  int seq = 0, t0 = 0, len = 0;
  if (!find_chunk<kC>(p.cu, chunk_start, num_sequences, g, seq, t0, len)) return;
  // the wave index in a scalar register: the tile table, the A / P choice and the W / U
  // role are then scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;

  constexpr int kHRow = kDim + 8;  // padded LDS row of the bf16 q / k (272 bytes)
  constexpr int kRow = kDim + 4;   // padded LDS row of W (floats)
  constexpr int kARow = kC + 4;    // padded LDS row of -A
  constexpr int kTRow = 20;        // padded LDS row of a diagonal block's inverse
  constexpr int kVCol = kC / 2 + 2;  // padded column of the v staging (token pairs, dwords)
  // q and k (the bf16 inputs, [64][136] each) for the whole workgroup; per v-head, -A
  // ([64][68] fp32) and above it (Wide) the U waves' v, column-major ([128][68] bf16, while
  // they form U's right-hand side), then W ([64][132] fp32) in their place on its way to
  // the workspace; the four inverses [4][16][20] have their own 5 KiB.
  constexpr int kHalfBytes = kC * kHRow * 2;
  constexpr int kApBytes = 2 * kC * kARow * 4;
  static_assert(kC * kRow * 4 <= kApBytes && kDim * kVCol * 4 <= kApBytes / 2, "LDS plan");
  __shared__ __attribute__((aligned(16))) uint8_t sQk[2 * kHalfBytes];
  __shared__ __attribute__((aligned(16))) uint8_t sAp[kApBytes];
  __shared__ __attribute__((aligned(16))) float sT[4 * 16 * kTRow];
  // a v-head's gates, double-buffered (v-head m in buffer m & 1): G_i, beta_i, exp(G_i),
  // exp(G_n-1 - G_i)
  __shared__ float sGates[2][4][kC];
  __shared__ float sRq[kC];     // rq_i scale (zero past the end)
  __shared__ float sRk[kC];     // rk_i (zero past the end)
  uint16_t (*const sQh)[kHRow] = reinterpret_cast<uint16_t (*)[kHRow]>(sQk);
  uint16_t (*const sKh)[kHRow] = reinterpret_cast<uint16_t (*)[kHRow]>(sQk + kHalfBytes);
  float* const sA = reinterpret_cast<float*>(sAp);
  float* const sW = reinterpret_cast<float*>(sAp);
  uint32_t* const sV = reinterpret_cast<uint32_t*>(sAp + kApBytes / 2);

  // Waves 0-3 solve for W's columns 32w .. 32w + 31, waves 4-7 for U's (2 column tiles
  // each).
  constexpr int kNt = 2;   // column tiles per wave
  const bool solves_u = wave >= 4;
  const int n0 = (wave & 3) * 16 * kNt;

  // A v-head's global inputs, fetched one v-head ahead (the first with q and k): U's
  // right-hand side v (U waves) and the gate inputs (wave 0, lane = token).  v comes in the
  // fragment layout, vr[rb][nt][r] = v of token 16 rb + 4 lg + r, column n0 + 16 nt + li,
  // or (Wide) as vw[pr][h] = columns n0 + 8 (lane & 3) .. + 7 of token 2 a + h, token pair
  // a = lane / 4 + 16 pr.
  uint16_t vr[4][kNt][4];
  u32x4 vw[2][2];
  uint16_t gate_a = 0, gate_b = 0;
  float gate_a_log = 0.0f, gate_dt_bias = 0.0f;
  auto fetch_v = [&](int head, int li, int lg) __attribute__((always_inline)) {
    const int v_col = (2 * p.num_k_heads + head) * kDim;
    if constexpr (Wide) {
      const int lane = 16 * lg + li;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t tok = t0 + min(2 * ((lane >> 2) + 16 * pr) + h, len - 1);
          vw[pr][h] = *reinterpret_cast<const u32x4*>(p.qkv + tok * p.qkv_row + v_col + n0 +
                                                      8 * (lane & 3));
        }
    } else {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t tok = t0 + min(16 * rb + 4 * lg + r, len - 1);
          const uint16_t* row = p.qkv + tok * p.qkv_row + v_col + n0 + li;
#pragma unroll
          for (int nt = 0; nt < kNt; ++nt) vr[rb][nt][r] = row[16 * nt];
        }
    }
  };
  auto fetch_gates = [&](int head, int lane) __attribute__((always_inline)) {
    const int64_t tok = t0 + min(lane, len - 1);
    gate_a = p.a[tok * p.a_row + head];
    gate_b = p.b[tok * p.b_row + head];
    gate_a_log = p.a_log[head];
    gate_dt_bias = load_param(p.dt_bias, head, DtBf16);
  };
  // The gates and the in-chunk cumulative log decay of v-head `member` from the fetched
  // inputs (one wave, lane = token), then the fetch of the inputs two v-heads on.  Wave 4
  // computes those of v-head 0 before the q / k barrier and those of v-head m + 1 while
  // waves 0-3 invert v-head m's diagonal blocks; each is read after at least one barrier.
  auto gates = [&](int member, int lane) __attribute__((always_inline)) {
    const int head = key_head * p.group + member;
    const bool live = lane < len;
    const float x = bf16_to_f32(gate_a) + gate_dt_bias;
    const float gl = live ? -__expf(gate_a_log) * softplus(x) : 0.0f;
    const float beta = live ? sigmoid(bf16_to_f32(gate_b)) : 0.0f;
    if (member + 1 < p.group) fetch_gates(head + 1, lane);
    float G = gl;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float up = __shfl_up(G, d);
      if (lane >= d) G += up;
    }
    const float glast = __shfl(G, len - 1);
    float (*const gb)[kC] = sGates[member & 1];
    gb[0][lane] = G;
    gb[1][lane] = beta;
    gb[2][lane] = __expf(G);
    gb[3][lane] = __expf(glast - G);
    if (lane == 0) ws[(static_cast<int64_t>(g) * p.num_v_heads + head) * kRecord + kOffMisc] = __expf(glast);
  };
  if (wave == 4) fetch_gates(key_head * p.group, threadIdx.x & 63);

  // q and k of the chunk's tokens and their inverse norms (zero rows past its end); wave w
  // does tokens 8w .. 8w+7, all 8 tokens' loads in flight before the first norm
  if constexpr (Wide) {
    // lane (row quarter, l16) holds elements 8 l16 .. 8 l16 + 7 of tokens 8w + 4h + quarter:
    // the sum of squares runs in wave_sum's order (a lane's four pairs as four of its lanes
    // would sum them, then the 16 lanes of the DPP row as its remaining levels)
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int quarter = lane >> 4;
    u32x4 qv[2], kv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t tok = t0 + min(wave * kPrepTokens + 4 * h + quarter, len - 1);
      const uint16_t* row = p.qkv + tok * p.qkv_row;
      qv[h] = *reinterpret_cast<const u32x4*>(row + q_col + 8 * l16);
      kv[h] = *reinterpret_cast<const u32x4*>(row + k_col + 8 * l16);
    }
    // v of the first v-head behind q and k (loads return in order; the norms come first)
    if (solves_u) fetch_v(key_head * p.group, threadIdx.x & 15, (threadIdx.x >> 4) & 3);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = wave * kPrepTokens + 4 * h + quarter;
      float pq[4], pk[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float q0 = __builtin_bit_cast(float, qv[h][m] << 16);
        const float q1 = __builtin_bit_cast(float, qv[h][m] & 0xffff0000u);
        const float k0 = __builtin_bit_cast(float, kv[h][m] << 16);
        const float k1 = __builtin_bit_cast(float, kv[h][m] & 0xffff0000u);
        pq[m] = fmaf(q1, q1, q0 * q0);
        pk[m] = fmaf(k1, k1, k0 * k0);
      }
      float qq = (pq[0] + pq[1]) + (pq[2] + pq[3]);
      float kk = (pk[0] + pk[1]) + (pk[2] + pk[3]);
      qq += dpp<kDppQuadXor1>(qq);
      kk += dpp<kDppQuadXor1>(kk);
      qq += dpp<kDppQuadXor2>(qq);
      kk += dpp<kDppQuadXor2>(kk);
      qq += dpp<kDppRowHalfMirror>(qq);
      kk += dpp<kDppRowHalfMirror>(kk);
      qq += dpp<kDppRowMirror>(qq);
      kk += dpp<kDppRowMirror>(kk);
      const bool live = i < len;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&sQh[i][8 * l16]) = live ? qv[h] : zero;
      *reinterpret_cast<u32x4*>(&sKh[i][8 * l16]) = live ? kv[h] : zero;
      if (l16 == 0) {
        sRq[i] = live ? fast_rsqrt(qq + 1e-6f) * p.scale : 0.0f;
        sRk[i] = live ? fast_rsqrt(kk + 1e-6f) : 0.0f;
      }
    }
  } else {
    const int lane = threadIdx.x & 63;
    uint32_t qr[kPrepTokens], kr[kPrepTokens];
#pragma unroll
    for (int ii = 0; ii < kPrepTokens; ++ii) {
      const int64_t tok = t0 + min(wave * kPrepTokens + ii, len - 1);
      const uint16_t* row = p.qkv + tok * p.qkv_row;
      qr[ii] = row[q_col + 2 * lane] | (static_cast<uint32_t>(row[q_col + 2 * lane + 1]) << 16);
      kr[ii] = row[k_col + 2 * lane] | (static_cast<uint32_t>(row[k_col + 2 * lane + 1]) << 16);
    }
    if (solves_u) fetch_v(key_head * p.group, threadIdx.x & 15, (threadIdx.x >> 4) & 3);
#pragma unroll
    for (int ii = 0; ii < kPrepTokens; ++ii) {
      const int i = wave * kPrepTokens + ii;
      const float q0 = __builtin_bit_cast(float, qr[ii] << 16);
      const float q1 = __builtin_bit_cast(float, qr[ii] & 0xffff0000u);
      const float k0 = __builtin_bit_cast(float, kr[ii] << 16);
      const float k1 = __builtin_bit_cast(float, kr[ii] & 0xffff0000u);
      const float qq = wave_sum(fmaf(q1, q1, q0 * q0));
      const float kk = wave_sum(fmaf(k1, k1, k0 * k0));
      const bool live = i < len;
      *reinterpret_cast<uint32_t*>(&sQh[i][2 * lane]) = live ? qr[ii] : 0u;
      *reinterpret_cast<uint32_t*>(&sKh[i][2 * lane]) = live ? kr[ii] : 0u;
      if (lane == 0) {
        sRq[i] = live ? fast_rsqrt(qq + 1e-6f) * p.scale : 0.0f;
        sRk[i] = live ? fast_rsqrt(kk + 1e-6f) : 0.0f;
      }
    }
  }
  if (wave == 4) gates(0, threadIdx.x & 63);
  __syncthreads();

  // Qr and Kr (the bf16 inputs in the scan's load order, item = one 16-byte piece) depend on
  // the k-head alone: they go once, to the record of the group's first v-head, where the
  // scans of all its v-heads read them
  {
    const int tid = threadIdx.x;
    float* rec0 = ws + (static_cast<int64_t>(g) * p.num_v_heads + key_head * p.group) * kRecord;
    u32x4* qdst = reinterpret_cast<u32x4*>(rec0 + kOffQr);
    u32x4* kdst = reinterpret_cast<u32x4*>(rec0 + kOffKr);
#pragma unroll
    for (int it = 0; it < kC * kDim / 8 / kPrepThreads; ++it) {
      const int item = it * kPrepThreads + tid;
      const int l = item & 63;
      const int i = 16 * (item >> 8) + (l & 15);
      const int c0 = 32 * (l >> 4) + 8 * ((item >> 6) & 3);
      qdst[item] = *reinterpret_cast<const u32x4*>(&sQh[i][c0]);
      const int k = 16 * (item >> 7) + (l & 15);
      const int j = 16 * (l >> 4) + 8 * ((item >> 6) & 1);
      kdst[item] = u32x4{sKh[j][k] | (static_cast<uint32_t>(sKh[j + 1][k]) << 16),
                         sKh[j + 2][k] | (static_cast<uint32_t>(sKh[j + 3][k]) << 16),
                         sKh[j + 4][k] | (static_cast<uint32_t>(sKh[j + 5][k]) << 16),
                         sKh[j + 6][k] | (static_cast<uint32_t>(sKh[j + 7][k]) << 16)};
    }
  }

  for (int member = 0; member < p.group; ++member) {
    // The lane coordinates are derived anew in every iteration, through a zero the compiler
    // cannot see through: the loop's per-lane addresses are then formed in the loop, where
    // they are used, instead of being hoisted and held in registers across it (which
    // spilled).
    int opaque_zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(opaque_zero));
    const int tid = static_cast<int>(threadIdx.x) + opaque_zero;
    const int lane = tid & 63;
    const int li = lane & 15;
    const int lg = lane >> 4;
    const int head = key_head * p.group + member;
    const bool next = member + 1 < p.group;
    float* rec = ws + (static_cast<int64_t>(g) * p.num_v_heads + head) * kRecord;
    const float* const sG = sGates[member & 1][0];
    const float* const sBeta = sGates[member & 1][1];
    const float* const sEg = sGates[member & 1][2];
    const float* const sEk = sGates[member & 1][3];

    // A and P tiles of the raw inputs, q_i . k_m and k_i . k_m: bf16 operands with exact
    // products and fp32 accumulation (v_mfma_f32_16x16x32_bf16, lane (li, lg) giving
    // X[row li][32 s + 8 lg + e]), 4 steps of 32 per tile; the third tile for waves 0-3 only
    // (a uniform branch).  Recomputed for each v-head (12 products), so that no register
    // carries them from one v-head to the next.
    const uint32_t codes = prep_tiles(wave);
    const int tiles = wave < 4 ? 3 : 2;
    f32x4 prod[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      if (t >= tiles) break;
      const uint32_t code = (codes >> (5 * t)) & 31u;
      const int mt = (code >> 2) & 3;
      const int nt = code & 3;
      // A tiles as K K^T (row tile mt, column tile nt); P tiles transposed, as K Q^T (row
      // tile nt of K against row tile mt of Q), so that a lane's four results are four
      // consecutive columns of one row of P: one 16-byte piece of its record layout
      const bool is_p = (code & 16u) != 0;
      const uint16_t* arow = &sKh[0][0] + (16 * (is_p ? nt : mt) + li) * kHRow + 8 * lg;
      const uint16_t* brow = (is_p ? &sQh[0][0] : &sKh[0][0]) + (16 * (is_p ? mt : nt) + li) * kHRow + 8 * lg;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + 32 * s4);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(brow + 32 * s4);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
      }
      prod[t] = acc;
    }

    // the right-hand sides in the fragment layout: x[rb][nt][r] = B[16 rb + 4 lg + r][n0 + 16 nt + li]
    // (one uniform branch around two straight-line loops)
    f32x4 x[4][kNt];
    if (solves_u) {
      if constexpr (Wide) {
        // the wave's 32 columns of v to LDS column by column, a dword per token pair, and
        // back in the fragment layout (4 tokens of one column per 8-byte read); the wave's
        // own region, so program order is the only ordering needed
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const int a = (lane >> 2) + 16 * pr;
          const int c0 = n0 + 8 * (lane & 3);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t lo = vw[pr][0][d];
            const uint32_t hi = vw[pr][1][d];
            sV[(c0 + 2 * d) * kVCol + a] = (lo & 0xffffu) | (hi << 16);
            sV[(c0 + 2 * d + 1) * kVCol + a] = (lo >> 16) | (hi & 0xffff0000u);
          }
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
          for (int nt = 0; nt < kNt; ++nt) {
            const uint2 t4 = *reinterpret_cast<const uint2*>(
                &sV[(n0 + 16 * nt + li) * kVCol + 8 * rb + 2 * lg]);
            const uint16_t tv[4] = {static_cast<uint16_t>(t4.x), static_cast<uint16_t>(t4.x >> 16),
                                    static_cast<uint16_t>(t4.y), static_cast<uint16_t>(t4.y >> 16)};
#pragma unroll
            for (int r = 0; r < 4; ++r)
              x[rb][nt][r] = sBeta[16 * rb + 4 * lg + r] * bf16_to_f32(tv[r]);  // beta: zero past the end
          }
      } else {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float beta = sBeta[16 * rb + 4 * lg + r];  // zero past the end
#pragma unroll
            for (int nt = 0; nt < kNt; ++nt) x[rb][nt][r] = beta * bf16_to_f32(vr[rb][nt][r]);
          }
      }
    } else {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * rb + 4 * lg + r;
          const float wscale = sBeta[i] * sEg[i] * sRk[i];
#pragma unroll
          for (int nt = 0; nt < kNt; ++nt)
            x[rb][nt][r] = wscale * bf16_to_f32(sKh[i][n0 + 16 * nt + li]);
        }
    }

    // the per-token scales to the v-head's record
    if (tid < kC)
      rec[kOffMisc + kMiscSq + tid] = sRq[tid] * sEg[tid];
    else if (tid < 2 * kC)
      rec[kOffMisc + kMiscCk + tid - kC] = sRk[tid - kC] * sEk[tid - kC];

    // scale the tiles: A (negated) to LDS; P straight to the record, where its piece
    // [row tile mt][q = lg][lane (li, column tile nt)] holds P[16 mt + li][16 nt + 4 lg + r]
    // (the products are of the raw inputs: q^_i . k^_m = (rq_i scale rk_m) (q_i . k_m))
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      if (t >= tiles) break;
      const uint32_t code = (codes >> (5 * t)) & 31u;
      const int mt = (code >> 2) & 3;
      const int nt = code & 3;
      if (code & 16u) {
        const int i = 16 * mt + li;
        const float gi = sG[i];
        const float rqi = sRq[i];
        f32x4 piece;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * nt + 4 * lg + r;
          const float gam = __expf(gi - sG[m]);
          piece[r] = (m <= i && i < len) ? gam * ((rqi * sRk[m]) * prod[t][r]) : 0.0f;
        }
        *reinterpret_cast<f32x4*>(rec + kOffP + ((mt * 4 + lg) * 64 + nt * 16 + li) * 4) = piece;
      } else {
        const int m = 16 * nt + li;
        const float gm = sG[m];
        const float rkm = sRk[m];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * mt + 4 * lg + r;
          const float gam = __expf(sG[i] - gm);
          sA[i * kARow + m] = m < i ? -(sBeta[i] * gam * ((sRk[i] * rkm) * prod[t][r])) : 0.0f;
        }
      }
    }
    // P's six tiles above the diagonal, (row tile, column tile) = (0, 1..3), (1, 2..3),
    // (2, 3): zeros, one 16-byte piece per thread
    if (tid < 6 * 64) {
      const int z = tid >> 6;
      const int mt = z < 3 ? 0 : (z < 5 ? 1 : 2);
      const int nt = z < 3 ? z + 1 : (z < 5 ? z - 1 : 3);
      *reinterpret_cast<f32x4*>(rec + kOffP + ((mt * 4 + lg) * 64 + nt * 16 + li) * 4) =
          f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
    if (wave == 4 && next) gates(member + 1, lane);
    // the U waves are idle here; the next v-head forms its right-hand side from these
    if (solves_u && next) fetch_v(head + 1, li, lg);
    // inverses of the unit lower-triangular diagonal blocks (I + A_bb), column li per lane
    // (block w by wave w < 4)
    if (wave < 4 && lane < 16) {
      const float* ab = sA + (16 * wave) * kARow + 16 * wave;
      // row by row: col[i] = delta(i, li) + sum over m < i of (-A)[i][m] col[m], the terms in
      // order of m (row i of -A read as it is needed)
      float col[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float acc = i == li ? 1.0f : 0.0f;
#pragma unroll
        for (int m = 0; m < i; ++m) acc = fmaf(ab[i * kARow + m], col[m], acc);
        col[i] = acc;
      }
      float* tb = sT + wave * 16 * kTRow;
#pragma unroll
      for (int i = 0; i < 16; ++i) tb[i * kTRow + li] = col[i];
    }
    __syncthreads();

    // blocked forward substitution: X_rb = T_rb (B_rb - sum over j < rb of A_rb,j X_j)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 y[kNt];
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) y[nt] = x[rb][nt];
#pragma unroll
      for (int j = 0; j < rb; ++j) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(sA + (16 * rb + li) * kARow + 16 * j + 4 * lg);
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt) {
          y[nt] = mfma(a.x, x[j][nt].x, y[nt]);
          y[nt] = mfma(a.y, x[j][nt].y, y[nt]);
          y[nt] = mfma(a.z, x[j][nt].z, y[nt]);
          y[nt] = mfma(a.w, x[j][nt].w, y[nt]);
        }
      }
      const f32x4 tr = *reinterpret_cast<const f32x4*>(sT + (rb * 16 + li) * kTRow + 4 * lg);
#pragma unroll
      for (int nt = 0; nt < kNt; ++nt) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        acc = mfma(tr.x, y[nt].x, acc);
        acc = mfma(tr.y, y[nt].y, acc);
        acc = mfma(tr.z, y[nt].z, acc);
        acc = mfma(tr.w, y[nt].w, acc);
        x[rb][nt] = acc;
      }
    }

    // U straight from the fragments (its row block rb is the scan wave, its column tile the
    // scan's block of v rows); W through LDS, once every wave is past its reads of -A (W takes
    // the region of -A and the v staging)
    if (solves_u) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt)
          *reinterpret_cast<f32x4*>(rec + kOffU + (((n0 >> 4) + nt) * 4 + rb) * 256 + lane * 4) =
              x[rb][nt];
    }
    __syncthreads();
    if (!solves_u) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int nt = 0; nt < kNt; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sW[(16 * rb + 4 * lg + r) * kRow + n0 + 16 * nt + li] = x[rb][nt][r];
    }
    __syncthreads();
    {
      f32x4* wdst = reinterpret_cast<f32x4*>(rec + kOffW);
#pragma unroll
      for (int it = 0; it < kC * kDim / 4 / kPrepThreads; ++it) {
        const int item = it * kPrepThreads + tid;
        const int l = item & 63;
        const int i = 16 * (item >> 9) + (l & 15);
        const int k4 = 32 * (l >> 4) + 4 * ((item >> 6) & 7);
        wdst[item] = *reinterpret_cast<const f32x4*>(sW + i * kRow + k4);
      }
    }
    // the next v-head rewrites the gates, -A, P and W
    __syncthreads();
  }
}

// ---- phase 1, 32-token chunks: per (chunk, k-head), then per v-head of its group -----------
// Four waves.  The q/k part -- loads, inverse norms, the raw q.k and k.k tiles on the bf16
// matrix cores, the bf16 queries and keys to the record -- once; then per v-head the gates,
// the per-token scales, the scaled A (to LDS) and P (to the record), the inverses T0, T1 of
// I + A's diagonal blocks, the block T10 = -T1 A10 T0 below them, and T to the record.  No
// forward substitution over v or k columns, and no v: the scan applies T itself.
constexpr int kPrep32Threads = 256;

// Offset (floats, from the start of P or T) of the 16-byte piece holding X[16 mt + li][c ..
// c + 3], c = 16 nt + 4 lg, in the layout [mt][q][lane (lg', li)][e] with 8 lg' + 4 q = c.
__device__ __forceinline__ int piece32(int mt, int nt, int lg, int li) {
  return ((mt * 2 + (lg & 1)) * 64 + (2 * nt + (lg >> 1)) * 16 + li) * 4;
}

// The 6 tiles of A (K K^T) and P (Q K^T) on or below the diagonal, as tile_code: A00, A10,
// A11, P00, P10, P11; wave w takes tiles w and w + 4.
__device__ __forceinline__ uint32_t prep32_tile(int index) {
  switch (index) {
    case 0: return tile_code(0, 0, 0);
    case 1: return tile_code(0, 1, 0);
    case 2: return tile_code(0, 1, 1);
    case 3: return tile_code(1, 0, 0);
    case 4: return tile_code(1, 1, 0);
    default: return tile_code(1, 1, 1);
  }
}

template <bool DtBf16, bool Wide>
__global__ __launch_bounds__(kPrep32Threads) __attribute__((amdgpu_waves_per_eu(5)))
void chunk_prep32_kernel(const DecodeParams p, int num_sequences, float* ws,
                         const int32_t* chunk_start, int records) {
  using R = Rec32;
  constexpr int kCs = R::kC;
  constexpr int kTokens = kCs / (kPrep32Threads / 64);   // tokens normalised per wave
  const int64_t unit = blockIdx.x;   // chunk * H + k-head
  const int g = static_cast<int>(unit / p.num_k_heads);
  if (g >= records) return;
  const int key_head = static_cast<int>(unit - static_cast<int64_t>(g) * p.num_k_heads);
  int seq = 0, t0 = 0, len = 0;
  if (!find_chunk<kCs>(p.cu, chunk_start, num_sequences, g, seq, t0, len)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;

  constexpr int kHRow = kDim + 8;   // padded LDS row of the bf16 q / k (272 bytes)
  constexpr int kARow = kCs + 4;    // padded LDS row of -A
  constexpr int kTRow = 20;         // padded LDS row of a 16 x 16 block of T
  __shared__ __attribute__((aligned(16))) uint16_t sQh[kCs][kHRow];
  __shared__ __attribute__((aligned(16))) uint16_t sKh[kCs][kHRow];
  __shared__ __attribute__((aligned(16))) float sA[kCs][kARow];     // -A of the v-head
  __shared__ __attribute__((aligned(16))) float sT[3][16][kTRow];   // T0, T1, T10
  // a v-head's gates, double-buffered (v-head m in buffer m & 1): G_i, beta_i, exp(G_i),
  // exp(G_n-1 - G_i), one entry per lane of the wave that forms them
  __shared__ float sGates[2][4][64];
  __shared__ float sRq[kCs];   // rq_i scale (zero past the end)
  __shared__ float sRk[kCs];   // rk_i (zero past the end)

  // The gate inputs of a v-head (wave 3, lane = token), fetched one v-head ahead, and the
  // gates and in-chunk cumulative log decay from them: the 64-token prep's arithmetic.
  uint16_t gate_a = 0, gate_b = 0;
  float gate_a_log = 0.0f, gate_dt_bias = 0.0f;
  auto fetch_gates = [&](int head) __attribute__((always_inline)) {
    const int64_t tok = t0 + min(lane, len - 1);
    gate_a = p.a[tok * p.a_row + head];
    gate_b = p.b[tok * p.b_row + head];
    gate_a_log = p.a_log[head];
    gate_dt_bias = load_param(p.dt_bias, head, DtBf16);
  };
  auto gates = [&](int member) __attribute__((always_inline)) {
    const int head = key_head * p.group + member;
    const bool live = lane < len;
    const float x = bf16_to_f32(gate_a) + gate_dt_bias;
    const float gl = live ? -__expf(gate_a_log) * softplus(x) : 0.0f;
    const float beta = live ? sigmoid(bf16_to_f32(gate_b)) : 0.0f;
    if (member + 1 < p.group) fetch_gates(head + 1);
    float G = gl;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float up = __shfl_up(G, d);
      if (lane >= d) G += up;
    }
    const float glast = __shfl(G, len - 1);
    float (*const gb)[64] = sGates[member & 1];
    gb[0][lane] = G;
    gb[1][lane] = beta;
    gb[2][lane] = __expf(G);
    gb[3][lane] = __expf(glast - G);
    if (lane == 0)
      ws[(static_cast<int64_t>(g) * p.num_v_heads + head) * R::kSize + R::kOffMisc] = __expf(glast);
  };
  if (wave == 3) fetch_gates(key_head * p.group);

  // q and k of the chunk's tokens and their inverse norms (zero rows past its end), as the
  // 64-token prep: wave w does tokens 8w .. 8w + 7
  if constexpr (Wide) {
    const int quarter = lane >> 4;
    u32x4 qv[kTokens / 4], kv[kTokens / 4];
#pragma unroll
    for (int h = 0; h < kTokens / 4; ++h) {
      const int64_t tok = t0 + min(wave * kTokens + 4 * h + quarter, len - 1);
      const uint16_t* row = p.qkv + tok * p.qkv_row;
      qv[h] = *reinterpret_cast<const u32x4*>(row + q_col + 8 * li);
      kv[h] = *reinterpret_cast<const u32x4*>(row + k_col + 8 * li);
    }
#pragma unroll
    for (int h = 0; h < kTokens / 4; ++h) {
      const int i = wave * kTokens + 4 * h + quarter;
      float pq[4], pk[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float q0 = __builtin_bit_cast(float, qv[h][m] << 16);
        const float q1 = __builtin_bit_cast(float, qv[h][m] & 0xffff0000u);
        const float k0 = __builtin_bit_cast(float, kv[h][m] << 16);
        const float k1 = __builtin_bit_cast(float, kv[h][m] & 0xffff0000u);
        pq[m] = fmaf(q1, q1, q0 * q0);
        pk[m] = fmaf(k1, k1, k0 * k0);
      }
      float qq = (pq[0] + pq[1]) + (pq[2] + pq[3]);
      float kk = (pk[0] + pk[1]) + (pk[2] + pk[3]);
      qq += dpp<kDppQuadXor1>(qq);
      kk += dpp<kDppQuadXor1>(kk);
      qq += dpp<kDppQuadXor2>(qq);
      kk += dpp<kDppQuadXor2>(kk);
      qq += dpp<kDppRowHalfMirror>(qq);
      kk += dpp<kDppRowHalfMirror>(kk);
      qq += dpp<kDppRowMirror>(qq);
      kk += dpp<kDppRowMirror>(kk);
      const bool live = i < len;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&sQh[i][8 * li]) = live ? qv[h] : zero;
      *reinterpret_cast<u32x4*>(&sKh[i][8 * li]) = live ? kv[h] : zero;
      if (li == 0) {
        sRq[i] = live ? fast_rsqrt(qq + 1e-6f) * p.scale : 0.0f;
        sRk[i] = live ? fast_rsqrt(kk + 1e-6f) : 0.0f;
      }
    }
  } else {
    uint32_t qr[kTokens], kr[kTokens];
#pragma unroll
    for (int ii = 0; ii < kTokens; ++ii) {
      const int64_t tok = t0 + min(wave * kTokens + ii, len - 1);
      const uint16_t* row = p.qkv + tok * p.qkv_row;
      qr[ii] = row[q_col + 2 * lane] | (static_cast<uint32_t>(row[q_col + 2 * lane + 1]) << 16);
      kr[ii] = row[k_col + 2 * lane] | (static_cast<uint32_t>(row[k_col + 2 * lane + 1]) << 16);
    }
#pragma unroll
    for (int ii = 0; ii < kTokens; ++ii) {
      const int i = wave * kTokens + ii;
      const float q0 = __builtin_bit_cast(float, qr[ii] << 16);
      const float q1 = __builtin_bit_cast(float, qr[ii] & 0xffff0000u);
      const float k0 = __builtin_bit_cast(float, kr[ii] << 16);
      const float k1 = __builtin_bit_cast(float, kr[ii] & 0xffff0000u);
      const float qq = wave_sum(fmaf(q1, q1, q0 * q0));
      const float kk = wave_sum(fmaf(k1, k1, k0 * k0));
      const bool live = i < len;
      *reinterpret_cast<uint32_t*>(&sQh[i][2 * lane]) = live ? qr[ii] : 0u;
      *reinterpret_cast<uint32_t*>(&sKh[i][2 * lane]) = live ? kr[ii] : 0u;
      if (lane == 0) {
        sRq[i] = live ? fast_rsqrt(qq + 1e-6f) * p.scale : 0.0f;
        sRk[i] = live ? fast_rsqrt(kk + 1e-6f) : 0.0f;
      }
    }
  }
  if (wave == 3) gates(0);
  __syncthreads();

  // Qr, Kq and Kr (the bf16 inputs in the scan's load order, item = one 16-byte piece) to
  // the record of the group's first v-head
  {
    float* rec0 = ws + (static_cast<int64_t>(g) * p.num_v_heads + key_head * p.group) * R::kSize;
    u32x4* qdst = reinterpret_cast<u32x4*>(rec0 + R::kOffQr);
    u32x4* kqdst = reinterpret_cast<u32x4*>(rec0 + R::kOffKq);
    u32x4* krdst = reinterpret_cast<u32x4*>(rec0 + R::kOffKr);
#pragma unroll
    for (int it = 0; it < kCs * kDim / 8 / kPrep32Threads; ++it) {
      const int item = it * kPrep32Threads + tid;
      const int l = item & 63;
      const int i = 16 * (item >> 8) + (l & 15);
      const int c0 = 32 * (l >> 4) + 8 * ((item >> 6) & 3);
      qdst[item] = *reinterpret_cast<const u32x4*>(&sQh[i][c0]);
      kqdst[item] = *reinterpret_cast<const u32x4*>(&sKh[i][c0]);
      const int k = 16 * (item >> 6) + (l & 15);
      const int j = 8 * (l >> 4);
      krdst[item] = u32x4{sKh[j][k] | (static_cast<uint32_t>(sKh[j + 1][k]) << 16),
                          sKh[j + 2][k] | (static_cast<uint32_t>(sKh[j + 3][k]) << 16),
                          sKh[j + 4][k] | (static_cast<uint32_t>(sKh[j + 5][k]) << 16),
                          sKh[j + 6][k] | (static_cast<uint32_t>(sKh[j + 7][k]) << 16)};
    }
  }

  // The raw tiles, q_i . k_m and k_i . k_m of the bf16 inputs (exact products, fp32 sums),
  // once for all the group's v-heads: A tiles as K K^T (row tile mt, column tile nt), P tiles
  // transposed, as K Q^T, so that a lane's four results are four consecutive columns of one
  // row of P
  const int tiles = wave < 2 ? 2 : 1;
  f32x4 prod[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t >= tiles) break;
    const uint32_t code = prep32_tile(wave + 4 * t);
    const int mt = (code >> 2) & 3;
    const int nt = code & 3;
    const bool is_p = (code & 16u) != 0;
    const uint16_t* arow = &sKh[16 * (is_p ? nt : mt) + li][8 * lg];
    const uint16_t* brow = is_p ? &sQh[16 * mt + li][8 * lg] : &sKh[16 * nt + li][8 * lg];
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + 32 * s4);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(brow + 32 * s4);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
    }
    prod[t] = acc;
  }

  for (int member = 0; member < p.group; ++member) {
    const int head = key_head * p.group + member;
    const bool next = member + 1 < p.group;
    float* rec = ws + (static_cast<int64_t>(g) * p.num_v_heads + head) * R::kSize;
    const float* const sG = sGates[member & 1][0];
    const float* const sBeta = sGates[member & 1][1];
    const float* const sEg = sGates[member & 1][2];
    const float* const sEk = sGates[member & 1][3];

    // the per-token scales: sq = rq scale exp(G), beta, ck = rk exp(G_n-1 - G),
    // ws = beta exp(G) rk (the 64-token prep's W scale)
    if (tid < kCs) {
      rec[R::kOffMisc + kMiscSq + tid] = sRq[tid] * sEg[tid];
      rec[R::kOffMisc + kMiscBeta + tid] = sBeta[tid];
    } else if (tid < 2 * kCs) {
      const int j = tid - kCs;
      rec[R::kOffMisc + kMiscCk + j] = sRk[j] * sEk[j];
      rec[R::kOffMisc + kMiscWs + j] = sBeta[j] * sEg[j] * sRk[j];
    }

    // scale the tiles: A (negated) to LDS, P to the record (the products are of the raw
    // inputs: q^_i . k^_m = (rq_i scale rk_m) (q_i . k_m)); P's tile above the diagonal
    // gets zeros
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= tiles) break;
      const uint32_t code = prep32_tile(wave + 4 * t);
      const int mt = (code >> 2) & 3;
      const int nt = code & 3;
      if (code & 16u) {
        const int i = 16 * mt + li;
        const float gi = sG[i];
        const float rqi = sRq[i];
        f32x4 piece;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * nt + 4 * lg + r;
          const float gam = __expf(gi - sG[m]);
          piece[r] = (m <= i && i < len) ? gam * ((rqi * sRk[m]) * prod[t][r]) : 0.0f;
        }
        *reinterpret_cast<f32x4*>(rec + R::kOffP + piece32(mt, nt, lg, li)) = piece;
      } else {
        const int m = 16 * nt + li;
        const float gm = sG[m];
        const float rkm = sRk[m];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * mt + 4 * lg + r;
          const float gam = __expf(sG[i] - gm);
          sA[i][m] = m < i ? -(sBeta[i] * gam * ((sRk[i] * rkm) * prod[t][r])) : 0.0f;
        }
      }
    }
    if (wave == 2)
      *reinterpret_cast<f32x4*>(rec + R::kOffP + piece32(0, 1, lg, li)) =
          f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();   // -A complete
    if (wave == 3 && next) gates(member + 1);
    // inverses of the unit lower-triangular diagonal blocks (I + A_bb), column li per lane
    // (block w by wave w < 2), row by row: col[i] = delta(i, li) + sum over m < i of
    // (-A)[i][m] col[m], the terms in order of m
    if (wave < 2 && lane < 16) {
      float col[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float acc = i == li ? 1.0f : 0.0f;
#pragma unroll
        for (int m = 0; m < i; ++m) acc = fmaf(sA[16 * wave + i][16 * wave + m], col[m], acc);
        col[i] = acc;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[wave][i][li] = col[i];
    }
    __syncthreads();   // T0, T1 complete
    // T10 = T1 ((-A10) T0) on the fp32 matrix cores, summation index k = 4 lg + step, so the
    // first product's d[r] is the second's b operand of step r
    if (wave == 0) {
      const f32x4 a10 = *reinterpret_cast<const f32x4*>(&sA[16 + li][4 * lg]);
      f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 4; ++st) z = mfma(a10[st], sT[0][4 * lg + st][li], z);
      const f32x4 t1 = *reinterpret_cast<const f32x4*>(&sT[1][li][4 * lg]);
      f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 4; ++st) d = mfma(t1[st], z[st], d);
#pragma unroll
      for (int r = 0; r < 4; ++r) sT[2][4 * lg + r][li] = d[r];
    }
    __syncthreads();   // T10 complete
    // T to the record, one piece per thread: piece (w, q) = tid / 64 holds
    // T[16 w + li][8 lg + 4 q ..]: T0 and zeros for w = 0, T10 and T1 for w = 1
    {
      const int w = tid >> 7;
      const int c = 8 * lg + 4 * ((tid >> 6) & 1);
      f32x4 v;
      if (w == 0)
        v = c < 16 ? *reinterpret_cast<const f32x4*>(&sT[0][li][c]) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      else
        v = c < 16 ? *reinterpret_cast<const f32x4*>(&sT[2][li][c])
                   : *reinterpret_cast<const f32x4*>(&sT[1][li][c - 16]);
      *reinterpret_cast<f32x4*>(rec + R::kOffT + tid * 4) = v;
    }
    // the next v-head writes -A after its first barrier (every read of -A and T above is
    // behind one of this v-head's) and its gates went to the other buffer
  }
}

// ---- phase 2: per (sequence, v-head, block of 16 RT state rows), chunk by chunk --------
// Eight waves, two per SIMD.  State wave w (0..3) owns k tiles 2w and 2w + 1 of the block's
// S^T, forms V_new for tokens 16 w .. 16 w + 15 and updates its tiles; output wave w (4..7,
// tokens 16 (w - 4) ..) forms the raw outputs.  Each SIMD carries one of each, so one
// wave's waits (barriers, LDS, loads) leave the matrix core to the other.
// RT = 1 or 2 row tiles of 16 state rows per workgroup: each operand a wave loads feeds RT
// products, so with RT = 2 the chunk operands cross each CU half as often per product (for
// many sequences, where the workgroups are plentiful); RT = 1 has twice the workgroups, for
// few sequences, where the scan's latency is the time.
// Per chunk and SIMD: W S^T (32 RT products of 16 x 16 x 4) and P V_new (16 RT) in fp32;
// Qr S^T and the update as 12 RT bf16 products of 16 x 16 x 32 each (split operands), where
// in fp32 they took 32 RT each: 1,920 matrix cycles per chunk, SIMD and row tile, where
// all-fp32 products took 3,584.
constexpr int kScanThreads = 512;

// x = s1 + s2 + s3 exactly, in bf16 (each part the round-to-nearest-even of what the
// earlier ones leave, and every remainder exact in fp32: 8 + 8 + 8 bits of x's 24), so a
// product of an exact bf16 operand with x runs on the bf16 matrix cores as three products
// with exact terms and fp32 sums.  p[i] holds part i + 1 of four values.
struct Split4 {
  uint2 p[3];
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two values to a packed bf16 pair (round to nearest even, one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t bf16_pair(f32x2 v) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Each remainder r - s in one instruction: a dot product of the rounded pair with (-1, 0)
// or (0, -1) added to r (v_dot2c_f32_bf16; exact products, and the sum is r - s, which
// fp32 holds exactly).  (-1, 0) is set in an SGPR: as an operand the compiler encodes it
// as the inline constant -1.0, which this instruction reads as the fp32 word 0xbf800000,
// i.e. (0, -1).  Being an intrinsic, the first remainder also keeps a product passed as x
// rounded to fp32 (x - s1 written out would be contracted into an fma of its factors).
__device__ __forceinline__ Split4 split4(f32x4 x) {
  Split4 sp;
  uint32_t minus_lo_bits;
  asm("s_mov_b32 %0, 0xbf80" : "=s"(minus_lo_bits));
  const bf16x2 minus_lo = __builtin_bit_cast(bf16x2, minus_lo_bits);
  const bf16x2 minus_hi = __builtin_bit_cast(bf16x2, 0xbf800000u);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x2 r = {x[2 * j], x[2 * j + 1]};
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const uint32_t w = bf16_pair(r);
      (j == 0 ? sp.p[i].x : sp.p[i].y) = w;
      if (i < 2) {
        const bf16x2 s = __builtin_bit_cast(bf16x2, w);
        r = f32x2{__builtin_amdgcn_fdot2_f32_bf16(s, minus_lo, r.x, false),
                  __builtin_amdgcn_fdot2_f32_bf16(s, minus_hi, r.y, false)};
      }
    }
  }
  return sp;
}

template <int RT>
struct StateOperands {
  f32x4 w[8];      // W [16 w + li][32 lg + step]
  u32x4 kr[2][2];  // Kr^T [16 (2w + t) + li][16 lg + 8 qq + e] (bf16)
  f32x4 u[RT];     // U [16 w + 4 lg + r][row0 + 16 h + li]
  f32x4 ck;        // ck of tokens 16 w + 4 lg + r
  float gamma;     // exp(G_n-1)
};

struct OutputOperands {
  u32x4 qr[4];     // Qr [16 w + li][32 lg + 8 qq + e] (bf16)
  f32x4 sq;        // sq of tokens 16 w + 4 lg + r
  f32x4 p[4];      // P [16 w + li][16 lg + step]
};

// Buffer resource over one chunk record (raw, byte-addressed; word 3 = 0x00020000, the
// gfx9 raw-buffer format) and a 16-byte load at lane offset + uniform offset: the address
// stays a scalar resource plus one offset register, whatever the compiler's register
// pressure.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t record_resource(const float* r, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(r), 0, bytes, 0x00020000);
}

// The state tile of (slot, head) as a buffer resource: over its 64 KiB when the sequence
// starts from it, else over 0 bytes, whose loads return zeros without touching memory.  Its
// loads then need no branch and go out together (a branch per load, as `from_slot ? load :
// 0` compiles, waited for each load before the next was issued).  Callers pass the whole
// offset per lane, so the range check sees all of it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t state_resource(const DecodeParams& p, int slot,
                                                                 int head, bool from_slot) {
  // (uniform: readfirstlane keeps the resource in scalar registers, where a vector-held one
  // would put each load in a loop over its distinct values)
  return record_resource(
      p.state + static_cast<int64_t>(slot) * p.state_slot + static_cast<int64_t>(head) * kDim * kDim,
      __builtin_amdgcn_readfirstlane(from_slot ? kDim * kDim * 4 : 0));
}

// bf16 by the hardware's round-to-nearest-even conversion (v_cvt_pk_bf16_f32): the same
// value as f32_to_bf16 for every finite input
__device__ __forceinline__ uint16_t to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ f32x4 load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lane16,
                                        int byte_offset) {
  return __builtin_bit_cast(
      f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(lane16), byte_offset, 0));
}

__device__ __forceinline__ u32x4 load16u(__amdgpu_buffer_rsrc_t rsrc, uint32_t lane16,
                                         int byte_offset) {
  return __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(lane16), byte_offset, 0));
}

__device__ __forceinline__ float load4(__amdgpu_buffer_rsrc_t rsrc, int byte_offset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, 0, byte_offset, 0));
}

// The operand loads of one chunk come in pieces that the scan issues between its products,
// a few at a time (issued in one burst at the top of a chunk, the CU's 116 loads would hold
// every wave at the chunk's first barrier until the last of them was accepted).
// State piece q < 4: W columns q and q + 4 (with U, ck and gamma at q = 0); piece 4 + q:
// Kr of tile 2w + (q & 1), step groups 8 (q >> 1) ..  Output piece q < 4: Qr step groups
// 2q, 2q + 1 (with sq at q = 0); piece 4 + q (q < 2): P columns q and q + 2.  `tile0`: the
// workgroup's first 16-row tile of U; lg16 = 16 lg (the lane's 4 tokens of ck and sq).
template <int RT>
__device__ __forceinline__ void load_state_piece(StateOperands<RT>& o,
                                                 __amdgpu_buffer_rsrc_t rs, int own, int w,
                                                 uint32_t lane16, uint32_t lg16, int tile0,
                                                 int piece) {
  if (piece < 4) {
    const int wbase = own + static_cast<int>(kOffW * 4) + w * 8 * 1024;
    o.w[piece] = load16(rs, lane16, wbase + piece * 1024);
    o.w[piece + 4] = load16(rs, lane16, wbase + (piece + 4) * 1024);
    if (piece == 0) {
#pragma unroll
      for (int h = 0; h < RT; ++h)
        o.u[h] = load16(rs, lane16, own + static_cast<int>(kOffU * 4) + ((tile0 + h) * 4 + w) * 1024);
      o.ck = load16(rs, lg16, own + static_cast<int>((kOffMisc + kMiscCk) * 4) + w * 64);
      o.gamma = load4(rs, own + static_cast<int>(kOffMisc * 4));
    }
  } else {
    const int q = piece - 4;
    o.kr[q & 1][q >> 1] = load16u(
        rs, lane16, static_cast<int>(kOffKr * 4) + ((2 * w + (q & 1)) * 2 + (q >> 1)) * 1024);
  }
}

__device__ __forceinline__ void load_output_piece(OutputOperands& o, __amdgpu_buffer_rsrc_t rs,
                                                  int own, int w, uint32_t lane16,
                                                  uint32_t lg16, int piece) {
  if (piece < 4) {
    o.qr[piece] = load16u(rs, lane16, static_cast<int>(kOffQr * 4) + (w * 4 + piece) * 1024);
    if (piece == 0)
      o.sq = load16(rs, lg16, own + static_cast<int>((kOffMisc + kMiscSq) * 4) + w * 64);
  } else {
    const int pbase = own + static_cast<int>(kOffP * 4) + w * 4 * 1024;
    o.p[piece - 4] = load16(rs, lane16, pbase + (piece - 4) * 1024);
    o.p[piece - 2] = load16(rs, lane16, pbase + (piece - 2) * 1024);
  }
}

// A sched_barrier mask for the step groups of the scan: vector and scalar ALU and LDS
// instructions may be moved across, vector memory and matrix instructions stay in their
// group.  (Matrix instructions allowed across let the compiler hoist every product above
// the group's loads, which then went out at the end of the phase: 2.27 -> 2.06 ms at
// 32 x 1024 with the group kept, 0.32 -> 0.31 ms at 1 x 4096.)
constexpr int kLoadGroup = 0x386;

// Chunks 0 .. chunks - 1 through a ring of three operand sets: step(op, fill, c) computes
// chunk c from op and loads chunk c + 2 into fill.  Whole rounds of the ring run in a loop
// with no exit inside it, the last chunks after it.  (An exit between the steps of a round
// joins the loop's latch, and the wait counts at the loop head then follow that shorter
// path: the set prefetched for the next chunk was waited for a chunk early.)
template <class Step, class Operands>
__device__ __forceinline__ void ring_scan(Step& step, Operands& ring0, Operands& ring1,
                                          Operands& ring2, int chunks) {
  int c = 0;
  for (; c + 3 <= chunks; c += 3) {
    step(ring0, ring2, c);
    step(ring1, ring0, c + 1);
    step(ring2, ring1, c + 2);
  }
  if (c < chunks) {
    step(ring0, ring2, c);
    if (c + 1 < chunks) step(ring1, ring0, c + 1);
  }
}

// The products with an exact bf16 operand -- the update's Kr^T (V_new ck) and the outputs'
// Qr S^T -- run on the bf16 matrix cores as three products against the other operand's
// exact three-way split, which the state waves keep in LDS (S's planes beside its fp32
// values, V_new ck's planes beside V_new); W S^T and P V_new stay fp32.
template <int RT>
__global__ __launch_bounds__(kScanThreads)
void chunk_scan_kernel(const DecodeParams p, int num_sequences, float* ws,
                       const int32_t* chunk_start, int records) {
  constexpr int kRows = 16 * RT;              // state rows per workgroup
  constexpr int kBlocks = kDim / kRows;       // workgroups per (sequence, head)
  // Operand sets: three for one row tile (the whole set of chunk c + 2 loaded while chunk c
  // computes); one for two row tiles, refilled piece by piece half a chunk ahead (the Kr
  // pieces of chunk c during its V_new products, the W, U and gamma pieces of chunk c + 1
  // during its update), which leaves the registers for two workgroups per CU (1% faster
  // at 32 x 1024 than two sets a chunk ahead, which needed 162 VGPRs).
  constexpr int kSets = RT == 1 ? 3 : 1;
  constexpr bool kHalf = kSets == 1;
  // Workgroups go to the 8 XCDs round-robin by id.  The row blocks of one (sequence, head)
  // read the same chunk operands, so they are given ids on one XCD and share its L2:
  // id = ((pair / 8) * kBlocks + block) * 8 + pair % 8.  The grid is padded to whole groups
  // of 8 pairs.
  const int xcd = blockIdx.x & 7;
  const int rank = blockIdx.x >> 3;   // position among the XCD's workgroups
  const int pair = (rank / kBlocks) * 8 + xcd;
  if (pair >= num_sequences * p.num_v_heads) return;
  const int seq = pair / p.num_v_heads;
  const int head = pair - seq * p.num_v_heads;
  const int row_block = rank % kBlocks;
  const int row0 = row_block * kRows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // the wave index in a scalar register: every operand address is then a scalar base plus
  // the lane's offset, and the role test a scalar branch
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int lg = lane >> 4;
  const uint32_t lane16 = static_cast<uint32_t>(lane) * 16;
  const bool state_wave = wave < 4;
  const int w = wave & 3;
  const int bos = p.cu[seq];
  const int eos = p.cu[seq + 1];
  const int slot = p.indices[seq];
  const bool from_slot = slot > 0 && p.has_initial[seq] != 0;
  const int gbase = chunk_start[seq];
  // (bounded by the records the workspace holds, whatever cu_seqlens says)
  const int chunks = min((eos - bos + kC - 1) / kC, max(records - gbase, 0));

  constexpr int kSRow = kDim + 4;
  constexpr int kVRow = kC + 4;
  __shared__ __attribute__((aligned(16))) float sS[kRows][kSRow];   // S rows [row][k]
  __shared__ __attribute__((aligned(16))) float sVn[kRows][kVRow];  // V_new^T [row][token]
  // the three planes of V_new^T with token j times ck_j, and of S
  __shared__ __attribute__((aligned(16))) uint16_t sVk[3][kRows][kC + 8];     // rows of 144 B
  __shared__ __attribute__((aligned(16))) uint16_t sSp[3][kRows][kDim + 8];   // rows of 272 B

  // The operands of chunk c: through a resource over the records of the head's group (the
  // first v-head's record holds the group's Qr and Kr), the head's own at byte `own`.
  const int member = head % p.group;
  const int own = member * static_cast<int>(kRecord * 4);
  const int group_bytes = p.group * static_cast<int>(kRecord * 4);
  auto record = [&](int c) {
    return record_resource(
        ws + (static_cast<int64_t>(gbase + c) * p.num_v_heads + head - member) * kRecord,
        group_bytes);
  };
  // B fragments of S^T for k = 32 lg + step (step = 4 q + e), rows 16 h + li
  auto s_fragment = [&](int h, int q) {
    return *reinterpret_cast<const f32x4*>(&sS[16 * h + li][32 * lg + 4 * q]);
  };
  // B fragments of V_new for j = 16 lg + step, rows 16 h + li
  auto vn_fragment = [&](int h, int q) {
    return *reinterpret_cast<const f32x4*>(&sVn[16 * h + li][16 * lg + 4 * q]);
  };
  // the state waves' pieces of S to LDS: fp32, and the three planes
  auto put_state = [&](int t, int h, f32x4 v) __attribute__((always_inline)) {
    const int k = 16 * (2 * w + t) + 4 * lg;
    *reinterpret_cast<f32x4*>(&sS[16 * h + li][k]) = v;
    const Split4 sp = split4(v);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl) *reinterpret_cast<uint2*>(&sSp[pl][16 * h + li][k]) = sp.p[pl];
  };
  const uint32_t lg16 = static_cast<uint32_t>(lg) * 16;

  if (state_wave) {
    // st[t][h][r] = S[row0 + 16 h + li][16 (2w + t) + 4 lg + r]
    float* tile_base = p.state + static_cast<int64_t>(slot) * p.state_slot +
                       static_cast<int64_t>(head) * kDim * kDim + (row0 + li) * kDim;
    const __amdgpu_buffer_rsrc_t srs = state_resource(p, slot, head, from_slot);
    const uint32_t soff = static_cast<uint32_t>(((row0 + li) * kDim + 32 * w + 4 * lg) * 4);
    f32x4 st[2][RT];
#pragma unroll
    for (int h = 0; h < RT; ++h)
#pragma unroll
      for (int t = 0; t < 2; ++t) st[t][h] = load16(srs, soff + (16 * h * kDim + 16 * t) * 4, 0);
#pragma unroll
    for (int h = 0; h < RT; ++h)
#pragma unroll
      for (int t = 0; t < 2; ++t) put_state(t, h, st[t][h]);
    // Operands of later chunks are loaded while chunk c computes: into a ring of three
    // register sets (the loop is unrolled by three, so no set is copied: each is waited for
    // only where it is used), or into the one set as its pieces fall free.
    auto step = [&](const StateOperands<RT>& op, StateOperands<RT>& fill, int c) {
      // fill: unconditionally (the last chunk's record again past the end: a branch around
      // the loads would make the waits that follow conservative)
      const __amdgpu_buffer_rsrc_t next = record(min(c + (kHalf ? 1 : 2), chunks - 1));
      const __amdgpu_buffer_rsrc_t cur = kHalf ? record(c) : next;
      __syncthreads();  // sS holds the state at the chunk's start
      // two accumulation chains per row tile (k < 64, k >= 64 of each lane group) so that
      // consecutive matrix instructions do not wait on each other's results
      f32x4 vn0[RT], vn1[RT];
#pragma unroll
      for (int h = 0; h < RT; ++h) {
        vn0[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        vn1[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        load_state_piece(fill, cur, own, w, lane16, lg16, row_block * RT, kHalf ? 4 + q : q);
#pragma unroll
        for (int h = 0; h < RT; ++h) {
          const f32x4 b0 = s_fragment(h, q);
          const f32x4 b1 = s_fragment(h, q + 4);
          vn0[h] = mfma(op.w[q].x, b0.x, vn0[h]);
          vn1[h] = mfma(op.w[q + 4].x, b1.x, vn1[h]);
          vn0[h] = mfma(op.w[q].y, b0.y, vn0[h]);
          vn1[h] = mfma(op.w[q + 4].y, b1.y, vn1[h]);
          vn0[h] = mfma(op.w[q].z, b0.z, vn0[h]);
          vn1[h] = mfma(op.w[q + 4].z, b1.z, vn1[h]);
          vn0[h] = mfma(op.w[q].w, b0.w, vn0[h]);
          vn1[h] = mfma(op.w[q + 4].w, b1.w, vn1[h]);
        }
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
#pragma unroll
      for (int h = 0; h < RT; ++h) {
        const f32x4 vn = op.u[h] - (vn0[h] + vn1[h]);
        *reinterpret_cast<f32x4*>(&sVn[16 * h + li][16 * w + 4 * lg]) = vn;
        const Split4 sp = split4(vn * op.ck);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint2*>(&sVk[pl][16 * h + li][16 * w + 4 * lg]) = sp.p[pl];
      }
      __syncthreads();  // V_new complete; every read of sS for this chunk done
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int h = 0; h < RT; ++h) st[t][h] *= op.gamma;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        load_state_piece(fill, next, own, w, lane16, lg16, row_block * RT, kHalf ? q : 4 + q);
        // after every second piece, token block qq: Kr^T's tokens 16 lg + 8 qq + e (exact
        // bf16) against V_new ck's three planes, smallest first
        if (q & 1) {
          const int qq = q >> 1;
#pragma unroll
          for (int h = 0; h < RT; ++h) {
            bf16x8 vk[3];
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
              vk[pl] = *reinterpret_cast<const bf16x8*>(&sVk[pl][16 * h + li][16 * lg + 8 * qq]);
#pragma unroll
            for (int pl = 2; pl >= 0; --pl)
#pragma unroll
              for (int t = 0; t < 2; ++t)
                st[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, op.kr[t][qq]), vk[pl], st[t][h], 0, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
#pragma unroll
      for (int h = 0; h < RT; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t) put_state(t, h, st[t][h]);
    };
    // The first sets, piece by piece in the loop's order, so that the wait counts at the
    // loop head are the same from either side.
    auto prefill_set = [&](StateOperands<RT>& set, int c) {
      const __amdgpu_buffer_rsrc_t r = record(c);
#pragma unroll
      for (int piece = 0; piece < 8; ++piece) {
        load_state_piece(set, r, own, w, lane16, lg16, row_block * RT, piece);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    StateOperands<RT> ring0;
    if constexpr (kSets == 3) {
      StateOperands<RT> ring1, ring2;
      if (chunks > 0) {
        prefill_set(ring0, 0);
        prefill_set(ring1, min(1, chunks - 1));
      }
      ring_scan(step, ring0, ring1, ring2, chunks);
    } else {
      if (chunks > 0) {
        const __amdgpu_buffer_rsrc_t r = record(0);
#pragma unroll
        for (int piece = 0; piece < 4; ++piece) {
          load_state_piece(ring0, r, own, w, lane16, lg16, row_block * RT, piece);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      for (int c = 0; c < chunks; ++c) step(ring0, ring0, c);
    }
    if (slot > 0) {
#pragma unroll
      for (int h = 0; h < RT; ++h)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          *reinterpret_cast<f32x4*>(tile_base + 16 * h * kDim + 16 * (2 * w + t) + 4 * lg) =
              st[t][h];
    }
  } else {
    const int out_row = p.num_v_heads * kDim;   // elements per token row of out
    uint16_t* out_block = p.out + static_cast<int64_t>(head) * kDim + row0;
    auto step = [&](const OutputOperands& op, OutputOperands& fill, int c) {
      const __amdgpu_buffer_rsrc_t next = record(min(c + (kHalf ? 1 : 2), chunks - 1));
      const __amdgpu_buffer_rsrc_t cur = kHalf ? record(c) : next;
      __syncthreads();  // sS holds the state at the chunk's start
      f32x4 o0[RT], o1[RT];
#pragma unroll
      for (int h = 0; h < RT; ++h) {
        o0[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        o1[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (!kHalf)
          load_output_piece(fill, next, own, w, lane16, lg16, q);
        else if (q < 2)
          load_output_piece(fill, cur, own, w, lane16, lg16, 4 + q);   // P of this chunk
#pragma unroll
        for (int h = 0; h < RT; ++h) {
          // Qr's k = 32 lg + 8 q + e (exact bf16) against S's three planes, smallest first,
          // on two accumulation chains
          f32x4& o = (q & 1) ? o1[h] : o0[h];
#pragma unroll
          for (int pl = 2; pl >= 0; --pl)
            o = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, op.qr[q]),
                *reinterpret_cast<const bf16x8*>(&sSp[pl][16 * h + li][32 * lg + 8 * q]), o, 0, 0,
                0);
        }
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
      // rows of q S^T scaled to (q^ exp(G)) S^T; P V_new accumulates on top
#pragma unroll
      for (int h = 0; h < RT; ++h) {
        o0[h] = (o0[h] + o1[h]) * op.sq;
        o1[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      __syncthreads();  // V_new complete
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (!kHalf) {
          load_output_piece(fill, next, own, w, lane16, lg16, 4 + q);
        } else {   // Qr of the next chunk
          load_output_piece(fill, next, own, w, lane16, lg16, 2 * q);
          load_output_piece(fill, next, own, w, lane16, lg16, 2 * q + 1);
        }
#pragma unroll
        for (int h = 0; h < RT; ++h) {
          const f32x4 b0 = vn_fragment(h, q);
          const f32x4 b1 = vn_fragment(h, q + 2);
          o0[h] = mfma(op.p[q].x, b0.x, o0[h]);
          o1[h] = mfma(op.p[q + 2].x, b1.x, o1[h]);
          o0[h] = mfma(op.p[q].y, b0.y, o0[h]);
          o1[h] = mfma(op.p[q + 2].y, b1.y, o1[h]);
          o0[h] = mfma(op.p[q].z, b0.z, o0[h]);
          o1[h] = mfma(op.p[q + 2].z, b1.z, o1[h]);
          o0[h] = mfma(op.p[q].w, b0.w, o0[h]);
          o1[h] = mfma(op.p[q + 2].w, b1.w, o1[h]);
        }
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
      // raw outputs of tokens 16 w + 4 lg + r, column row0 + 16 h + li, through a buffer
      // over the chunk's rows of out: rows past the sequence's end fall outside it and are
      // dropped
      const int t0 = bos + c * kC;
      const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
          out_block + static_cast<int64_t>(t0) * out_row, 0, min(kC, eos - t0) * out_row * 2,
          0x00020000);
#pragma unroll
      for (int h = 0; h < RT; ++h) {
        const f32x4 o = o0[h] + o1[h];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          __builtin_amdgcn_raw_buffer_store_b16(
              to_bf16(o[r]), ors, ((16 * w + 4 * lg + r) * out_row + 16 * h + li) * 2, 0, 0);
      }
    };
    auto prefill_set = [&](OutputOperands& set, int c) {
      const __amdgpu_buffer_rsrc_t r = record(c);
#pragma unroll
      for (int piece = 0; piece < 6; ++piece) {
        load_output_piece(set, r, own, w, lane16, lg16, piece);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    OutputOperands ring0;
    if constexpr (kSets == 3) {
      OutputOperands ring1, ring2;
      if (chunks > 0) {
        prefill_set(ring0, 0);
        prefill_set(ring1, min(1, chunks - 1));
      }
      ring_scan(step, ring0, ring1, ring2, chunks);
    } else {
      if (chunks > 0) {
        const __amdgpu_buffer_rsrc_t r = record(0);
#pragma unroll
        for (int piece = 0; piece < 4; ++piece) {
          load_output_piece(ring0, r, own, w, lane16, lg16, piece);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      for (int c = 0; c < chunks; ++c) step(ring0, ring0, c);
    }
  }
}

// ---- phase 2, 32-token chunks: per (sequence, v-head, block of 32 state rows) ----------
// Eight waves, two per SIMD, each on one (token tile a, row tile h) = (w & 1, w >> 1) of the
// chunk.  State wave w (0..3): Y = K_a S_h^T from the bf16 keys, X = diag(beta) V -
// diag(ws) Y with V read from qkv; after a barrier V_new = T_a X_h (all 32 tokens of X);
// after another, the update of k tiles 2w and 2w + 1 of both row tiles.  Output wave 4 + w:
// the raw outputs of its tile.  Per chunk and SIMD the work of 112 products of 16 x 16 x 4
// for 32 tokens: the 96 of them with S or V_new ck as an operand run as 36 bf16 products of
// 16 x 16 x 32 against their exact three-way splits (a third of the matrix time), the other
// 16 (T X, P V_new) stay fp32.

struct Scan32State {
  u32x4 kq[4];  // Kq [16 a + li][32 lg + 8 qq + e] (bf16)
  f32x4 beta;   // beta of tokens 16 a + 4 lg + r
  f32x4 ws;     // ws of tokens 16 a + 4 lg + r
  uint16_t v[4];  // V [16 a + 4 lg + r][row0 + 16 h + li] (bf16)
  f32x4 t[2];   // T [16 a + li][8 lg + 4 q + e]
  f32x4 ck;     // ck of tokens 16 a + 4 lg + r
  u32x4 kr[2];  // Kr^T [16 (2w + t) + li][8 lg + e] (bf16)
  float gamma;  // exp(G_n-1)
};

struct Scan32Output {
  u32x4 qr[4];  // Qr [16 a + li][32 lg + 8 qq + e] (bf16)
  f32x4 sq;     // sq of tokens 16 a + 4 lg + r
  f32x4 p[2];   // P [16 a + li][8 lg + 4 q + e]
};

// The operand loads in pieces, as in chunk_scan_kernel.  State wave: piece 0 (Kq, beta, ws
// and v: the first products) and piece 1 (T and ck: V_new) of the next chunk during the
// update, piece 2 (Kr and gamma: the update) during this chunk's first products.  Output
// wave: piece 2 (P) of this chunk during its q S^T products, pieces 0 and 1 (Qr, sq) of the
// next during P V_new.  `vs`: a resource over the chunk's rows of qkv, `voff` the lane's
// byte offset of V[16 a + 4 lg][row0 + 16 h + li] in it.
__device__ __forceinline__ void load_state32(Scan32State& o, __amdgpu_buffer_rsrc_t rs,
                                             __amdgpu_buffer_rsrc_t vs, uint32_t voff,
                                             uint32_t vrow, int own, int w, int a,
                                             uint32_t lane16, uint32_t lg16, int piece) {
  using R = Rec32;
  if (piece == 0) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
      o.kq[qq] = load16u(rs, lane16, static_cast<int>(R::kOffKq * 4) + (a * 4 + qq) * 1024);
    o.beta = load16(rs, lg16, own + static_cast<int>((R::kOffMisc + kMiscBeta) * 4) + a * 64);
    o.ws = load16(rs, lg16, own + static_cast<int>((R::kOffMisc + kMiscWs) * 4) + a * 64);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o.v[r] = __builtin_amdgcn_raw_buffer_load_b16(vs, static_cast<int>(voff + r * vrow), 0, 0);
  } else if (piece == 1) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      o.t[q] = load16(rs, lane16, own + static_cast<int>(R::kOffT * 4) + (a * 2 + q) * 1024);
    o.ck = load16(rs, lg16, own + static_cast<int>((R::kOffMisc + kMiscCk) * 4) + a * 64);
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t)
      o.kr[t] = load16u(rs, lane16, static_cast<int>(R::kOffKr * 4) + (2 * w + t) * 1024);
    o.gamma = load4(rs, own + static_cast<int>(R::kOffMisc * 4));
  }
}

__device__ __forceinline__ void load_output32(Scan32Output& o, __amdgpu_buffer_rsrc_t rs, int own,
                                              int a, uint32_t lane16, uint32_t lg16, int piece) {
  using R = Rec32;
  if (piece < 2) {
#pragma unroll
    for (int e = 0; e < 2; ++e)
      o.qr[2 * piece + e] =
          load16u(rs, lane16, static_cast<int>(R::kOffQr * 4) + (a * 4 + 2 * piece + e) * 1024);
    if (piece == 0)
      o.sq = load16(rs, lg16, own + static_cast<int>((R::kOffMisc + kMiscSq) * 4) + a * 64);
  } else {
#pragma unroll
    for (int q = 0; q < 2; ++q)
      o.p[q] = load16(rs, lane16, own + static_cast<int>(R::kOffP * 4) + (a * 2 + q) * 1024);
  }
}

// The products with S and with V_new ck on the bf16 matrix cores, each as three products
// against split4's parts (fp32-exact operands, fp32 sums, 80 VGPRs).  (Prompts of one
// chunk once kept fp32 products, before the splits took one instruction per remainder.)
__global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(6)))
void chunk_scan32_kernel(const DecodeParams p, int num_sequences, float* ws,
                         const int32_t* chunk_start, int records) {
  using R = Rec32;
  constexpr int kCs = R::kC;                 // 32 tokens per chunk
  constexpr int kRows = 32;                  // state rows per workgroup
  constexpr int kBlocks = kDim / kRows;
  // XCD-aware ids as in chunk_scan_kernel: the 4 row blocks of one (sequence, head) on one XCD
  const int xcd = blockIdx.x & 7;
  const int rank = blockIdx.x >> 3;
  const int pair = (rank / kBlocks) * 8 + xcd;
  if (pair >= num_sequences * p.num_v_heads) return;
  const int seq = pair / p.num_v_heads;
  const int head = pair - seq * p.num_v_heads;
  const int row_block = rank % kBlocks;
  const int row0 = row_block * kRows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int lg = lane >> 4;
  const uint32_t lane16 = static_cast<uint32_t>(lane) * 16;
  const uint32_t lg16 = static_cast<uint32_t>(lg) * 16;
  const int w = wave & 3;
  const int a = w & 1;    // the wave's token tile
  const int h = w >> 1;   // the wave's row tile
  const int bos = p.cu[seq];
  const int eos = p.cu[seq + 1];
  const int slot = p.indices[seq];
  const bool from_slot = slot > 0 && p.has_initial[seq] != 0;
  const int gbase = chunk_start[seq];
  const int chunks = min((eos - bos + kCs - 1) / kCs, max(records - gbase, 0));

  constexpr int kVRow = kCs + 4;    // fp32 row of V_new or X
  // S [row][k] and V_new with its rows scaled by ck [row][token] as three bf16 planes each
  // (split4: their sum is the fp32 value exactly); V_new and X in fp32 for the fp32 products
  __shared__ __attribute__((aligned(16))) uint16_t sS[3][32][kDim + 8];   // rows of 272 bytes
  __shared__ __attribute__((aligned(16))) uint16_t sVk[3][32][32 + 8];
  __shared__ __attribute__((aligned(16))) float sVn[kRows][kVRow];   // V_new^T [row][token]
  __shared__ __attribute__((aligned(16))) float sX[kRows][kVRow];    // X^T [row][token]

  const int member = head % p.group;
  const int own = member * static_cast<int>(R::kSize * 4);
  const int group_bytes = p.group * static_cast<int>(R::kSize * 4);
  // chunk c's records; past the last chunk a resource over 0 bytes, whose loads return
  // zeros without touching memory (the refills stay unconditional, so the waits that follow
  // them stay exact)
  auto record = [&](int c) {
    return record_resource(
        ws + (static_cast<int64_t>(gbase + min(c, chunks - 1)) * p.num_v_heads + head - member) *
                 R::kSize,
        c < chunks ? group_bytes : 0);
  };
  // X_a S_h^T for bf16 rows X, the lane's values k = 32 lg + 8 qq .. + 7 in x[qq], row
  // 16 h + li of S: instruction qq of a bf16 product takes those 8 values against each of
  // S's planes, smallest first; `load()` issues operand loads ahead of the products.
  auto times_st = [&](const u32x4 (&x)[4], auto&& load) __attribute__((always_inline)) {
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    load();
    __builtin_amdgcn_sched_barrier(kLoadGroup);
#pragma unroll
    for (int pl = 2; pl >= 0; --pl)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, x[qq]),
            *reinterpret_cast<const bf16x8*>(&sS[pl][16 * h + li][32 * lg + 8 * qq]), acc, 0, 0,
            0);
    return acc;
  };
  // chunk c's rows of qkv (0 bytes past the last chunk, or a sequence's rows past its end:
  // their v reads as zeros), and the lane's offset of v[16 a + 4 lg][row0 + 16 h + li] in it
  const int v_col = (2 * p.num_k_heads + head) * kDim + row0 + 16 * h + li;
  auto v_rows = [&](int c) {
    const int t0 = bos + min(c, max(chunks - 1, 0)) * kCs;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.qkv + static_cast<int64_t>(t0) * p.qkv_row), 0,
        c < chunks ? min(kCs, eos - t0) * static_cast<int>(p.qkv_row) * 2 : 0, 0x00020000);
  };
  const uint32_t vrow = static_cast<uint32_t>(p.qkv_row) * 2;
  const uint32_t voff = (16 * a + 4 * lg) * vrow + static_cast<uint32_t>(v_col) * 2;

  if (wave < 4) {
    // The wave's pieces of the state, S[row0 + 16 hh + li][16 (2w + t) + 4 lg + r], live in
    // sS between chunks, in its planes: split on the way in and summed on the way out,
    // exactly.
    auto put_own = [&](int t, int hh, f32x4 v) __attribute__((always_inline)) {
      const int k = 16 * (2 * w + t) + 4 * lg;
      const Split4 sp = split4(v);
#pragma unroll
      for (int pl = 0; pl < 3; ++pl) *reinterpret_cast<uint2*>(&sS[pl][16 * hh + li][k]) = sp.p[pl];
    };
    // The identity in the A layout of v_mfma_f32_16x16x16_bf16 (lane (li, lg): row
    // li, columns 4 lg .. 4 lg + 3), so that I B hands each lane its own four B values:
    // three such products sum the planes in fp32, (s1 + s2) + s3, exactly (every partial
    // sum is the value less a tail it lacks), on the matrix pipe instead of 20 VALU
    // instructions per piece
    const uint32_t one_at = static_cast<uint32_t>(li - 4 * lg);
    const bf16v4 ident = __builtin_bit_cast(
        bf16v4, one_at < 4 ? 0x3f80ull << (16 * one_at) : 0ull);
    auto get_own = [&](int t, int hh) __attribute__((always_inline)) {
      const int k = 16 * (2 * w + t) + 4 * lg;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int pl = 0; pl < 3; ++pl)
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            ident, *reinterpret_cast<const bf16v4*>(&sS[pl][16 * hh + li][k]), acc, 0, 0, 0);
      return acc;
    };
    // the first chunk's pieces 0 and 1 go out before the state's loads, so that their
    // latencies overlap (the state is waited for first, to reach sS)
    Scan32State op;
    if (chunks > 0) {
      const __amdgpu_buffer_rsrc_t r = record(0);
      const __amdgpu_buffer_rsrc_t vr = v_rows(0);
#pragma unroll
      for (int piece = 0; piece < 2; ++piece) {
        load_state32(op, r, vr, voff, vrow, own, w, a, lane16, lg16, piece);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    {
      const __amdgpu_buffer_rsrc_t srs = state_resource(p, slot, head, from_slot);
      const uint32_t soff = static_cast<uint32_t>(((row0 + li) * kDim + 32 * w + 4 * lg) * 4);
      f32x4 st[2][2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int t = 0; t < 2; ++t) st[t][hh] = load16(srs, soff + (16 * hh * kDim + 16 * t) * 4, 0);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int t = 0; t < 2; ++t) put_own(t, hh, st[t][hh]);
    }
    // The state's final pieces straight to the tile (through its resource; the lane's offset
    // formed anew from the lane count, mbcnt, as a work-item id or offset held across the
    // chunk loop took a register that loop needs: a spill).
    auto store_own = [&](int t, int hh, f32x4 v) __attribute__((always_inline)) {
      const int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
      const __amdgpu_buffer_rsrc_t srs = state_resource(p, slot, head, true);
      const uint32_t soff =
          static_cast<uint32_t>(((row0 + (l & 15)) * kDim + 32 * w + 4 * (l >> 4)) * 4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), srs,
                                             static_cast<int>(soff + (16 * hh * kDim + 16 * t) * 4),
                                             0, 0);
    };
    // One chunk; the last one's updated pieces go to the tile instead of through sS's planes
    // (nothing reads them there again), which spares prompts of one chunk a split and a sum
    // per piece.
    auto chunk = [&](int c, auto last) __attribute__((always_inline)) {
      const __amdgpu_buffer_rsrc_t cur = record(c);
      const __amdgpu_buffer_rsrc_t next = record(c + 1);
      const __amdgpu_buffer_rsrc_t vnext = v_rows(c + 1);
      __syncthreads();  // sS holds the state at the chunk's start
      // Y = K_a S_h^T (this chunk's Kr and gamma loaded beside it)
      const f32x4 y = times_st(op.kq, [&]() {
        load_state32(op, cur, vnext, voff, vrow, own, w, a, lane16, lg16, 2);
      });
      // X = diag(beta) V - diag(ws) Y for tokens 16 a + 4 lg + r, row 16 h + li (beta and ws
      // are zero past the chunk's end, and so is v)
      {
        f32x4 x;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = op.beta[r] * bf16_to_f32(op.v[r]) - op.ws[r] * y[r];
        *reinterpret_cast<f32x4*>(&sX[16 * h + li][16 * a + 4 * lg]) = x;
      }
      __syncthreads();  // X complete
      // V_new = T_a X_h over the chunk's 32 tokens j = 8 lg + 4 q + e
      f32x4 vn0 = {0.0f, 0.0f, 0.0f, 0.0f};
      f32x4 vn1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(&sX[16 * h + li][8 * lg + 4 * q]);
        f32x4& vn = q == 0 ? vn0 : vn1;
        vn = mfma(op.t[q].x, b.x, vn);
        vn = mfma(op.t[q].y, b.y, vn);
        vn = mfma(op.t[q].z, b.z, vn);
        vn = mfma(op.t[q].w, b.w, vn);
      }
      const f32x4 vn = vn0 + vn1;
      *reinterpret_cast<f32x4*>(&sVn[16 * h + li][16 * a + 4 * lg]) = vn;
      {
        const Split4 sp = split4(vn * op.ck);
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          *reinterpret_cast<uint2*>(&sVk[pl][16 * h + li][16 * a + 4 * lg]) = sp.p[pl];
      }
      __syncthreads();  // V_new complete; every read of sS for this chunk done
      // the update: Kr^T (exact bf16; the lane's k row 16 (2w + t) + li, tokens
      // j = 8 lg + e) against V_new ck (tokens j, rows 16 hh + li); the next chunk's
      // pieces 0 and 1 loaded beside it
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        load_state32(op, next, vnext, voff, vrow, own, w, a, lane16, lg16, hh);
        // V_new ck's three planes, smallest first
        bf16x8 vk[3];
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
          vk[pl] = *reinterpret_cast<const bf16x8*>(&sVk[pl][16 * hh + li][8 * lg]);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          f32x4 st = get_own(t, hh) * op.gamma;
#pragma unroll
          for (int pl = 2; pl >= 0; --pl)
            st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, op.kr[t]),
                                                         vk[pl], st, 0, 0, 0);
          if constexpr (decltype(last)::value) {
            if (slot > 0) store_own(t, hh, st);
          } else {
            put_own(t, hh, st);
          }
        }
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
    };
    for (int c = 0; c + 1 < chunks; ++c) chunk(c, std::false_type{});
    if (chunks > 0) {
      chunk(chunks - 1, std::true_type{});
    } else if (slot > 0) {
      // no chunk: the state as it came in (zeros for a sequence that does not start from
      // its slot; its LDS accesses complete in order, so no barrier is needed)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int t = 0; t < 2; ++t) store_own(t, hh, get_own(t, hh));
    }
  } else {
    const int out_row = p.num_v_heads * kDim;   // elements per token row of out
    uint16_t* out_block = p.out + static_cast<int64_t>(head) * kDim + row0;
    Scan32Output op;
    if (chunks > 0) {
      const __amdgpu_buffer_rsrc_t r = record(0);
#pragma unroll
      for (int piece = 0; piece < 2; ++piece) {
        load_output32(op, r, own, a, lane16, lg16, piece);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    for (int c = 0; c < chunks; ++c) {
      const __amdgpu_buffer_rsrc_t cur = record(c);
      const __amdgpu_buffer_rsrc_t next = record(c + 1);
      __syncthreads();  // sS holds the state at the chunk's start
      f32x4 o0 = times_st(op.qr, [&]() {   // P of this chunk beside it
        load_output32(op, cur, own, a, lane16, lg16, 2);
      });
      // rows of q S^T scaled to (q^ exp(G)) S^T; P V_new accumulates on top
      o0 = o0 * op.sq;
      f32x4 o1 = {0.0f, 0.0f, 0.0f, 0.0f};
      __syncthreads();  // X complete
      __syncthreads();  // V_new complete
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        load_output32(op, next, own, a, lane16, lg16, q);   // Qr and sq of the next chunk
        // V_new for tokens j = 8 lg + 4 q + e, rows 16 h + li
        const f32x4 b = *reinterpret_cast<const f32x4*>(&sVn[16 * h + li][8 * lg + 4 * q]);
        f32x4& o = q == 0 ? o0 : o1;
        o = mfma(op.p[q].x, b.x, o);
        o = mfma(op.p[q].y, b.y, o);
        o = mfma(op.p[q].z, b.z, o);
        o = mfma(op.p[q].w, b.w, o);
        __builtin_amdgcn_sched_barrier(kLoadGroup);
      }
      // raw outputs of tokens 16 a + 4 lg + r, column row0 + 16 h + li (rows past the
      // sequence's end fall outside the buffer and are dropped)
      const int t0 = bos + c * kCs;
      const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
          out_block + static_cast<int64_t>(t0) * out_row, 0, min(kCs, eos - t0) * out_row * 2,
          0x00020000);
      const f32x4 o = o0 + o1;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_raw_buffer_store_b16(
            to_bf16(o[r]), ors, ((16 * a + 4 * lg + r) * out_row + 16 * h + li) * 2, 0, 0);
    }
  }
}

template <int C>
int64_t max_chunks(int64_t num_tokens, int64_t num_sequences) {
  return num_tokens / C + num_sequences;  // each sequence adds at most one partial chunk
}

// Workspace: the records, then chunk_start (num_sequences + 1 int32, rounded up to 256 B).
// Sized for 64-token chunks, which covers 32-token ones: with S >= 1 sequences,
// (T / 32 + S) R32 <= (2 (T / 64) + 1 + S) R32 <= (T / 64 + S) R64 as 2 R32 <= R64.
static_assert(2 * Rec32::kSize <= kRecord, "32-token records fit the workspace");
int64_t records_bytes(int64_t num_tokens, int64_t num_sequences, int64_t num_v_heads) {
  return max_chunks<kC>(num_tokens, num_sequences) * num_v_heads * kRecord * 4;
}

template <int TT>
int launch_chunks(const DecodeParams& p, int num_sequences, int64_t num_tokens, bool dt_bf16,
                  float* ws, int32_t* chunk_start, hipStream_t stream) {
  constexpr int kCt = TT == 2 ? Rec32::kC : kC;
  const int64_t chunks = max_chunks<kCt>(num_tokens, num_sequences);
  if (chunks > 0x7fffffff || p.num_v_heads > 65535)
    return fail(LD_ERR_INVALID_ARGUMENT, "prefill too large for the chunked form");
  // one workgroup per (chunk, k-head)
  const int64_t prep_groups = chunks * p.num_k_heads;
  if (prep_groups > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "prefill too large");
  const dim3 per_chunk(static_cast<uint32_t>(prep_groups));
  hipLaunchKernelGGL(chunk_index_kernel<kCt>, dim3(1), dim3(kThreads), 0, stream, p.cu,
                     num_sequences, chunk_start);
  // 16-byte pieces of q and k (and v) when every row starts at a 16-byte boundary
  const bool wide = (reinterpret_cast<uintptr_t>(p.qkv) & 15) == 0 && (p.qkv_row & 7) == 0;
#define LD_PREP_LAUNCH(K, D, W, N)                                                             \
  hipLaunchKernelGGL((K<D, W>), per_chunk, dim3(N), 0, stream, p, num_sequences, ws,          \
                     chunk_start, static_cast<int>(chunks))
#define LD_PREP_LAUNCHES(K, N)                                                                 \
  if (dt_bf16) {                                                                               \
    if (wide)                                                                                  \
      LD_PREP_LAUNCH(K, true, true, N);                                                        \
    else                                                                                       \
      LD_PREP_LAUNCH(K, true, false, N);                                                       \
  } else {                                                                                     \
    if (wide)                                                                                  \
      LD_PREP_LAUNCH(K, false, true, N);                                                       \
    else                                                                                       \
      LD_PREP_LAUNCH(K, false, false, N);                                                      \
  }
  if constexpr (TT == 2) {
    LD_PREP_LAUNCHES(chunk_prep32_kernel, kPrep32Threads)
  } else {
    LD_PREP_LAUNCHES(chunk_prep_kernel, kPrepThreads)
  }
#undef LD_PREP_LAUNCHES
#undef LD_PREP_LAUNCH
  const int64_t pairs = static_cast<int64_t>(num_sequences) * p.num_v_heads;
  if constexpr (TT == 2) {
    const int64_t scan_groups = (pairs + 7) / 8 * 8 * (kDim / 32);
    if (scan_groups > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "prefill too large");
    hipLaunchKernelGGL(chunk_scan32_kernel, dim3(static_cast<uint32_t>(scan_groups)),
                       dim3(kScanThreads), 0, stream, p, num_sequences, ws, chunk_start,
                       static_cast<int>(chunks));
  } else {
    // two row tiles per workgroup once they still give 2 workgroups per CU
    const bool two_tiles = pairs * (kDim / 32) >= 512;
    const int64_t scan_groups = (pairs + 7) / 8 * 8 * (two_tiles ? kDim / 32 : kDim / 16);
    if (scan_groups > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "prefill too large");
    if (two_tiles)
      hipLaunchKernelGGL(chunk_scan_kernel<2>, dim3(static_cast<uint32_t>(scan_groups)),
                         dim3(kScanThreads), 0, stream, p, num_sequences, ws, chunk_start,
                         static_cast<int>(chunks));
    else
      hipLaunchKernelGGL(chunk_scan_kernel<1>, dim3(static_cast<uint32_t>(scan_groups)),
                         dim3(kScanThreads), 0, stream, p, num_sequences, ws, chunk_start,
                         static_cast<int>(chunks));
  }
  return check_launch("ld_gdn_prefill (chunked)");
}

}  // namespace

int64_t prefill_chunked_workspace_bytes(int64_t num_tokens, int64_t num_sequences,
                                        int64_t num_v_heads) {
  return records_bytes(num_tokens, num_sequences, num_v_heads) +
         ((num_sequences + 1) * 4 + 255) / 256 * 256;
}

int launch_prefill_chunked(const DecodeParams& p, int num_sequences, int64_t num_tokens,
                           bool dt_bf16, int chunk_tokens, void* workspace, hipStream_t stream) {
  float* ws = static_cast<float*>(workspace);
  int32_t* chunk_start = reinterpret_cast<int32_t*>(
      static_cast<char*>(workspace) + records_bytes(num_tokens, num_sequences, p.num_v_heads));
  if (chunk_tokens == 32)
    return launch_chunks<2>(p, num_sequences, num_tokens, dt_bf16, ws, chunk_start, stream);
  return launch_chunks<4>(p, num_sequences, num_tokens, dt_bf16, ws, chunk_start, stream);
}

}  // namespace ld
