// Chunked prefill for gfx950: the delta rule over chunks of 64 tokens in the WY form, for
// prompts too few to fill the GPU with one token-serial workgroup per (sequence, head).
//
// Per chunk (tokens i = 0 .. n-1, n <= 64), with g_i the log decay, G_i = g_0 + .. + g_i,
// Gam_ij = exp(G_i - G_j), beta_i, normalised q^_i (scaled) and k^_i, and S the state at
// the chunk's start ([V, K], row v):
//   A_im = beta_i Gam_im (k^_i . k^_m) for m < i            (strictly lower, 64 x 64)
//   (I + A) W = rows beta_i exp(G_i) k^_i,  (I + A) U = rows beta_i v_i   (forward subst.)
//   V_new = U - W S^T                                        (64 x 128)
//   O     = (q^_i exp(G_i)) S^T + P V_new,  P_ij = Gam_ij (q^_i . k^_j) for j <= i
//   S'    = exp(G_{n-1}) S + V_new^T (k^_j exp(G_{n-1} - G_j))
// which equals the token-by-token recurrence of the decode kernel (checked against it in
// float64: 7e-8 relative on the state).  Three launches:
//   chunk_prep_kernel  one workgroup per (chunk, v-head), all chunks in parallel: norms,
//                      gates, A, the forward substitution for W and U, P, and the scaled
//                      q and k; everything to a workspace record.
//   chunk_scan_kernel  one workgroup per (sequence, v-head, block of 16 state rows), the only
//                      sequential part: chunk by chunk, V_new and the state update, saving
//                      the state at each chunk's start; rows evolve independently, so a
//                      head's 128 rows spread over 8 workgroups.
//   chunk_out_kernel   one workgroup per (chunk, v-head), in parallel: the raw outputs,
//                      rounded to bf16 into `out` (the reference's rounding point before the
//                      gated RMSNorm, which prefill_norm_kernel applies afterwards).
// All arithmetic is fp32 on the vector ALUs, with operands staged in LDS.
#include "gdn_common.h"

namespace ld {
namespace {

constexpr int kC = 64;                          // tokens per chunk
constexpr int kScanRows = 16;                   // state rows per scan workgroup
constexpr int kScanBlocks = kDim / kScanRows;   // scan workgroups per (sequence, head)

// Workspace record of one (chunk, v-head), offsets in floats.
constexpr int64_t kOffWT = 0;                        // W^T   [128][64]
constexpr int64_t kOffU = kOffWT + kDim * kC;        // U     [64][128]
constexpr int64_t kOffQT = kOffU + kC * kDim;        // Qg^T  [128][64]  q^_i exp(G_i)
constexpr int64_t kOffKd = kOffQT + kDim * kC;       // Kd    [64][128]  k^_j exp(G_n-1 - G_j)
constexpr int64_t kOffPT = kOffKd + kC * kDim;       // P^T   [64][64]
constexpr int64_t kOffVn = kOffPT + kC * kC;         // V_new [64][128]
constexpr int64_t kOffH = kOffVn + kC * kDim;        // H     [128][128] state at chunk start
constexpr int64_t kOffMisc = kOffH + kDim * kDim;    // [0] exp(G_n-1)
constexpr int64_t kRecord = kOffMisc + 64;           // floats (a multiple of 64: 256 B)

// Chunks of sequence n start at chunk_base(n) = sum over m < n of ceil(L_m / 64).
__device__ int chunk_base(const int32_t* cu, int n) {
  int base = 0;
  for (int m = 0; m < n; ++m) base += (cu[m + 1] - cu[m] + kC - 1) / kC;
  return base;
}

// Global chunk g -> (sequence, first row, tokens); false past the last chunk.
__device__ bool find_chunk(const int32_t* cu, int num_sequences, int g, int& seq, int& t0,
                           int& len) {
  int base = 0;
  for (int n = 0; n < num_sequences; ++n) {
    const int b = cu[n];
    const int e = cu[n + 1];
    const int chunks = (e - b + kC - 1) / kC;
    if (g < base + chunks) {
      seq = n;
      t0 = b + (g - base) * kC;
      len = min(kC, e - t0);
      return true;
    }
    base += chunks;
  }
  return false;
}

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  float acc = a.x * b.x;
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  return fmaf(a.w, b.w, acc);
}

// ---- phase 1: per (chunk, v-head) ----------------------------------------------------
template <bool DtBf16>
__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(const DecodeParams p,
                                                              int num_sequences, float* ws) {
  const int head = blockIdx.y;
  int seq = 0, t0 = 0, len = 0;
  if (!find_chunk(p.cu, num_sequences, blockIdx.x, seq, t0, len)) return;
  float* rec = ws + (static_cast<int64_t>(blockIdx.x) * p.num_v_heads + head) * kRecord;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int key_head = head / p.group;
  const int q_col = key_head * kDim;
  const int k_col = (p.num_k_heads + key_head) * kDim;
  const int v_col = (2 * p.num_k_heads + head) * kDim;

  constexpr int kRow = kDim + 4;   // padded LDS row (floats) of q^ and k^
  constexpr int kARow = kC + 4;    // padded LDS row of A^T (16-byte aligned)
  __shared__ float sQ[kC][kRow];
  __shared__ float sK[kC][kRow];
  __shared__ float sAt[kC][kARow];  // A^T: [m][i]
  __shared__ float sG[kC];
  __shared__ float sBeta[kC];
  __shared__ float sEg[kC];     // exp(G_i)
  __shared__ float sEk[kC];     // exp(G_n-1 - G_i)

  // q^ and k^ of the chunk's tokens (zero rows past its end); wave w does tokens
  // 16w .. 16w+15, all 16 tokens' loads in flight before the first norm
  {
    uint16_t qr[16][2], kr[16][2];
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      const int64_t tok = t0 + min(wave * 16 + ii, len - 1);
      const uint16_t* row = p.qkv + tok * p.qkv_row;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        qr[ii][e] = row[q_col + 2 * lane + e];
        kr[ii][e] = row[k_col + 2 * lane + e];
      }
    }
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
      const int i = wave * 16 + ii;
      float q[2], k[2];
      float qq = 0.0f, kk = 0.0f;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        q[e] = bf16_to_f32(qr[ii][e]);
        k[e] = bf16_to_f32(kr[ii][e]);
        qq = fmaf(q[e], q[e], qq);
        kk = fmaf(k[e], k[e], kk);
      }
      qq = wave_sum(qq);
      kk = wave_sum(kk);
      const bool live = i < len;
      const float rq = fast_rsqrt(qq + 1e-6f);
      const float rk = fast_rsqrt(kk + 1e-6f);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        sQ[i][2 * lane + e] = live ? (q[e] * rq) * p.scale : 0.0f;
        sK[i][2 * lane + e] = live ? k[e] * rk : 0.0f;
      }
    }
  }
  // gates and the in-chunk cumulative log decay (wave 0, lane = token)
  if (wave == 0) {
    const bool live = lane < len;
    const int64_t tok = t0 + min(lane, len - 1);
    const float dt_bias = load_param(p.dt_bias, head, DtBf16);
    const float x = bf16_to_f32(p.a[tok * p.a_row + head]) + dt_bias;
    const float g = live ? -__expf(p.a_log[head]) * softplus(x) : 0.0f;
    const float beta = live ? sigmoid(bf16_to_f32(p.b[tok * p.b_row + head])) : 0.0f;
    float G = g;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float up = __shfl_up(G, d);
      if (lane >= d) G += up;
    }
    const float glast = __shfl(G, len - 1);
    sG[lane] = G;
    sBeta[lane] = beta;
    sEg[lane] = __expf(G);
    sEk[lane] = __expf(glast - G);
    if (lane == 0) rec[kOffMisc] = __expf(glast);
  }
  __syncthreads();

  // A (strictly lower) and P (lower, diagonal included) in 4 x 4 blocks: thread (ib, mb) owns
  // rows 4 ib .. 4 ib + 3 and columns 4 mb .. 4 mb + 3.  A is kept transposed for the
  // substitution; P goes to the workspace transposed.
  const int ib = tid >> 4;
  const int mb = tid & 15;
  {
    f32x4 aa[4], pp[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) aa[r] = pp[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (mb <= ib) {
#pragma unroll 2
      for (int kb = 0; kb < kDim; kb += 4) {
        f32x4 km[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) km[c] = *reinterpret_cast<const f32x4*>(&sK[4 * mb + c][kb]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f32x4 ki = *reinterpret_cast<const f32x4*>(&sK[4 * ib + r][kb]);
          const f32x4 qi = *reinterpret_cast<const f32x4*>(&sQ[4 * ib + r][kb]);
          aa[r] += f32x4{dot4(ki, km[0]), dot4(ki, km[1]), dot4(ki, km[2]), dot4(ki, km[3])};
          pp[r] += f32x4{dot4(qi, km[0]), dot4(qi, km[1]), dot4(qi, km[2]), dot4(qi, km[3])};
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 4 * ib + r;
      const float gi = sG[i];
      const float bi = sBeta[i];
      const bool live = i < len;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int m = 4 * mb + c;
        const float gam = __expf(gi - sG[m]);
        sAt[m][i] = m < i ? bi * gam * aa[r][c] : 0.0f;
        rec[kOffPT + m * kC + i] = (live && m <= i) ? gam * pp[r][c] : 0.0f;
      }
    }
  }
  __syncthreads();

  // forward substitution, one column per thread: W (threads 0..127) and U (128..255).
  // Column form: once x[m] is final, its multiple of A[i][m] leaves every later x[i] -- the
  // updates of one step are independent.
  {
    const int c = tid & (kDim - 1);
    const bool is_u = tid >= kDim;
    // every lane loads its v column (W lanes too: the select below keeps the loads free of
    // branches, so all 64 are in flight together)
    uint16_t vr[kC];
#pragma unroll
    for (int i = 0; i < kC; ++i) vr[i] = p.qkv[(t0 + min(i, len - 1)) * p.qkv_row + v_col + c];
    float x[kC];
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const float w = sEg[i] * sK[i][c];
      x[i] = sBeta[i] * (is_u ? bf16_to_f32(vr[i]) : w);  // beta = 0 past the end
    }
#pragma unroll
    for (int m = 0; m < kC - 1; ++m) {
      const float xm = x[m];
#pragma unroll
      for (int i4 = (m + 1) & ~3; i4 < kC; i4 += 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(&sAt[m][i4]);
        if (i4 > m) x[i4] = fmaf(-a.x, xm, x[i4]);
        if (i4 + 1 > m) x[i4 + 1] = fmaf(-a.y, xm, x[i4 + 1]);
        if (i4 + 2 > m) x[i4 + 2] = fmaf(-a.z, xm, x[i4 + 2]);
        if (i4 + 3 > m) x[i4 + 3] = fmaf(-a.w, xm, x[i4 + 3]);
      }
    }
    if (!is_u) {
      f32x4* dst = reinterpret_cast<f32x4*>(rec + kOffWT + c * kC);
#pragma unroll
      for (int i4 = 0; i4 < kC / 4; ++i4)
        dst[i4] = f32x4{x[4 * i4], x[4 * i4 + 1], x[4 * i4 + 2], x[4 * i4 + 3]};
    } else {
#pragma unroll
      for (int i = 0; i < kC; ++i) rec[kOffU + i * kDim + c] = x[i];
    }
  }

  // Qg^T and Kd: thread (k, half) covers tokens 32 half .. 32 half + 31
  {
    const int k = tid & (kDim - 1);
    const int i0 = (tid >> 7) * 32;
    f32x4* qdst = reinterpret_cast<f32x4*>(rec + kOffQT + k * kC + i0);
#pragma unroll
    for (int i4 = 0; i4 < 8; ++i4) {
      const int i = i0 + 4 * i4;
      qdst[i4] = f32x4{sQ[i][k] * sEg[i], sQ[i + 1][k] * sEg[i + 1], sQ[i + 2][k] * sEg[i + 2],
                       sQ[i + 3][k] * sEg[i + 3]};
    }
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) {
      const int i = i0 + ii;
      rec[kOffKd + i * kDim + k] = sK[i][k] * sEk[i];  // zero rows past the end
    }
  }
}

// ---- phase 2: per (sequence, v-head, block of 16 state rows), chunk by chunk ------------
__global__ __launch_bounds__(kThreads) void chunk_scan_kernel(const DecodeParams p,
                                                              int num_sequences, float* ws) {
  const int tile = blockIdx.x;
  const int seq = tile / (p.num_v_heads * kScanBlocks);
  const int rest = tile - seq * p.num_v_heads * kScanBlocks;
  const int head = rest / kScanBlocks;
  const int row0 = (rest - head * kScanBlocks) * kScanRows;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int bos = p.cu[seq];
  const int eos = p.cu[seq + 1];
  const int slot = p.indices[seq];
  const bool from_slot = slot > 0 && p.has_initial[seq] != 0;
  const int chunks = (eos - bos + kC - 1) / kC;
  const int gbase = chunk_base(p.cu, seq);

  constexpr int kSRow = 20;   // padded LDS row of S^T / V_new (16 rows, 16-byte aligned)
  __shared__ float sS[kDim][kSRow];   // S^T: [k][row]
  __shared__ float sW[kDim][kC];      // W^T
  __shared__ float sKd[kC][kDim];
  __shared__ float sVn[kC][kSRow];

  // thread (k, rh) owns S[row0 + 8 rh + e][k], e < 8, in the update
  const int k = tid & (kDim - 1);
  const int rh = tid >> 7;
  float* tile_base = p.state + static_cast<int64_t>(slot) * p.state_slot +
                     static_cast<int64_t>(head) * kDim * kDim;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    sS[k][8 * rh + e] = from_slot ? tile_base[(row0 + 8 * rh + e) * kDim + k] : 0.0f;

  // The next chunk's W^T, Kd (8 + 8 pieces of 16 bytes per thread) and U (one piece) are
  // loaded into registers while the current chunk computes.
  constexpr int kCopy = kDim * kC / 4 / kThreads;
  f32x4 wnext[kCopy], knext[kCopy], unext;
  float gnext = 0.0f;
  auto fetch = [&](int c) {
    const float* r = ws + (static_cast<int64_t>(gbase + c) * p.num_v_heads + head) * kRecord;
    const f32x4* wsrc = reinterpret_cast<const f32x4*>(r + kOffWT);
    const f32x4* ksrc = reinterpret_cast<const f32x4*>(r + kOffKd);
#pragma unroll
    for (int i = 0; i < kCopy; ++i) {
      wnext[i] = wsrc[i * kThreads + tid];
      knext[i] = ksrc[i * kThreads + tid];
    }
    unext = *reinterpret_cast<const f32x4*>(r + kOffU + lane * kDim + row0 + 4 * wave);
    gnext = r[kOffMisc];
  };
  if (chunks > 0) fetch(0);
  for (int c = 0; c < chunks; ++c) {
    float* rec = ws + (static_cast<int64_t>(gbase + c) * p.num_v_heads + head) * kRecord;
    __syncthreads();  // S of the chunk's start complete; the previous chunk's LDS reads done
#pragma unroll
    for (int e = 0; e < 8; ++e)
      rec[kOffH + (row0 + 8 * rh + e) * kDim + k] = sS[k][8 * rh + e];
    {
      f32x4* wdst = reinterpret_cast<f32x4*>(&sW[0][0]);
      f32x4* kdst = reinterpret_cast<f32x4*>(&sKd[0][0]);
#pragma unroll
      for (int i = 0; i < kCopy; ++i) {
        wdst[i * kThreads + tid] = wnext[i];
        kdst[i * kThreads + tid] = knext[i];
      }
    }
    const f32x4 u = unext;
    const float gamma = gnext;
    if (c + 1 < chunks) fetch(c + 1);
    __syncthreads();
    // V_new for token `lane` and local rows 4 wave .. 4 wave + 3
    {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
      for (int kk = 0; kk < kDim; ++kk)
        acc += sW[kk][lane] * *reinterpret_cast<const f32x4*>(&sS[kk][4 * wave]);
      const f32x4 vn = u - acc;
      *reinterpret_cast<f32x4*>(rec + kOffVn + lane * kDim + row0 + 4 * wave) = vn;
      *reinterpret_cast<f32x4*>(&sVn[lane][4 * wave]) = vn;
    }
    __syncthreads();
    // S' = exp(G_n-1) S + V_new^T Kd
    {
      f32x4 lo = gamma * *reinterpret_cast<const f32x4*>(&sS[k][8 * rh]);
      f32x4 hi = gamma * *reinterpret_cast<const f32x4*>(&sS[k][8 * rh + 4]);
#pragma unroll 8
      for (int j = 0; j < kC; ++j) {
        const float kd = sKd[j][k];
        lo += kd * *reinterpret_cast<const f32x4*>(&sVn[j][8 * rh]);
        hi += kd * *reinterpret_cast<const f32x4*>(&sVn[j][8 * rh + 4]);
      }
      *reinterpret_cast<f32x4*>(&sS[k][8 * rh]) = lo;
      *reinterpret_cast<f32x4*>(&sS[k][8 * rh + 4]) = hi;
    }
  }
  __syncthreads();
  if (slot > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) tile_base[(row0 + 8 * rh + e) * kDim + k] = sS[k][8 * rh + e];
  }
}

// ---- phase 3: per (chunk, v-head), raw outputs -----------------------------------------
__global__ __launch_bounds__(kThreads) void chunk_out_kernel(const DecodeParams p,
                                                             int num_sequences, float* ws) {
  const int head = blockIdx.y;
  int seq = 0, t0 = 0, len = 0;
  if (!find_chunk(p.cu, num_sequences, blockIdx.x, seq, t0, len)) return;
  const float* rec = ws + (static_cast<int64_t>(blockIdx.x) * p.num_v_heads + head) * kRecord;
  const int tid = threadIdx.x;

  constexpr int kHRow = kDim + 4;
  __shared__ float sQt[kDim][kC];      // Qg^T [k][i]
  __shared__ float sH[kDim][kHRow];    // H^T  [k][v]
  __shared__ float sPt[kC][kC];        // P^T  [j][i]
  __shared__ float sVn[kC][kDim];      // V_new [j][v]
  {
    const f32x4* q4 = reinterpret_cast<const f32x4*>(rec + kOffQT);
    const f32x4* v4 = reinterpret_cast<const f32x4*>(rec + kOffVn);
    f32x4* qd = reinterpret_cast<f32x4*>(&sQt[0][0]);
    f32x4* vd = reinterpret_cast<f32x4*>(&sVn[0][0]);
#pragma unroll
    for (int r = 0; r < kDim * kC / 4 / kThreads; ++r) {
      qd[r * kThreads + tid] = q4[r * kThreads + tid];
      vd[r * kThreads + tid] = v4[r * kThreads + tid];
    }
    const f32x4* p4 = reinterpret_cast<const f32x4*>(rec + kOffPT);
    f32x4* pd = reinterpret_cast<f32x4*>(&sPt[0][0]);
#pragma unroll
    for (int r = 0; r < kC * kC / 4 / kThreads; ++r) pd[r * kThreads + tid] = p4[r * kThreads + tid];
    // H[v][k] -> sH[k][v]: thread (k4, vgroup) loads 16 rows' 4 columns at once
    const int k4 = (tid & 31) * 4;
    const int v0 = (tid >> 5) * 16;
    f32x4 h[16];
#pragma unroll
    for (int vv = 0; vv < 16; ++vv)
      h[vv] = *reinterpret_cast<const f32x4*>(rec + kOffH + (v0 + vv) * kDim + k4);
#pragma unroll
    for (int vv = 0; vv < 16; ++vv) {
      sH[k4][v0 + vv] = h[vv].x;
      sH[k4 + 1][v0 + vv] = h[vv].y;
      sH[k4 + 2][v0 + vv] = h[vv].z;
      sH[k4 + 3][v0 + vv] = h[vv].w;
    }
  }
  __syncthreads();
  // lane block: tokens 4 ib .. 4 ib + 3, columns 8 vb .. 8 vb + 7 (3 LDS reads per 32 FMAs)
  const int vb = tid & 15;
  const int ib = tid >> 4;
  f32x4 acc[4][2];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) acc[ii][0] = acc[ii][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int kk = 0; kk < kDim; ++kk) {
    const f32x4 q = *reinterpret_cast<const f32x4*>(&sQt[kk][4 * ib]);
    const f32x4 h0 = *reinterpret_cast<const f32x4*>(&sH[kk][8 * vb]);
    const f32x4 h1 = *reinterpret_cast<const f32x4*>(&sH[kk][8 * vb + 4]);
    acc[0][0] += q.x * h0; acc[0][1] += q.x * h1;
    acc[1][0] += q.y * h0; acc[1][1] += q.y * h1;
    acc[2][0] += q.z * h0; acc[2][1] += q.z * h1;
    acc[3][0] += q.w * h0; acc[3][1] += q.w * h1;
  }
#pragma unroll 4
  for (int j = 0; j < kC; ++j) {
    const f32x4 pj = *reinterpret_cast<const f32x4*>(&sPt[j][4 * ib]);
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(&sVn[j][8 * vb]);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(&sVn[j][8 * vb + 4]);
    acc[0][0] += pj.x * v0; acc[0][1] += pj.x * v1;
    acc[1][0] += pj.y * v0; acc[1][1] += pj.y * v1;
    acc[2][0] += pj.z * v0; acc[2][1] += pj.z * v1;
    acc[3][0] += pj.w * v0; acc[3][1] += pj.w * v1;
  }
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const int i = 4 * ib + ii;
    if (i < len) {
      uint32_t packed[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        packed[2 * h] = f32_to_bf16(acc[ii][h].x) | (static_cast<uint32_t>(f32_to_bf16(acc[ii][h].y)) << 16);
        packed[2 * h + 1] = f32_to_bf16(acc[ii][h].z) | (static_cast<uint32_t>(f32_to_bf16(acc[ii][h].w)) << 16);
      }
      uint16_t* orow = p.out + (static_cast<int64_t>(t0 + i) * p.num_v_heads + head) * kDim + 8 * vb;
      *reinterpret_cast<uint4*>(orow) = uint4{packed[0], packed[1], packed[2], packed[3]};
    }
  }
}

int64_t max_chunks(int64_t num_tokens, int64_t num_sequences) {
  return num_tokens / kC + num_sequences;  // each sequence adds at most one partial chunk
}

}  // namespace

int64_t prefill_chunked_workspace_bytes(int64_t num_tokens, int64_t num_sequences,
                                        int64_t num_v_heads) {
  return max_chunks(num_tokens, num_sequences) * num_v_heads * kRecord * 4;
}

int launch_prefill_chunked(const DecodeParams& p, int num_sequences, int64_t num_tokens,
                           bool dt_bf16, void* workspace, hipStream_t stream) {
  float* ws = static_cast<float*>(workspace);
  const int64_t chunks = max_chunks(num_tokens, num_sequences);
  if (chunks > 0x7fffffff || p.num_v_heads > 65535)
    return fail(LD_ERR_INVALID_ARGUMENT, "prefill too large for the chunked form");
  const dim3 per_chunk(static_cast<uint32_t>(chunks), static_cast<uint32_t>(p.num_v_heads));
  if (dt_bf16)
    hipLaunchKernelGGL(chunk_prep_kernel<true>, per_chunk, dim3(kThreads), 0, stream, p,
                       num_sequences, ws);
  else
    hipLaunchKernelGGL(chunk_prep_kernel<false>, per_chunk, dim3(kThreads), 0, stream, p,
                       num_sequences, ws);
  const int64_t scan_tiles = static_cast<int64_t>(num_sequences) * p.num_v_heads * kScanBlocks;
  hipLaunchKernelGGL(chunk_scan_kernel, dim3(static_cast<uint32_t>(scan_tiles)), dim3(kThreads), 0,
                     stream, p, num_sequences, ws);
  hipLaunchKernelGGL(chunk_out_kernel, per_chunk, dim3(kThreads), 0, stream, p, num_sequences, ws);
  return check_launch("ld_gdn_prefill (chunked)");
}

}  // namespace ld
