// Shared device/host helpers for the gfx950 GDN decode library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lightdelta_hip.h"

namespace ld {

// ---- error reporting (host) -------------------------------------------------------

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const char* msg);
// Records a formatted launch error from `err` and returns LD_ERR_LAUNCH.
int launch_failed(const char* what, hipError_t err);
// Returns LD_OK after a launch, or LD_ERR_LAUNCH if the runtime reported an error.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- bf16 <-> fp32 (device) -----------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet (the rounding torch applies in
// `.to(torch.bfloat16)`).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// fp32 value of the bf16 nearest to f.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ---- cross-lane moves within a 16-lane DPP row -------------------------------------------

// DPP controls (GFX9 encoding).
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i of its 16-lane row
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i of its 8-lane half row
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]

template <int Ctrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), Ctrl, 0xF, 0xF, false));
}

// x of this lane and of lane i ^ 16 (Span 16) or i ^ 32 (Span 32), summed: gfx950's
// v_permlane16_swap / v_permlane32_swap on two copies of x exchange the odd rows of the
// first with the even rows of the second (rows of 16 lanes; for 32, the upper half of the
// first with the lower half of the second), so every lane ends with its own value in one
// and its partner's in the other.  A VALU exchange, where a shuffle goes through the LDS
// crossbar; the sum is the same (addition commutes), so the bits are those of
// x + shfl_xor(x, Span).
template <int Span>
__device__ __forceinline__ float add_partner(float x) {
  const uint32_t u = __float_as_uint(x);
  if constexpr (Span == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    static_assert(Span == 32, "rows of 16 or halves of 32");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  // Rows of 16 -> 64 (the same sums as x += shfl_xor(x, 16), then 32; 19.84 -> 19.81 us
  // for the B=32 step, bit-identical).
  x = add_partner<16>(x);
  x = add_partner<32>(x);
  return x;
}

}  // namespace ld
