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

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  // Rows of 16 -> 64 through the LDS crossbar.
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

}  // namespace ld
