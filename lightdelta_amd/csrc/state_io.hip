// Slot-indexed state-pool copies for gfx950: gather into a packed buffer, scatter back, and
// slot-to-slot copy.  Byte-generic (fp32 SSM pool, bf16 conv pool); bit-exact.
//
// Semantics follow the reference's copy kernel (csrc/state_io.cu:11-27): a slot <= 0 is
// padding; gather zero-fills rows whose slot is padding or whose `valid` flag is false,
// scatter and copy skip padding.  Zero resets whole slots in place (padding skipped).  Unlike the reference (one 4-byte element per thread per
// iteration, csrc/state_io.cu:22-26), every thread here moves 128-bit vectors with four
// loads in flight before the first store, and each workgroup owns one 16 KiB chunk of a row.
#include "common.h"

namespace ld {
namespace {

constexpr int kThreads = 256;
constexpr int kVecsPerThread = 4;
constexpr int64_t kVecsPerChunk = static_cast<int64_t>(kThreads) * kVecsPerThread;  // 16 KiB

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum Mode { kGather = 0, kScatter = 1, kCopy = 2, kZero = 3 };

struct CopyParams {
  const char* src;        // gather: pool; scatter: packed; copy: pool
  char* dst;              // gather: out; scatter: pool; copy: pool
  int64_t src_stride;     // bytes between consecutive src rows / slots
  int64_t dst_stride;     // bytes between consecutive dst rows / slots
  const int32_t* slots;   // gather/scatter/zero: slot per row; copy: source slot per pair
  int64_t slot_stride;    // elements between consecutive slots entries (gather/scatter)
  const int32_t* dst_slots;  // copy only
  const uint8_t* valid;   // gather only; NULL = all valid
  int32_t* rejected;      // copy only, optional: per pair, 1 = rejected for overlap, else 0
  int64_t rows;           // rows (copy: pairs)
  int64_t vecs;           // 16-byte vectors per row
  uint32_t chunks;        // chunks per row
};

// Cache hints: the pool side (rows at random slots, touched once) is non-temporal; the
// packed side of gather / scatter is a buffer the next kernel reads or the previous one
// wrote, so it stays cacheable.  Slot-to-slot copies read plainly and write non-temporally.
// Measured on 128 rows of 2 MiB against non-temporal on both sides: gather 86 -> 78 us,
// scatter 92-94 -> 77 us, copy 92 -> 76 us with the same pairs repeated (95 us when they
// rotate through the pool, as before).
template <int M>
__device__ __forceinline__ u32x4 load_row(const u32x4* src) {
  if constexpr (M == kGather) return __builtin_nontemporal_load(src);
  return *src;
}

template <int M>
__device__ __forceinline__ void store_row(u32x4 v, u32x4* dst) {
  if constexpr (M == kGather)
    *dst = v;
  else
    __builtin_nontemporal_store(v, dst);
}

// Copy: whether live pair `row` (source `from`, destination `to`, both > 0) conflicts with
// another live pair -- its source is another pair's destination, or its destination is
// another pair's source or destination.  Such pairs are rejected (nothing is written for
// them); the remaining pairs read slots no pair writes and write slots no other pair
// touches, so their copies are independent of the order of all reads and writes.  Every
// thread scans a share of the pairs; the verdict is the workgroup's OR (uniform).
__device__ __forceinline__ bool copy_conflicts(const CopyParams& p, uint32_t row, int from,
                                               int to) {
  bool conflict = false;
  for (int64_t q = threadIdx.x; q < p.rows; q += kThreads) {
    const int s = p.slots[q];
    const int d = p.dst_slots[q];
    conflict |= q != row && s > 0 && d > 0 && (d == from || s == to || d == to);
  }
  return __syncthreads_or(conflict);
}

// Copy: the conflict verdict of live pair `row` (uniform over the workgroup), recorded in
// the optional per-pair status by the workgroup of the row's first chunk: every pair's entry
// is written on every call, so the array needs no clearing beforehand.
__device__ __forceinline__ bool copy_rejected(const CopyParams& p, uint32_t row, uint32_t chunk) {
  const bool conflict = copy_conflicts(p, row, p.slots[row], p.dst_slots[row]);
  if (p.rejected != nullptr && chunk == 0 && threadIdx.x == 0) p.rejected[row] = conflict ? 1 : 0;
  return conflict;
}

// One workgroup moves one 16 KiB chunk of one row: 4 128-bit loads per thread in flight,
// then 4 stores.  Every branch below is uniform over the workgroup.
template <int M>
__global__ __launch_bounds__(kThreads) void slot_copy_kernel(const CopyParams p) {
  const uint32_t block = blockIdx.x;
  const uint32_t row = block / p.chunks;
  const uint32_t chunk = block - row * p.chunks;

  const u32x4* src;
  u32x4* dst;
  bool live = true;
  if (M == kGather) {
    const int slot = p.slots[row * p.slot_stride];
    live = slot > 0 && (p.valid == nullptr || p.valid[row] != 0);
    src = reinterpret_cast<const u32x4*>(p.src + (live ? slot : 0) * p.src_stride);
    dst = reinterpret_cast<u32x4*>(p.dst + row * p.dst_stride);
  } else if (M == kScatter) {
    const int slot = p.slots[row * p.slot_stride];
    if (slot <= 0) return;
    src = reinterpret_cast<const u32x4*>(p.src + row * p.src_stride);
    dst = reinterpret_cast<u32x4*>(p.dst + slot * p.dst_stride);
  } else if (M == kCopy) {
    const int from = p.slots[row];
    const int to = p.dst_slots[row];
    if (from <= 0 || to <= 0) {  // padding pair: not copied, not rejected
      if (p.rejected != nullptr && chunk == 0 && threadIdx.x == 0) p.rejected[row] = 0;
      return;
    }
    src = reinterpret_cast<const u32x4*>(p.src + from * p.src_stride);
    dst = reinterpret_cast<u32x4*>(p.dst + to * p.dst_stride);
  } else {  // zero fill of a slot (reuse by a new sequence)
    const int slot = p.slots[row];
    if (slot <= 0) return;
    src = nullptr;
    dst = reinterpret_cast<u32x4*>(p.dst + slot * p.dst_stride);
    live = false;
  }

  const int64_t begin = static_cast<int64_t>(chunk) * kVecsPerChunk;
  const int64_t first = begin + threadIdx.x;
  if (!live) {  // zero fill: gather of a padding / invalid row, or a slot reset
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i) {
      const int64_t idx = first + i * kThreads;
      if (idx < p.vecs) store_row<M>(u32x4{0u, 0u, 0u, 0u}, dst + idx);
    }
    return;
  }
  u32x4 v[kVecsPerThread];
  if (begin + kVecsPerChunk <= p.vecs) {  // whole chunk: unguarded, all loads in flight
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i)
      v[i] = load_row<M>(src + first + i * kThreads);
    // copy: the pair-conflict scan's loads go out right behind the chunk's (L2 hits), so the
    // scan adds little to the time the stores wait for the chunk anyway
    if (M == kCopy && copy_rejected(p, row, chunk)) return;
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i)
      store_row<M>(v[i], dst + first + i * kThreads);
    return;
  }
  // tail chunk of a row
#pragma unroll
  for (int i = 0; i < kVecsPerThread; ++i) {
    const int64_t idx = first + i * kThreads;
    v[i] = load_row<M>(src + (idx < p.vecs ? idx : 0));
  }
  if (M == kCopy && copy_rejected(p, row, chunk)) return;
#pragma unroll
  for (int i = 0; i < kVecsPerThread; ++i) {
    const int64_t idx = first + i * kThreads;
    if (idx < p.vecs) store_row<M>(v[i], dst + idx);
  }
}

int launch(const char* what, int mode, CopyParams p, int64_t rows, int64_t row_bytes,
           void* stream) {
  if (rows < 0 || row_bytes < 0) return fail(LD_ERR_INVALID_ARGUMENT, "negative size");
  if (rows == 0 || row_bytes == 0) return LD_OK;
  if ((row_bytes & 15) != 0 || (p.src_stride & 15) != 0 || (p.dst_stride & 15) != 0 ||
      (mode != kZero && !aligned16(p.src)) || !aligned16(p.dst))
    return fail(LD_ERR_INVALID_ARGUMENT,
                "state rows, strides and base pointers must be 16-byte aligned");
  p.rows = rows;
  p.vecs = row_bytes / 16;
  const int64_t chunks = (p.vecs + kVecsPerChunk - 1) / kVecsPerChunk;
  p.chunks = static_cast<uint32_t>(chunks);
  const int64_t blocks = rows * chunks;
  if (blocks > 0x7fffffff) return fail(LD_ERR_INVALID_ARGUMENT, "copy too large for one launch");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (mode == kGather)
    hipLaunchKernelGGL(slot_copy_kernel<kGather>, grid, dim3(kThreads), 0, s, p);
  else if (mode == kScatter)
    hipLaunchKernelGGL(slot_copy_kernel<kScatter>, grid, dim3(kThreads), 0, s, p);
  else if (mode == kCopy)
    hipLaunchKernelGGL(slot_copy_kernel<kCopy>, grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(slot_copy_kernel<kZero>, grid, dim3(kThreads), 0, s, p);
  return check_launch(what);
}

}  // namespace
}  // namespace ld

namespace ld {
namespace {

// The packed path's bookkeeping for a batch of `batch` requests of `width` slots each, one
// thread per (request r, token t) (python/lightdelta/backend.py:39-47, 87-91):
//   source[r]       = slots[r, clamp(accepted[r], 1, width) - 1]
//   valid[r]        = 1 <= accepted[r] <= width and source[r] > 0
//   indices[r, t]   = valid[r] ? 1 + r * width + t : 0       (the request's scratch rows)
//   destinations[r * width + t] = t < cu[r+1] - cu[r] and valid[r] and slots[r, t] > 0
//                                 ? slots[r, t] : 0
__global__ __launch_bounds__(kThreads) void packed_plan_kernel(
    const int32_t* slots, const int32_t* cu, const int32_t* accepted, int32_t batch,
    int32_t width, int32_t* source, uint8_t* valid, int32_t* indices, int32_t* destinations) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= static_cast<int64_t>(batch) * width) return;
  const int32_t r = static_cast<int32_t>(i / width);
  const int32_t t = static_cast<int32_t>(i - static_cast<int64_t>(r) * width);
  const int32_t acc = accepted[r];
  const int32_t src = slots[static_cast<int64_t>(r) * width + min(max(acc, 1), width) - 1];
  const bool ok = acc >= 1 && acc <= width && src > 0;
  if (t == 0) {
    source[r] = src;
    valid[r] = ok ? 1 : 0;
  }
  const int32_t slot = slots[i];
  const bool live = t < cu[r + 1] - cu[r];
  indices[i] = ok ? static_cast<int32_t>(1 + i) : 0;
  destinations[i] = live && ok && slot > 0 ? slot : 0;
}

}  // namespace
}  // namespace ld

extern "C" int ld_packed_plan(const int32_t* slots, const int32_t* cu, const int32_t* accepted,
                              int32_t batch, int32_t width, int32_t* source, uint8_t* valid,
                              int32_t* indices, int32_t* destinations, void* stream) {
  using namespace ld;
  if (batch < 0 || width < 1 || width > LD_MAX_TOKENS)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_packed_plan: batch must be >= 0 and width 1..4");
  if (batch == 0) return LD_OK;
  if (!slots || !cu || !accepted || !source || !valid || !indices || !destinations)
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_packed_plan: NULL pointer");
  const int64_t items = static_cast<int64_t>(batch) * width;
  const uint32_t blocks = static_cast<uint32_t>((items + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(packed_plan_kernel, dim3(blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), slots, cu, accepted, batch, width, source,
                     valid, indices, destinations);
  return check_launch("ld_packed_plan");
}

extern "C" int ld_state_gather(const void* pool, int64_t pool_slot_stride_bytes,
                               const int32_t* slots, int64_t slot_stride, const uint8_t* valid,
                               void* out, int64_t out_row_stride_bytes, int64_t row_bytes,
                               int64_t rows, void* stream) {
  using namespace ld;
  if (rows > 0 && (!pool || !slots || !out))
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_state_gather: NULL pointer");
  CopyParams p{};
  p.src = static_cast<const char*>(pool);
  p.dst = static_cast<char*>(out);
  p.src_stride = pool_slot_stride_bytes;
  p.dst_stride = out_row_stride_bytes;
  p.slots = slots;
  p.slot_stride = slot_stride;
  p.valid = valid;
  return launch("ld_state_gather", kGather, p, rows, row_bytes, stream);
}

extern "C" int ld_state_scatter(const void* packed, int64_t packed_row_stride_bytes,
                                const int32_t* slots, int64_t slot_stride, void* pool,
                                int64_t pool_slot_stride_bytes, int64_t row_bytes, int64_t rows,
                                void* stream) {
  using namespace ld;
  if (rows > 0 && (!pool || !slots || !packed))
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_state_scatter: NULL pointer");
  CopyParams p{};
  p.src = static_cast<const char*>(packed);
  p.dst = static_cast<char*>(pool);
  p.src_stride = packed_row_stride_bytes;
  p.dst_stride = pool_slot_stride_bytes;
  p.slots = slots;
  p.slot_stride = slot_stride;
  return launch("ld_state_scatter", kScatter, p, rows, row_bytes, stream);
}

namespace ld {
namespace {

int state_copy(const char* what, void* pool, int64_t pool_slot_stride_bytes,
               const int32_t* src_slots, const int32_t* dst_slots, int64_t pairs,
               int64_t slot_bytes, int32_t* rejected, void* stream) {
  if (pairs > 0 && (!pool || !src_slots || !dst_slots))
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_state_copy: NULL pointer");
  CopyParams p{};
  p.src = static_cast<const char*>(pool);
  p.dst = static_cast<char*>(pool);
  p.src_stride = pool_slot_stride_bytes;
  p.dst_stride = pool_slot_stride_bytes;
  p.slots = src_slots;
  p.dst_slots = dst_slots;
  p.rejected = rejected;
  return launch(what, kCopy, p, pairs, slot_bytes, stream);
}

}  // namespace
}  // namespace ld

extern "C" int ld_state_copy(void* pool, int64_t pool_slot_stride_bytes, const int32_t* src_slots,
                             const int32_t* dst_slots, int64_t pairs, int64_t slot_bytes,
                             void* stream) {
  return ld::state_copy("ld_state_copy", pool, pool_slot_stride_bytes, src_slots, dst_slots,
                        pairs, slot_bytes, nullptr, stream);
}

extern "C" int ld_state_copy_checked(void* pool, int64_t pool_slot_stride_bytes,
                                     const int32_t* src_slots, const int32_t* dst_slots,
                                     int64_t pairs, int64_t slot_bytes, int32_t* rejected,
                                     void* stream) {
  if (pairs > 0 && rejected == nullptr)
    return ld::fail(LD_ERR_INVALID_ARGUMENT, "ld_state_copy_checked: rejected is NULL");
  if (pairs > 0 && slot_bytes == 0)  // nothing would launch, so no status would be written
    return ld::fail(LD_ERR_INVALID_ARGUMENT, "ld_state_copy_checked: slot_bytes must be positive");
  return ld::state_copy("ld_state_copy_checked", pool, pool_slot_stride_bytes, src_slots,
                        dst_slots, pairs, slot_bytes, rejected, stream);
}

extern "C" int ld_state_zero(void* pool, int64_t pool_slot_stride_bytes, const int32_t* slots,
                             int64_t count, int64_t slot_bytes, void* stream) {
  using namespace ld;
  if (count > 0 && (!pool || !slots))
    return fail(LD_ERR_INVALID_ARGUMENT, "ld_state_zero: NULL pointer");
  CopyParams p{};
  p.dst = static_cast<char*>(pool);
  p.dst_stride = pool_slot_stride_bytes;
  p.slots = slots;
  return launch("ld_state_zero", kZero, p, count, slot_bytes, stream);
}
