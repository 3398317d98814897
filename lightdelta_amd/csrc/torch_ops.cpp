// Dispatcher kernels of the lightdelta ops (CUDA key, under which HIP tensors dispatch on
// PyTorch-ROCm): decode and decode_conv with the argument checks of the reference's launcher
// (csrc/gdn_decode.cu:366-403), generalised to any H, HV with HV % H == 0, with its
// messages; the state-pool ops with the checks of the reference's state_io
// (csrc/state_io.cu:29-49) and of the additive ones; then the C ABI of liblightdelta_hip.so
// on the current HIP stream of the tensors' device.  The schemas are defined by
// lightdelta_amd/ops.py, which loads this library (prefill keeps a Python kernel).
// Host-only C++ (no device code): one eager call costs a few microseconds of host time, as
// the reference's C++ launcher does, where a Python kernel costs about twelve.
#include <ATen/core/Tensor.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <atomic>
#include <optional>

#include "lightdelta_hip.h"

namespace {

constexpr int64_t kDim = LD_HEAD_DIM;

std::atomic<int> g_cache_policy{LD_CACHE_STREAM};

bool floats(const at::Tensor& t) {
  return t.scalar_type() == at::kFloat || t.scalar_type() == at::kBFloat16;
}

int32_t dtype_code(const at::Tensor& t) {
  return t.scalar_type() == at::kBFloat16 ? LD_DTYPE_BF16 : LD_DTYPE_F32;
}

// The decode step's checks (ops.py _decode_layout has the same ones for the Python-side
// callers); returns H, HV.
std::pair<int64_t, int64_t> check_decode(const at::Tensor& qkv, const at::Tensor& a,
                                         const at::Tensor& b, const at::Tensor& a_log,
                                         const at::Tensor& dt_bias, const at::Tensor& indices,
                                         const at::Tensor& cu, const at::Tensor& accepted,
                                         const at::Tensor& state, const at::Tensor& gate,
                                         const at::Tensor& weight, const at::Tensor& out,
                                         double eps) {
  TORCH_CHECK(qkv.is_cuda() && qkv.scalar_type() == at::kBFloat16, "qkv must be CUDA BF16");
  const c10::Device device = qkv.device();
  for (const at::Tensor* t : {&a, &b, &gate, &out})
    TORCH_CHECK(t->device() == device && t->scalar_type() == at::kBFloat16 && t->dim() > 0 &&
                    t->stride(-1) == 1,
                "activations must be BF16 with dense rows");
  for (const at::Tensor* t : {&a_log, &state})
    TORCH_CHECK(t->device() == device && t->scalar_type() == at::kFloat && t->dim() > 0 &&
                    t->stride(-1) == 1,
                "state and A_log must be CUDA FP32 with dense rows");
  for (const at::Tensor* t : {&indices, &cu, &accepted})
    TORCH_CHECK(t->device() == device && t->scalar_type() == at::kInt && t->is_contiguous(),
                "metadata must be contiguous CUDA int32");
  for (const at::Tensor* t : {&dt_bias, &weight})
    TORCH_CHECK(t->device() == device && t->is_contiguous() && floats(*t),
                "weights must be contiguous FP32/BF16");
  // H and HV from qkv's width (2H + HV) * 128 and the state's head count
  const int64_t hv = state.dim() == 4 ? state.size(1) : 0;
  const int64_t cols = qkv.dim() == 2 ? qkv.size(1) : 0;
  const int64_t h2 = cols / kDim - hv;
  const int64_t h = h2 / 2;
  const bool geometry = hv > 0 && cols % kDim == 0 && h2 > 0 && h2 % 2 == 0 && hv % h == 0;
  TORCH_CHECK(qkv.dim() == 2 && geometry && qkv.stride(1) == 1,
              "qkv must be [tokens,(2*H+HV)*128] with HV a multiple of H");
  TORCH_CHECK(state.dim() == 4 && state.size(2) == kDim && state.size(3) == kDim &&
                  state.stride(2) == kDim && state.stride(1) == kDim * kDim,
              "state must be [slots,HV,128,128]");
  TORCH_CHECK(indices.dim() == 2 && indices.size(1) >= 1 && indices.size(1) <= LD_MAX_TOKENS,
              "decode/MTP supports 1 through 4 tokens per request");
  const int64_t n = qkv.size(0);
  TORCH_CHECK(a.dim() == 2 && a.size(0) == n && a.size(1) == hv && b.dim() == 2 &&
                  b.size(0) == n && b.size(1) == hv && gate.dim() == 3 && gate.size(0) == n &&
                  gate.size(1) == hv && gate.size(2) == kDim && out.dim() == 3 &&
                  out.size(0) == n && out.size(1) == hv && out.size(2) == kDim &&
                  out.is_contiguous() && gate.stride(1) == kDim,
              "invalid activation shape or output layout");
  TORCH_CHECK(a_log.numel() == hv && dt_bias.numel() == hv && weight.numel() == kDim,
              "invalid weight shapes");
  const int64_t requests = indices.size(0);
  TORCH_CHECK(cu.dim() == 1 && cu.numel() == requests + 1 && accepted.dim() == 1 &&
                  accepted.numel() == requests,
              "invalid request metadata shapes");
  TORCH_CHECK(eps > 0, "norm epsilon must be positive");
  return {h, hv};
}

ld_gdn_decode_args decode_args(const at::Tensor& qkv, const at::Tensor& a,
                               const at::Tensor& b, const at::Tensor& a_log,
                               const at::Tensor& dt_bias, const at::Tensor& indices,
                               const at::Tensor& cu, const at::Tensor& accepted,
                               const at::Tensor& state, const at::Tensor& gate,
                               const at::Tensor& weight, const at::Tensor& out, double eps,
                               std::pair<int64_t, int64_t> heads) {
  ld_gdn_decode_args args{};
  args.qkv = qkv.data_ptr();
  args.qkv_row_stride = qkv.stride(0);
  args.a = a.data_ptr();
  args.a_row_stride = a.stride(0);
  args.b = b.data_ptr();
  args.b_row_stride = b.stride(0);
  args.a_log = static_cast<const float*>(a_log.data_ptr());
  args.dt_bias = dt_bias.data_ptr();
  args.dt_bias_dtype = dtype_code(dt_bias);
  args.norm_weight_dtype = dtype_code(weight);
  args.indices = static_cast<const int32_t*>(indices.data_ptr());
  args.cu = static_cast<const int32_t*>(cu.data_ptr());
  args.accepted = static_cast<const int32_t*>(accepted.data_ptr());
  args.state = static_cast<float*>(state.data_ptr());
  args.state_slot_stride = state.stride(0);
  args.gate = gate.data_ptr();
  args.gate_row_stride = gate.stride(0);
  args.norm_weight = weight.data_ptr();
  args.out = out.data_ptr();
  args.num_requests = static_cast<int32_t>(indices.size(0));
  args.width = static_cast<int32_t>(indices.size(1));
  args.num_k_heads = static_cast<int32_t>(heads.first);
  args.num_v_heads = static_cast<int32_t>(heads.second);
  args.scale = static_cast<float>(0.08838834764831845);  // 128^-0.5 (reference csrc/gdn_decode.cu:417)
  args.eps = static_cast<float>(eps);
  args.cache_policy = g_cache_policy.load(std::memory_order_relaxed);
  return args;
}

void decode(const at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b,
            const at::Tensor& a_log, const at::Tensor& dt_bias, const at::Tensor& indices,
            const at::Tensor& cu, const at::Tensor& accepted, at::Tensor state,
            const at::Tensor& gate, const at::Tensor& weight, at::Tensor out, double eps) {
  const auto heads = check_decode(qkv, a, b, a_log, dt_bias, indices, cu, accepted, state, gate,
                                  weight, out, eps);
  if (indices.size(0) == 0) return;
  const ld_gdn_decode_args args = decode_args(qkv, a, b, a_log, dt_bias, indices, cu, accepted,
                                              state, gate, weight, out, eps, heads);
  const c10::DeviceGuard guard(qkv.device());
  const int rc = ld_gdn_decode(&args, c10::hip::getCurrentHIPStream(qkv.get_device()).stream());
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void decode_conv(const at::Tensor& mixed_qkv, at::Tensor conv_state, const at::Tensor& conv_weight,
                 const std::optional<at::Tensor>& conv_bias, const at::Tensor& a,
                 const at::Tensor& b, const at::Tensor& a_log, const at::Tensor& dt_bias,
                 const at::Tensor& indices, const at::Tensor& cu, const at::Tensor& accepted,
                 at::Tensor state, const at::Tensor& gate, const at::Tensor& weight,
                 at::Tensor out, double eps) {
  const auto heads = check_decode(mixed_qkv, a, b, a_log, dt_bias, indices, cu, accepted, state,
                                  gate, weight, out, eps);
  const int64_t conv_dim = mixed_qkv.size(1);
  TORCH_CHECK(conv_state.device() == mixed_qkv.device() &&
                  conv_state.scalar_type() == at::kBFloat16 && conv_state.dim() == 3 &&
                  conv_state.size(1) == conv_dim && conv_state.size(2) >= 3 &&
                  conv_state.size(2) <= 8,
              "conv_state must be CUDA BF16 [slots, conv_dim, 3..8]");
  TORCH_CHECK(conv_weight.device() == mixed_qkv.device() &&
                  conv_weight.scalar_type() == at::kBFloat16 && conv_weight.dim() == 2 &&
                  conv_weight.size(0) == conv_dim && conv_weight.size(1) == 4 &&
                  conv_weight.is_contiguous() &&
                  reinterpret_cast<uintptr_t>(conv_weight.data_ptr()) % 8 == 0,
              "conv_weight must be contiguous CUDA BF16 [conv_dim, 4]");
  const at::Tensor* bias = conv_bias.has_value() ? &*conv_bias : nullptr;
  if (bias != nullptr)
    TORCH_CHECK(bias->device() == mixed_qkv.device() && bias->scalar_type() == at::kBFloat16 &&
                    bias->numel() == conv_dim && bias->is_contiguous(),
                "conv_bias must be contiguous CUDA BF16 [conv_dim]");
  ld_gdn_decode_args args = decode_args(mixed_qkv, a, b, a_log, dt_bias, indices, cu, accepted,
                                        state, gate, weight, out, eps, heads);
  args.qkv = nullptr;  // the post-conv activations are the kernel's own
  args.qkv_row_stride = 0;
  ld_conv_args conv{};
  conv.x = mixed_qkv.data_ptr();
  conv.x_row_stride = mixed_qkv.stride(0);
  conv.state = conv_state.data_ptr();
  conv.state_slots = conv_state.size(0);
  conv.state_slot_stride = conv_state.stride(0);
  conv.state_dim_stride = conv_state.stride(1);
  conv.state_len_stride = conv_state.stride(2);
  conv.state_len = static_cast<int32_t>(conv_state.size(2));
  conv.width = 4;
  conv.weight = conv_weight.data_ptr();
  conv.weight_dtype = LD_DTYPE_BF16;
  conv.bias_dtype = LD_DTYPE_BF16;
  conv.bias = bias != nullptr ? bias->data_ptr() : nullptr;
  const c10::DeviceGuard guard(mixed_qkv.device());
  const int rc = ld_gdn_decode_conv(
      &args, &conv, c10::hip::getCurrentHIPStream(mixed_qkv.get_device()).stream());
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

// ---- state-pool ops ----------------------------------------------------------------------

// Every dimension after the first densely packed (row-major).
bool dense_inner(const at::Tensor& t) {
  int64_t expected = 1;
  for (int64_t d = t.dim() - 1; d >= 1; --d) {
    if (t.size(d) != 1 && t.stride(d) != expected) return false;
    expected *= t.size(d);
  }
  return true;
}

int64_t row_bytes(const at::Tensor& t) {
  int64_t count = 1;
  for (int64_t d = 1; d < t.dim(); ++d) count *= t.size(d);
  return count * static_cast<int64_t>(t.element_size());
}

bool same_row_shape(const at::Tensor& a, const at::Tensor& b) {
  if (a.dim() != b.dim()) return false;
  for (int64_t d = 1; d < a.dim(); ++d)
    if (a.size(d) != b.size(d)) return false;
  return true;
}

// The reference's `check` (csrc/state_io.cu:29-41); fp32_4d = false drops the fp32 / 4-D
// requirement for the dtype-generic ops.
void check_state_layout(const at::Tensor& pool, const at::Tensor& slots, const at::Tensor& packed,
                        bool fp32_4d) {
  if (fp32_4d) {
    TORCH_CHECK(pool.is_cuda() && pool.scalar_type() == at::kFloat && pool.dim() == 4 &&
                    pool.stride(3) == 1 && pool.stride(2) == pool.size(3) &&
                    pool.stride(1) == pool.size(2) * pool.size(3),
                "pool must be CUDA FP32 with dense inner dimensions");
  } else {
    TORCH_CHECK(pool.is_cuda() && pool.dim() >= 1 && dense_inner(pool),
                "pool must be a CUDA tensor with dense inner dimensions");
  }
  TORCH_CHECK(slots.device() == pool.device() && slots.scalar_type() == at::kInt &&
                  slots.dim() == 1,
              "slots must be a CUDA int32 vector");
  TORCH_CHECK(packed.device() == pool.device() && packed.scalar_type() == pool.scalar_type() &&
                  packed.dim() == pool.dim() && packed.size(0) == slots.numel() &&
                  same_row_shape(packed, pool) && dense_inner(packed),
              "invalid packed layout");
}

void check_valid(const at::Tensor& valid, const at::Tensor& slots, const at::Tensor& pool) {
  TORCH_CHECK(valid.device() == pool.device() && valid.scalar_type() == at::kBool &&
                  valid.sizes() == slots.sizes() && valid.is_contiguous(),
              "valid must be a CUDA bool vector");
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void gather(const at::Tensor& pool, const at::Tensor& slots, const at::Tensor& valid,
            at::Tensor out) {
  if (slots.numel() == 0) return;
  const int64_t size = static_cast<int64_t>(pool.element_size());
  const c10::DeviceGuard guard(pool.device());
  const int rc = ld_state_gather(pool.data_ptr(), pool.stride(0) * size,
                                 static_cast<const int32_t*>(slots.data_ptr()), slots.stride(0),
                                 static_cast<const uint8_t*>(valid.data_ptr()), out.data_ptr(),
                                 out.stride(0) * size, row_bytes(pool), slots.numel(),
                                 stream_of(pool));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void scatter(const at::Tensor& packed, const at::Tensor& slots, at::Tensor pool) {
  if (slots.numel() == 0) return;
  const int64_t size = static_cast<int64_t>(pool.element_size());
  const c10::DeviceGuard guard(pool.device());
  const int rc = ld_state_scatter(packed.data_ptr(), packed.stride(0) * size,
                                  static_cast<const int32_t*>(slots.data_ptr()), slots.stride(0),
                                  pool.data_ptr(), pool.stride(0) * size, row_bytes(pool),
                                  slots.numel(), stream_of(pool));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void gather_state(const at::Tensor& pool, const at::Tensor& slots, const at::Tensor& valid,
                  at::Tensor out) {
  check_state_layout(pool, slots, out, true);
  check_valid(valid, slots, pool);
  gather(pool, slots, valid, out);
}

void scatter_state(const at::Tensor& packed, const at::Tensor& slots, at::Tensor pool) {
  check_state_layout(pool, slots, packed, true);
  scatter(packed, slots, pool);
}

void gather_slots(const at::Tensor& pool, const at::Tensor& slots, const at::Tensor& valid,
                  at::Tensor out) {
  check_state_layout(pool, slots, out, false);
  check_valid(valid, slots, pool);
  gather(pool, slots, valid, out);
}

void scatter_slots(const at::Tensor& packed, const at::Tensor& slots, at::Tensor pool) {
  check_state_layout(pool, slots, packed, false);
  scatter(packed, slots, pool);
}

void check_copy(const at::Tensor& pool, const at::Tensor& src, const at::Tensor& dst) {
  TORCH_CHECK(pool.is_cuda() && pool.dim() >= 1 && dense_inner(pool),
              "pool must be a CUDA tensor with dense inner dimensions");
  for (const at::Tensor* t : {&src, &dst})
    TORCH_CHECK(t->device() == pool.device() && t->scalar_type() == at::kInt && t->dim() == 1 &&
                    t->is_contiguous(),
                "src and dst must be contiguous CUDA int32 vectors");
  TORCH_CHECK(src.numel() == dst.numel(), "src and dst must have the same length");
}

void copy_state(at::Tensor pool, const at::Tensor& src, const at::Tensor& dst) {
  check_copy(pool, src, dst);
  if (src.numel() == 0) return;
  const c10::DeviceGuard guard(pool.device());
  const int rc = ld_state_copy(pool.data_ptr(),
                               pool.stride(0) * static_cast<int64_t>(pool.element_size()),
                               static_cast<const int32_t*>(src.data_ptr()),
                               static_cast<const int32_t*>(dst.data_ptr()), src.numel(),
                               row_bytes(pool), stream_of(pool));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void copy_state_checked(at::Tensor pool, const at::Tensor& src, const at::Tensor& dst,
                        at::Tensor rejected) {
  check_copy(pool, src, dst);
  TORCH_CHECK(rejected.device() == pool.device() && rejected.scalar_type() == at::kInt &&
                  rejected.dim() == 1 && rejected.is_contiguous() &&
                  rejected.numel() == src.numel(),
              "rejected must be a contiguous CUDA int32 vector with one entry per pair");
  if (src.numel() == 0) return;
  TORCH_CHECK(row_bytes(pool) > 0, "pool slots must not be empty");
  const c10::DeviceGuard guard(pool.device());
  const int rc = ld_state_copy_checked(
      pool.data_ptr(), pool.stride(0) * static_cast<int64_t>(pool.element_size()),
      static_cast<const int32_t*>(src.data_ptr()), static_cast<const int32_t*>(dst.data_ptr()),
      src.numel(), row_bytes(pool), static_cast<int32_t*>(rejected.data_ptr()), stream_of(pool));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void zero_slots(at::Tensor pool, const at::Tensor& slots) {
  TORCH_CHECK(pool.is_cuda() && pool.dim() >= 1 && dense_inner(pool),
              "pool must be a CUDA tensor with dense inner dimensions");
  TORCH_CHECK(slots.device() == pool.device() && slots.scalar_type() == at::kInt &&
                  slots.dim() == 1 && slots.is_contiguous(),
              "slots must be a contiguous CUDA int32 vector");
  if (slots.numel() == 0) return;
  const c10::DeviceGuard guard(pool.device());
  const int rc = ld_state_zero(pool.data_ptr(),
                               pool.stride(0) * static_cast<int64_t>(pool.element_size()),
                               static_cast<const int32_t*>(slots.data_ptr()), slots.numel(),
                               row_bytes(pool), stream_of(pool));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

void packed_plan(const at::Tensor& slots, const at::Tensor& cu, const at::Tensor& accepted,
                 at::Tensor source, at::Tensor valid, at::Tensor indices,
                 at::Tensor destinations) {
  TORCH_CHECK(slots.is_cuda() && slots.scalar_type() == at::kInt && slots.dim() == 2 &&
                  slots.is_contiguous() && slots.size(1) >= 1 && slots.size(1) <= LD_MAX_TOKENS,
              "slots must be a contiguous CUDA int32 [batch, 1..4] tensor");
  const int64_t batch = slots.size(0);
  const int64_t width = slots.size(1);
  const std::pair<const at::Tensor*, std::vector<int64_t>> ints[] = {
      {&cu, {batch + 1}}, {&accepted, {batch}}, {&source, {batch}},
      {&indices, {batch, width}}, {&destinations, {batch * width}}};
  for (const auto& [t, shape] : ints)
    TORCH_CHECK(t->device() == slots.device() && t->scalar_type() == at::kInt &&
                    t->sizes() == at::IntArrayRef(shape) && t->is_contiguous(),
                "packed_plan tensors must be contiguous CUDA int32 of the batch's shapes");
  TORCH_CHECK(valid.device() == slots.device() && valid.scalar_type() == at::kBool &&
                  valid.dim() == 1 && valid.size(0) == batch && valid.is_contiguous(),
              "valid must be a contiguous CUDA bool vector");
  TORCH_CHECK(batch <= INT32_MAX, "batch too large");
  if (batch == 0) return;
  const c10::DeviceGuard guard(slots.device());
  const int rc = ld_packed_plan(
      static_cast<const int32_t*>(slots.data_ptr()), static_cast<const int32_t*>(cu.data_ptr()),
      static_cast<const int32_t*>(accepted.data_ptr()), static_cast<int32_t>(batch),
      static_cast<int32_t>(width), static_cast<int32_t*>(source.data_ptr()),
      static_cast<uint8_t*>(valid.data_ptr()), static_cast<int32_t*>(indices.data_ptr()),
      static_cast<int32_t*>(destinations.data_ptr()), stream_of(slots));
  TORCH_CHECK(rc == LD_OK, ld_last_error());
}

}  // namespace

TORCH_LIBRARY_IMPL(lightdelta, CUDA, m) {
  m.impl("decode", &decode);
  m.impl("decode_conv", &decode_conv);
  m.impl("gather_state", &gather_state);
  m.impl("scatter_state", &scatter_state);
  m.impl("gather_slots", &gather_slots);
  m.impl("scatter_slots", &scatter_slots);
  m.impl("copy_state", &copy_state);
  m.impl("copy_state_checked", &copy_state_checked);
  m.impl("zero_slots", &zero_slots);
  m.impl("packed_plan", &packed_plan);
}

// The state cache policy these kernels pass (LD_CACHE_KEEP / LD_CACHE_STREAM), set from
// lightdelta_amd.ops.set_state_cache_policy.
extern "C" int ld_torch_set_cache_policy(int policy) {
  if (policy != LD_CACHE_KEEP && policy != LD_CACHE_STREAM) return LD_ERR_INVALID_ARGUMENT;
  g_cache_policy.store(policy, std::memory_order_relaxed);
  return LD_OK;
}
