"""`torch.ops.lightdelta.*` on PyTorch-ROCm, backed by the gfx950 HIP library.

The three reference ops keep their schema strings verbatim (reference csrc/register.cpp:5-9)
and are registered for the CUDA dispatch key, under which HIP tensors dispatch on ROCm; the
fake (meta) impls return None like the reference's (python/lightdelta/ops/__init__.py:10-22).
Argument validation raises RuntimeError with the reference's messages
(csrc/gdn_decode.cu:367-403, csrc/state_io.cu:29-49), generalised from the hard-coded
16 k-heads / 48 v-heads / qkv width 10240 to any H, HV with HV % H == 0 (dk = dv = 128).

Additive ops (no reference counterpart):
  copy_state(pool, src, dst)            slot -> slot copy inside one pool (MTP commit,
                                        slot reuse), any dtype, padding slot <= 0 skipped;
                                        a pair that overlaps another (its source another's
                                        destination, its destination another's source or
                                        destination) is rejected and writes nothing
  copy_state_checked(pool, src, dst, rejected)
                                        copy_state that also writes, per pair, 1 to
                                        rejected (int32 [pairs]) if it was rejected for
                                        overlap, else 0 (every entry on every call, so no
                                        clearing is needed; graph-safe)
  zero_slots(pool, slots)               zero whole slots in place (a slot reused by a new
                                        sequence), any dtype, padding slot <= 0 skipped
  decode_conv(mixed_qkv, conv_state, conv_weight, conv_bias, <decode args without qkv>)
                                        causal conv1d (width 4, SiLU, bf16 output) of the
                                        pre-conv activations fused into the decode step;
                                        conv_state [slots, conv_dim, state_len] (any strides,
                                        so vLLM's transposed dim-last view works); 1 to 4
                                        tokens per request, speculative verify with vLLM's
                                        num_accepted_tokens semantics (accepted)
  prefill(qkv, a, b, a_log, dt_bias, slots, has_initial, cu_seqlens, state, gate, weight,
          out, eps)                     the layer's prefill (post-conv activations of several
                                        sequences, cu_seqlens rows each) in one launch: state
                                        from slots[n] if has_initial[n] else zeros, the
                                        decode recurrence token by token, gated RMSNorm
                                        outputs, final state to slots[n]
  gather_slots / scatter_slots          dtype-generic gather_state / scatter_state, for the
                                        bf16 conv-state pool and any dense-inner pool
  packed_plan(slots, cu, accepted, source, valid, indices, destinations)
                                        the packed path's bookkeeping (GDNBackend,
                                        state_io = "packed") in one launch: each request's
                                        source slot and validity, its scratch rows, and the
                                        slots its per-token states go back to

Every kernel launches on the caller's current stream and reads no device memory on the host,
so it can be captured in a HIP graph.  None allocates, except prefill's chunked form, which
keeps one workspace per device and stream for later eager calls (release_prefill_workspaces
frees them) and gives a call under graph capture a workspace the graph keeps.  The kernels of every op but prefill are C++ (csrc/torch_ops.cpp,
liblightdelta_torch.so); the check_* functions below restate their argument checks so they
can run without a GPU.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

from . import _lib

SCHEMAS = {
    "decode": (
        "decode(Tensor qkv, Tensor a, Tensor b, Tensor a_log, Tensor dt_bias, "
        "Tensor indices, Tensor cu, Tensor accepted, Tensor(s!) state, Tensor gate, "
        "Tensor weight, Tensor(o!) out, float eps) -> ()"
    ),
    "gather_state": "gather_state(Tensor pool, Tensor slots, Tensor valid, Tensor(o!) out) -> ()",
    "scatter_state": "scatter_state(Tensor packed, Tensor slots, Tensor(p!) pool) -> ()",
    "copy_state": "copy_state(Tensor(p!) pool, Tensor src, Tensor dst) -> ()",
    "copy_state_checked": (
        "copy_state_checked(Tensor(p!) pool, Tensor src, Tensor dst, Tensor(r!) rejected) -> ()"
    ),
    "zero_slots": "zero_slots(Tensor(p!) pool, Tensor slots) -> ()",
    "prefill": (
        "prefill(Tensor qkv, Tensor a, Tensor b, Tensor a_log, Tensor dt_bias, Tensor slots, "
        "Tensor has_initial, Tensor cu_seqlens, Tensor(s!) state, Tensor gate, Tensor weight, "
        "Tensor(o!) out, float eps) -> ()"
    ),
    "decode_conv": (
        "decode_conv(Tensor mixed_qkv, Tensor(c!) conv_state, Tensor conv_weight, "
        "Tensor? conv_bias, Tensor a, Tensor b, Tensor a_log, Tensor dt_bias, Tensor indices, "
        "Tensor cu, Tensor accepted, Tensor(s!) state, Tensor gate, Tensor weight, "
        "Tensor(o!) out, float eps) -> ()"
    ),
    "gather_slots": "gather_slots(Tensor pool, Tensor slots, Tensor valid, Tensor(o!) out) -> ()",
    "packed_plan": (
        "packed_plan(Tensor slots, Tensor cu, Tensor accepted, Tensor(s!) source, "
        "Tensor(v!) valid, Tensor(i!) indices, Tensor(d!) destinations) -> ()"
    ),
    "scatter_slots": "scatter_slots(Tensor packed, Tensor slots, Tensor(p!) pool) -> ()",
}

HEAD_DIM = _lib.HEAD_DIM
QK_SCALE = HEAD_DIM**-0.5  # reference csrc/gdn_decode.cu:417

# State cache policy of the decode kernel (never changes results, only which kernel shape and
# cache hints move the state): "stream" is tuned for working sets far beyond the 256 MB
# Infinity Cache -- a model's many layers between two steps of one layer, the serving regime
# -- and is the default; "keep" for one layer's working set stepped again while it is still
# cached (a single-layer benchmark), where it is ~4% faster and "stream" ~17% slower cold.
# Set with set_state_cache_policy() or the LIGHTDELTA_STATE_CACHE environment variable.
_POLICIES = {"keep": _lib.CACHE_KEEP, "stream": _lib.CACHE_STREAM}


def _policy_from_env() -> int:
    name = os.environ.get("LIGHTDELTA_STATE_CACHE", "stream")
    if name not in _POLICIES:
        raise ValueError(f"LIGHTDELTA_STATE_CACHE={name!r}: the state cache policy must be one of "
                         f"{sorted(_POLICIES)}")
    return _POLICIES[name]


_cache_policy = _policy_from_env()


def set_state_cache_policy(policy: str) -> None:
    global _cache_policy
    if policy not in _POLICIES:
        raise ValueError(f"state cache policy must be one of {sorted(_POLICIES)}")
    _cache_policy = _POLICIES[policy]
    if _TORCH_KERNELS is not None:
        _TORCH_KERNELS.ld_torch_set_cache_policy(_cache_policy)


def state_cache_policy() -> str:
    return next(name for name, code in _POLICIES.items() if code == _cache_policy)

_FLOATS = (torch.float32, torch.bfloat16)


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _is_gpu(t: torch.Tensor) -> bool:
    return t.is_cuda


_BF16, _F32, _I32 = torch.bfloat16, torch.float32, torch.int32

# The calling thread's current device and a device's current stream as plain integers:
# torch's raw accessors where this build has them (torch.cuda.current_stream() builds a Stream
# object, ~2 us per call), the public API otherwise.
_current_device = getattr(torch._C, "_cuda_getDevice", torch.cuda.current_device)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device) -> int:
    index = device if isinstance(device, int) else device.index
    if index is None:
        index = _current_device()
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


class _DeviceGuard:
    """Makes `device` current for the duration of a launch (the reference's CUDAGuard)."""

    __slots__ = ("index", "previous")

    def __init__(self, device):
        index = device if isinstance(device, int) else device.index
        self.index = index if index is not None else _current_device()
        self.previous = None

    def __enter__(self):
        current = _current_device()
        if current != self.index:
            self.previous = current
            torch.cuda.set_device(self.index)

    def __exit__(self, *exc):
        if self.previous is not None:
            torch.cuda.set_device(self.previous)


# ---------------------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------------------


def decode_geometry(qkv: torch.Tensor, state: torch.Tensor) -> tuple[int, int]:
    """(H, HV) implied by qkv's width (2*H + HV)*128 and the state's head count."""
    hv = state.shape[1] if state.dim() == 4 else 0
    cols = qkv.shape[1] if qkv.dim() == 2 else 0
    h2 = cols // HEAD_DIM - hv
    h = h2 // 2
    valid = (
        hv > 0
        and cols % HEAD_DIM == 0
        and h2 > 0
        and h2 % 2 == 0
        and hv % h == 0
    )
    return (h, hv) if valid else (0, hv)


def _decode_layout(qkv, a, b, a_log, dt_bias, indices, cu, accepted, state, gate, weight, out,
                   eps):
    """Validation of lightdelta::decode (reference csrc/gdn_decode.cu:366-403), reading each
    tensor property once: returns (H, HV, device index, requests, width) and the row strides
    of qkv, a, b, state and gate, which the launch needs."""
    if not (_is_gpu(qkv) and qkv.dtype is _BF16):
        raise RuntimeError("qkv must be CUDA BF16")
    dev = qkv.get_device()
    for t in (a, b, gate, out):
        if not (t.get_device() == dev and t.dtype is _BF16 and t.dim() > 0 and t.stride(-1) == 1):
            raise RuntimeError("activations must be BF16 with dense rows")
    for t in (a_log, state):
        if not (t.get_device() == dev and t.dtype is _F32 and t.dim() > 0 and t.stride(-1) == 1):
            raise RuntimeError("state and A_log must be CUDA FP32 with dense rows")
    for t in (indices, cu, accepted):
        if not (t.get_device() == dev and t.dtype is _I32 and t.is_contiguous()):
            raise RuntimeError("metadata must be contiguous CUDA int32")
    for t in (dt_bias, weight):
        if not (t.get_device() == dev and t.is_contiguous() and t.dtype in _FLOATS):
            raise RuntimeError("weights must be contiguous FP32/BF16")
    qkv_shape, qkv_stride = qkv.shape, qkv.stride()
    state_shape, state_stride = state.shape, state.stride()
    h, hv = decode_geometry(qkv, state)
    if not (len(qkv_shape) == 2 and h > 0 and qkv_stride[1] == 1):
        raise RuntimeError("qkv must be [tokens,(2*H+HV)*128] with HV a multiple of H")
    if not (len(state_shape) == 4 and state_shape[2] == HEAD_DIM and state_shape[3] == HEAD_DIM
            and state_stride[2] == HEAD_DIM and state_stride[1] == HEAD_DIM * HEAD_DIM):
        raise RuntimeError("state must be [slots,HV,128,128]")
    indices_shape = indices.shape
    if not (len(indices_shape) == 2 and 1 <= indices_shape[1] <= _lib.MAX_TOKENS):
        raise RuntimeError("decode/MTP supports 1 through 4 tokens per request")
    n = qkv_shape[0]
    gate_stride = gate.stride()
    if not (a.shape == (n, hv) and b.shape == (n, hv) and gate.shape == (n, hv, HEAD_DIM)
            and out.shape == (n, hv, HEAD_DIM) and out.is_contiguous()
            and gate_stride[1] == HEAD_DIM):
        raise RuntimeError("invalid activation shape or output layout")
    if not (a_log.numel() == hv and dt_bias.numel() == hv and weight.numel() == HEAD_DIM):
        raise RuntimeError("invalid weight shapes")
    requests = indices_shape[0]
    if not (cu.dim() == 1 and cu.numel() == requests + 1 and accepted.dim() == 1
            and accepted.numel() == requests):
        raise RuntimeError("invalid request metadata shapes")
    if not eps > 0:
        raise RuntimeError("norm epsilon must be positive")
    return (h, hv, dev, requests, indices_shape[1], qkv_stride[0], a.stride(0), b.stride(0),
            state_stride[0], gate_stride[0])


def check_decode(qkv, a, b, a_log, dt_bias, indices, cu, accepted, state, gate, weight, out, eps):
    """Validation of lightdelta::decode (reference csrc/gdn_decode.cu:366-403); returns
    (H, HV)."""
    return _decode_layout(qkv, a, b, a_log, dt_bias, indices, cu, accepted, state, gate, weight,
                          out, eps)[:2]


def check_prefill(qkv, a, b, a_log, dt_bias, slots, has_initial, cu_seqlens, state, gate,
                  weight, out, eps):
    """Validation of prefill: decode's activation, weight and state rules, with per-sequence
    metadata slots [N] int32, has_initial [N] bool and cu_seqlens [N+1] int32."""
    for t in (slots, cu_seqlens):
        _require(
            t.device == qkv.device and t.dtype == torch.int32 and t.dim() == 1
            and t.is_contiguous(),
            "metadata must be contiguous CUDA int32",
        )
    _require(
        has_initial.device == qkv.device and has_initial.dtype == torch.bool
        and has_initial.dim() == 1 and has_initial.is_contiguous(),
        "has_initial must be a contiguous CUDA bool vector",
    )
    _require(
        cu_seqlens.numel() == slots.numel() + 1 and has_initial.numel() == slots.numel(),
        "invalid sequence metadata shapes",
    )
    return check_decode(qkv, a, b, a_log, dt_bias, slots.view(-1, 1), cu_seqlens, slots, state,
                        gate, weight, out, eps)


# Prefill algorithm: "auto" runs chunks in the WY form, of 64 or 32 tokens, for the shapes
# where they are faster (ld_gdn_prefill_auto_chunked gives the chunk length, 0 for none),
# else the token-serial recurrence; "token_serial", "chunked" (64-token chunks) and
# "chunked_32" force one.  Results agree within rounding; the token-serial form reproduces
# the decode kernel bit for bit.
_PREFILL_ALGORITHMS = {"auto": _lib.PREFILL_AUTO, "token_serial": _lib.PREFILL_TOKEN_SERIAL,
                       "chunked": _lib.PREFILL_CHUNKED, "chunked_32": _lib.PREFILL_CHUNKED_32}
_prefill_algorithm = _lib.PREFILL_AUTO


def set_prefill_algorithm(name: str) -> None:
    global _prefill_algorithm
    if name not in _PREFILL_ALGORITHMS:
        raise ValueError(f"prefill algorithm must be one of {sorted(_PREFILL_ALGORITHMS)}")
    _prefill_algorithm = _PREFILL_ALGORITHMS[name]


def prefill_algorithm() -> str:
    return next(k for k, v in _PREFILL_ALGORITHMS.items() if v == _prefill_algorithm)


# Chunked-prefill workspaces of eager calls, one per (device, stream), kept and grown to the
# largest prefill seen (ld_gdn_prefill_workspace_bytes: 115,712 bytes per 64-token chunk and
# v-head, e.g. 2.0 GB for 32 x 1024 tokens at 32 v-heads).  Eager calls on one stream run in
# order, so they can share one; the buffer comes from torch's allocator once instead of on
# every call.  release_prefill_workspaces() drops them.
#
# A call under HIP-graph capture never touches this cache: the graph records the raw pointer
# and writes through it on every replay, so its workspace must stay the graph's for the
# graph's lifetime.  It gets a buffer of its own, allocated during the capture, which torch
# takes from the graph's private memory pool; that memory stays reserved for the graph's
# replays after the tensor is dropped (later allocations of the same capture may reuse it,
# which is stream-ordered after this call), and no eager call, cache growth or release can
# hand it to other tensors while the graph exists.
_workspaces: dict = {}


def _prefill_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index, _stream(device))
    buffer = _workspaces.get(key)
    if buffer is None or buffer.numel() < nbytes:
        _workspaces.pop(key, None)
        buffer = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _workspaces[key] = buffer
    return buffer


def release_prefill_workspaces() -> None:
    """Frees the cached chunked-prefill workspaces of eager calls (the next chunked prefill
    allocates again).  Captured graphs hold workspaces of their own and are unaffected."""
    _workspaces.clear()


def _prefill_impl(qkv, a, b, a_log, dt_bias, slots, has_initial, cu_seqlens, state, gate,
                  weight, out, eps):
    h, hv = check_prefill(qkv, a, b, a_log, dt_bias, slots, has_initial, cu_seqlens, state,
                          gate, weight, out, eps)
    if slots.numel() == 0:
        return
    lib = _lib.load()
    algorithm = _prefill_algorithm
    chunked = algorithm in (_lib.PREFILL_CHUNKED, _lib.PREFILL_CHUNKED_32) or (
        algorithm == _lib.PREFILL_AUTO
        and lib.ld_gdn_prefill_auto_chunked(qkv.shape[0], slots.numel(), hv) != 0)
    workspace = None
    if chunked:
        nbytes = lib.ld_gdn_prefill_workspace_bytes(qkv.shape[0], slots.numel(), hv)
        workspace = _prefill_workspace(qkv.device, nbytes)
    args = _lib.PrefillArgs(
        qkv.data_ptr(), qkv.stride(0), a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
        a_log.data_ptr(), dt_bias.data_ptr(), _dtype_code(dt_bias), _dtype_code(weight),
        slots.data_ptr(), has_initial.data_ptr(), cu_seqlens.data_ptr(), state.data_ptr(),
        state.stride(0), gate.data_ptr(), gate.stride(0), weight.data_ptr(), out.data_ptr(),
        qkv.shape[0], slots.numel(), h, hv, QK_SCALE, eps, algorithm,
        0 if workspace is None else workspace.data_ptr(),
        0 if workspace is None else workspace.numel(),
    )
    with _DeviceGuard(qkv.device):
        _lib.check(lib.ld_gdn_prefill(args, _stream(qkv.device)))


def _dtype_code(t: torch.Tensor) -> int:
    return _lib.DTYPE_BF16 if t.dtype == torch.bfloat16 else _lib.DTYPE_F32


def check_decode_conv(mixed_qkv, conv_state, conv_weight, conv_bias, a, b, a_log, dt_bias,
                      indices, cu, accepted, state, gate, weight, out, eps):
    """Validation of decode_conv: decode's checks on the pre-conv activations, plus the conv
    pool, weight and bias."""
    h, hv = check_decode(mixed_qkv, a, b, a_log, dt_bias, indices, cu, accepted, state, gate,
                         weight, out, eps)
    conv_dim = mixed_qkv.shape[1]
    _require(
        conv_state.device == mixed_qkv.device
        and conv_state.dtype == torch.bfloat16
        and conv_state.dim() == 3
        and conv_state.shape[1] == conv_dim
        and 3 <= conv_state.shape[2] <= 8,
        "conv_state must be CUDA BF16 [slots, conv_dim, 3..8]",
    )
    _require(
        conv_weight.device == mixed_qkv.device
        and conv_weight.dtype == torch.bfloat16
        and tuple(conv_weight.shape) == (conv_dim, 4)
        and conv_weight.is_contiguous()
        and conv_weight.data_ptr() % 8 == 0,
        "conv_weight must be contiguous CUDA BF16 [conv_dim, 4]",
    )
    if conv_bias is not None:
        _require(
            conv_bias.device == mixed_qkv.device
            and conv_bias.dtype == torch.bfloat16
            and conv_bias.numel() == conv_dim
            and conv_bias.is_contiguous(),
            "conv_bias must be contiguous CUDA BF16 [conv_dim]",
        )
    return h, hv


# ---------------------------------------------------------------------------------------
# state-pool copies: the checks of the C++ kernels (csrc/torch_ops.cpp), restated
# ---------------------------------------------------------------------------------------


def _dense_inner(t: torch.Tensor) -> bool:
    """Every dimension after the first is densely packed (row-major)."""
    expected = 1
    for size, stride in zip(reversed(t.shape[1:]), reversed(t.stride()[1:])):
        if size != 1 and stride != expected:
            return False
        expected *= size
    return True


def check_state_layout(pool, slots, packed, *, fp32_4d: bool):
    """The reference's `check` (csrc/state_io.cu:29-41); `fp32_4d=False` drops the fp32 /
    4-D requirement for the dtype-generic ops."""
    if fp32_4d:
        _require(
            _is_gpu(pool)
            and pool.dtype == torch.float32
            and pool.dim() == 4
            and pool.stride(3) == 1
            and pool.stride(2) == pool.shape[3]
            and pool.stride(1) == pool.shape[2] * pool.shape[3],
            "pool must be CUDA FP32 with dense inner dimensions",
        )
    else:
        _require(
            _is_gpu(pool) and pool.dim() >= 1 and _dense_inner(pool),
            "pool must be a CUDA tensor with dense inner dimensions",
        )
    _require(
        slots.device == pool.device and slots.dtype == torch.int32 and slots.dim() == 1,
        "slots must be a CUDA int32 vector",
    )
    _require(
        packed.device == pool.device
        and packed.dtype == pool.dtype
        and packed.dim() == pool.dim()
        and packed.shape[0] == slots.numel()
        and tuple(packed.shape[1:]) == tuple(pool.shape[1:])
        and _dense_inner(packed),
        "invalid packed layout",
    )


def _check_valid(valid, slots, pool):
    _require(
        valid.device == pool.device
        and valid.dtype == torch.bool
        and tuple(valid.shape) == tuple(slots.shape)
        and valid.is_contiguous(),
        "valid must be a CUDA bool vector",
    )


def check_copy(pool, src, dst):
    _require(
        _is_gpu(pool) and pool.dim() >= 1 and _dense_inner(pool),
        "pool must be a CUDA tensor with dense inner dimensions",
    )
    for t in (src, dst):
        _require(
            t.device == pool.device and t.dtype == torch.int32 and t.dim() == 1 and t.is_contiguous(),
            "src and dst must be contiguous CUDA int32 vectors",
        )
    _require(src.numel() == dst.numel(), "src and dst must have the same length")


def check_copy_checked(pool, src, dst, rejected):
    check_copy(pool, src, dst)
    _require(
        rejected.device == pool.device and rejected.dtype == torch.int32 and rejected.dim() == 1
        and rejected.is_contiguous() and rejected.numel() == src.numel(),
        "rejected must be a contiguous CUDA int32 vector with one entry per pair",
    )


def check_packed_plan(slots, cu, accepted, source, valid, indices, destinations):
    """Validation of packed_plan: int32 metadata [B, W] / [B + 1] / [B], outputs source [B]
    int32, valid [B] bool, indices [B, W] int32, destinations [B * W] int32, all contiguous
    on one device."""
    _require(
        _is_gpu(slots) and slots.dtype == torch.int32 and slots.dim() == 2
        and slots.is_contiguous() and 1 <= slots.shape[1] <= _lib.MAX_TOKENS,
        "slots must be a contiguous CUDA int32 [batch, 1..4] tensor",
    )
    batch, width = slots.shape
    for t, shape in ((cu, (batch + 1,)), (accepted, (batch,)), (source, (batch,)),
                     (indices, (batch, width)), (destinations, (batch * width,))):
        _require(
            t.device == slots.device and t.dtype == torch.int32 and tuple(t.shape) == shape
            and t.is_contiguous(),
            "packed_plan tensors must be contiguous CUDA int32 of the batch's shapes",
        )
    _require(
        valid.device == slots.device and valid.dtype == torch.bool
        and tuple(valid.shape) == (batch,) and valid.is_contiguous(),
        "valid must be a contiguous CUDA bool vector",
    )


def check_zero(pool, slots):
    _require(
        _is_gpu(pool) and pool.dim() >= 1 and _dense_inner(pool),
        "pool must be a CUDA tensor with dense inner dimensions",
    )
    _require(
        slots.device == pool.device and slots.dtype == torch.int32 and slots.dim() == 1
        and slots.is_contiguous(),
        "slots must be a contiguous CUDA int32 vector",
    )


# ---------------------------------------------------------------------------------------
# registration
# ---------------------------------------------------------------------------------------

# The per-step ops have C++ kernels (csrc/torch_ops.cpp, liblightdelta_torch.so): their host
# path is on every decode step.  prefill's kernel is the Python function below (it keeps the
# chunked form's workspace cache and the algorithm choice).
_CXX_KERNELS = ("decode", "decode_conv", "gather_state", "scatter_state", "gather_slots",
                "scatter_slots", "copy_state", "copy_state_checked", "zero_slots", "packed_plan")
_IMPLS = {
    "prefill": _prefill_impl,
}


def _fake(*args, **kwargs):
    return None


TORCH_KERNELS_PATH = Path(__file__).resolve().with_name("liblightdelta_torch.so")


def _not_built(*args, **kwargs):
    raise RuntimeError(f"{TORCH_KERNELS_PATH.name} is not built; run `python -m "
                       "lightdelta_amd.build` (hipcc, gfx950, and g++ against torch) before "
                       "using the lightdelta ops")


def _register():
    """Defines the ops, registers their fakes and their CUDA-key kernels: the C++ ones by
    loading liblightdelta_torch.so (with its liblightdelta_hip.so), the others from _IMPLS.
    Without the C++ library, decode and decode_conv raise."""
    library = torch.library.Library("lightdelta", "DEF")
    for name, schema in SCHEMAS.items():
        library.define(schema)
        torch.library.register_fake(f"lightdelta::{name}", _fake, lib=library)
        if name in _IMPLS:
            library.impl(name, _IMPLS[name], "CUDA")
    kernels = None
    if TORCH_KERNELS_PATH.exists():
        torch.ops.load_library(str(TORCH_KERNELS_PATH))
        kernels = ctypes.CDLL(str(TORCH_KERNELS_PATH))
        kernels.ld_torch_set_cache_policy.argtypes = [ctypes.c_int]
        kernels.ld_torch_set_cache_policy.restype = ctypes.c_int
        kernels.ld_torch_set_cache_policy(_cache_policy)
    else:
        for name in _CXX_KERNELS:
            library.impl(name, _not_built, "CUDA")
    return library, kernels


_LIBRARY, _TORCH_KERNELS = _register()
