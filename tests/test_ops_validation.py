"""Argument validation of the torch.ops.lightdelta impls raises the reference's messages
(csrc/gdn_decode.cu:367-403, csrc/state_io.cu:29-49).  Runs on CPU: tensors live on the
meta device and the impls' device predicate is pointed at it, so no kernel is reached."""

from __future__ import annotations

import pytest
import torch

from lightdelta_amd import ops


@pytest.fixture
def meta(monkeypatch):
    monkeypatch.setattr(ops, "_is_gpu", lambda t: t.device.type == "meta")
    return torch.device("meta")


def decode_args(device, n=4, h=16, hv=32, width=1, slots=10):
    def t(*shape, dtype=torch.bfloat16):
        return torch.empty(*shape, dtype=dtype, device=device)

    qkvz = t(n, (2 * h + hv) * 128 + hv * 128)
    ba = t(n, 2 * hv)
    args = dict(
        qkv=qkvz[:, : (2 * h + hv) * 128], a=ba[:, hv:], b=ba[:, :hv],
        a_log=t(hv, dtype=torch.float32), dt_bias=t(hv, dtype=torch.float32),
        indices=t(n // width, width, dtype=torch.int32), cu=t(n // width + 1, dtype=torch.int32),
        accepted=t(n // width, dtype=torch.int32), state=t(slots, hv, 128, 128, dtype=torch.float32),
        gate=qkvz[:, (2 * h + hv) * 128:].view(n, hv, 128), weight=t(128), out=t(n, hv, 128),
        eps=1e-6,
    )
    if torch.device(device).type != "meta":
        # Metadata that is safe even if a case were launched: every request's slots are
        # padding, so a kernel would only zero its outputs.
        args["indices"].zero_()
        args["cu"].copy_(torch.arange(0, n + 1, width, dtype=torch.int32))
        args["accepted"].fill_(1)
    return args


def conv_args(device, length=3, bias=True, **kw):
    """decode_conv's arguments: decode_args with qkv as the pre-conv activations, then the conv
    pool [slots, conv_dim, length], weight [conv_dim, 4] and bias [conv_dim], all bf16."""
    args = decode_args(device, **kw)
    conv_dim = args["qkv"].shape[1]
    slots = args["state"].shape[0]
    conv = dict(
        mixed_qkv=args.pop("qkv"),
        conv_state=torch.zeros(slots, conv_dim, length, dtype=torch.bfloat16, device=device),
        conv_weight=torch.zeros(conv_dim, 4, dtype=torch.bfloat16, device=device),
        conv_bias=(torch.zeros(conv_dim, dtype=torch.bfloat16, device=device) if bias else None),
    )
    conv.update(args)
    return conv


def check(args):
    return ops.check_decode(*args.values())


def test_valid_geometries(meta):
    assert check(decode_args(meta)) == (16, 32)
    assert check(decode_args(meta, h=16, hv=48)) == (16, 48)
    assert check(decode_args(meta, h=4, hv=8, width=4)) == (4, 8)


# Invalid decode arguments and the message each must raise: mutate(args, device) edits the
# valid arguments of decode_args(device).
DECODE_CASES = [
    (lambda d, m: d.update(qkv=d["qkv"].float()), "qkv must be CUDA BF16"),
    (lambda d, m: d.update(qkv=torch.empty(4, 8192, dtype=torch.bfloat16)), "qkv must be CUDA BF16"),
    (lambda d, m: d.update(a=d["a"].float()), "activations must be BF16"),
    (lambda d, m: d.update(gate=torch.empty(4, 32, 256, dtype=torch.bfloat16, device=m)[..., ::2]),
     "activations must be BF16 with dense rows"),
    (lambda d, m: d.update(out=torch.empty(32, 4, 128, dtype=torch.bfloat16, device=m).transpose(0, 1)),
     "invalid activation shape or output layout"),
    (lambda d, m: d.update(state=d["state"].double()), "state and A_log must be CUDA FP32"),
    (lambda d, m: d.update(a_log=d["a_log"].bfloat16()), "state and A_log must be CUDA FP32"),
    (lambda d, m: d.update(indices=d["indices"].long()), "metadata must be contiguous CUDA int32"),
    (lambda d, m: d.update(cu=torch.empty(10, dtype=torch.int32, device=m)[::2]),
     "metadata must be contiguous CUDA int32"),
    (lambda d, m: d.update(dt_bias=d["dt_bias"].half()), "weights must be contiguous FP32/BF16"),
    (lambda d, m: d.update(qkv=torch.empty(4, 10000, dtype=torch.bfloat16, device=m)), "qkv must be"),
    (lambda d, m: d.update(state=torch.empty(4, 32, 128, 64, device=m)), "state must be"),
    (lambda d, m: d.update(state=torch.empty(4, 128, 32, 128, device=m).transpose(1, 2)),
     "state must be"),
    (lambda d, m: d.update(indices=torch.empty(1, 5, dtype=torch.int32, device=m),
                           cu=torch.empty(2, dtype=torch.int32, device=m),
                           accepted=torch.empty(1, dtype=torch.int32, device=m)),
     "1 through 4 tokens"),
    (lambda d, m: d.update(a=torch.empty(4, 31, dtype=torch.bfloat16, device=m)),
     "invalid activation shape"),
    (lambda d, m: d.update(out=torch.empty(4, 32, 256, dtype=torch.bfloat16, device=m)[..., :128]),
     "activations must be BF16 with dense rows|invalid activation shape"),
    (lambda d, m: d.update(weight=torch.empty(64, dtype=torch.bfloat16, device=m)),
     "invalid weight shapes"),
    (lambda d, m: d.update(cu=torch.empty(4, dtype=torch.int32, device=m)),
     "invalid request metadata shapes"),
    (lambda d, m: d.update(eps=0.0), "norm epsilon must be positive"),
]


@pytest.mark.parametrize("mutate,message", DECODE_CASES)
def test_decode_validation_messages(meta, mutate, message):
    args = decode_args(meta)
    mutate(args, meta)
    with pytest.raises(RuntimeError, match=message):
        check(args)


# Invalid decode_conv arguments (on top of decode's) and the message each must raise.
CONV_DIM = (2 * 16 + 32) * 128
CONV_STATE_MSG = r"conv_state must be CUDA BF16 \[slots, conv_dim, 3..8\]"
CONV_WEIGHT_MSG = r"conv_weight must be contiguous CUDA BF16 \[conv_dim, 4\]"
CONV_BIAS_MSG = r"conv_bias must be contiguous CUDA BF16 \[conv_dim\]"
CONV_CASES = [
    (lambda d, m: d.update(conv_state=torch.zeros(10, CONV_DIM, 2, dtype=torch.bfloat16, device=m)),
     CONV_STATE_MSG),
    (lambda d, m: d.update(conv_state=torch.zeros(10, CONV_DIM, 9, dtype=torch.bfloat16, device=m)),
     CONV_STATE_MSG),
    (lambda d, m: d.update(conv_state=d["conv_state"].float()), CONV_STATE_MSG),
    (lambda d, m: d.update(conv_state=torch.zeros(10, CONV_DIM - 128, 3, dtype=torch.bfloat16,
                                                  device=m)), CONV_STATE_MSG),
    (lambda d, m: d.update(conv_state=d["conv_state"][:, :, 0]), CONV_STATE_MSG),
    (lambda d, m: d.update(conv_weight=d["conv_weight"].float()), CONV_WEIGHT_MSG),
    (lambda d, m: d.update(conv_weight=torch.zeros(4, CONV_DIM, dtype=torch.bfloat16,
                                                   device=m).t()), CONV_WEIGHT_MSG),
    (lambda d, m: d.update(conv_weight=torch.zeros(CONV_DIM, 3, dtype=torch.bfloat16, device=m)),
     CONV_WEIGHT_MSG),
    (lambda d, m: d.update(conv_bias=torch.zeros(CONV_DIM - 1, dtype=torch.bfloat16, device=m)),
     CONV_BIAS_MSG),
    (lambda d, m: d.update(conv_bias=d["conv_bias"].float()), CONV_BIAS_MSG),
    (lambda d, m: d.update(conv_bias=torch.zeros(2 * CONV_DIM, dtype=torch.bfloat16,
                                                 device=m)[::2]), CONV_BIAS_MSG),
    # decode's own checks still apply to the pre-conv activations
    (lambda d, m: d.update(mixed_qkv=d["mixed_qkv"].float()), "qkv must be CUDA BF16"),
]


def test_decode_conv_valid_arguments(meta):
    assert ops.check_decode_conv(*conv_args(meta).values()) == (16, 32)
    assert ops.check_decode_conv(*conv_args(meta, length=8, bias=False).values()) == (16, 32)
    dim_last = conv_args(meta)
    dim_last["conv_state"] = torch.zeros(10, 3, CONV_DIM, dtype=torch.bfloat16,
                                         device=meta).transpose(1, 2)
    assert ops.check_decode_conv(*dim_last.values()) == (16, 32)


@pytest.mark.parametrize("mutate,message", CONV_CASES)
def test_decode_conv_validation_messages(meta, mutate, message):
    args = conv_args(meta)
    mutate(args, meta)
    with pytest.raises(RuntimeError, match=message):
        ops.check_decode_conv(*args.values())


def test_copy_state_checked_validation_messages(meta):
    pool = torch.empty(8, 4, 128, 128, device=meta)
    src = torch.empty(3, dtype=torch.int32, device=meta)
    ops.check_copy_checked(pool, src, src, torch.empty(3, dtype=torch.int32, device=meta))
    for bad in (torch.empty(2, dtype=torch.int32, device=meta),
                torch.empty(3, dtype=torch.int64, device=meta),
                torch.empty(6, dtype=torch.int32, device=meta)[::2]):
        with pytest.raises(RuntimeError, match="rejected must be a contiguous CUDA int32 vector"):
            ops.check_copy_checked(pool, src, src, bad)
    with pytest.raises(RuntimeError, match="same length"):
        ops.check_copy_checked(pool, src, src[:2], src)


def test_packed_plan_validation_messages(meta):
    def plan(batch=4, width=2, **over):
        t = dict(slots=torch.empty(batch, width, dtype=torch.int32, device=meta),
                 cu=torch.empty(batch + 1, dtype=torch.int32, device=meta),
                 accepted=torch.empty(batch, dtype=torch.int32, device=meta),
                 source=torch.empty(batch, dtype=torch.int32, device=meta),
                 valid=torch.empty(batch, dtype=torch.bool, device=meta),
                 indices=torch.empty(batch, width, dtype=torch.int32, device=meta),
                 destinations=torch.empty(batch * width, dtype=torch.int32, device=meta))
        t.update(over)
        return t
    ops.check_packed_plan(*plan().values())
    with pytest.raises(RuntimeError, match=r"slots must be a contiguous CUDA int32 \[batch, 1..4\]"):
        ops.check_packed_plan(*plan(width=5).values())
    with pytest.raises(RuntimeError, match="slots must be"):
        ops.check_packed_plan(*plan(slots=torch.empty(4, 2, dtype=torch.int64, device=meta)).values())
    for name, bad in (("cu", torch.empty(4, dtype=torch.int32, device=meta)),
                      ("source", torch.empty(4, dtype=torch.int64, device=meta)),
                      ("indices", torch.empty(8, dtype=torch.int32, device=meta)),
                      ("destinations", torch.empty(4, 2, dtype=torch.int32, device=meta))):
        with pytest.raises(RuntimeError, match="packed_plan tensors must be"):
            ops.check_packed_plan(*plan(**{name: bad}).values())
    with pytest.raises(RuntimeError, match="valid must be a contiguous CUDA bool vector"):
        ops.check_packed_plan(*plan(valid=torch.empty(4, dtype=torch.uint8, device=meta)).values())


def test_state_io_validation_messages(meta):
    pool = torch.empty(8, 4, 128, 128, device=meta)
    slots = torch.empty(3, dtype=torch.int32, device=meta)
    packed = torch.empty(3, 4, 128, 128, device=meta)
    ops.check_state_layout(pool, slots, packed, fp32_4d=True)
    with pytest.raises(RuntimeError, match="pool must be CUDA FP32"):
        ops.check_state_layout(pool.bfloat16(), slots, packed, fp32_4d=True)
    with pytest.raises(RuntimeError, match="pool must be CUDA FP32"):
        ops.check_state_layout(torch.empty(8, 4, 128, 256, device=meta)[..., :128], slots, packed,
                               fp32_4d=True)
    with pytest.raises(RuntimeError, match="slots must be a CUDA int32 vector"):
        ops.check_state_layout(pool, slots.long(), packed, fp32_4d=True)
    with pytest.raises(RuntimeError, match="invalid packed layout"):
        ops.check_state_layout(pool, slots, packed[:2], fp32_4d=True)
    with pytest.raises(RuntimeError, match="valid must be a CUDA bool vector"):
        ops._check_valid(torch.empty(3, dtype=torch.int32, device=meta), slots, pool)
    conv = torch.empty(8, 4, 8192, dtype=torch.bfloat16, device=meta)
    ops.check_state_layout(conv, slots, torch.empty(3, 4, 8192, dtype=torch.bfloat16, device=meta),
                           fp32_4d=False)
    with pytest.raises(RuntimeError, match="invalid packed layout"):
        ops.check_state_layout(conv, slots, torch.empty(3, 4, 8192, device=meta), fp32_4d=False)
    with pytest.raises(RuntimeError, match="same length"):
        ops.check_copy(pool, slots, slots[:2])
    ops.check_zero(conv, slots)
    with pytest.raises(RuntimeError, match="slots must be a contiguous CUDA int32 vector"):
        ops.check_zero(pool, slots.long())
    with pytest.raises(RuntimeError, match="dense inner dimensions"):
        ops.check_zero(torch.empty(8, 4, 128, 256, device=meta)[..., :128], slots)


@pytest.mark.gpu
@pytest.mark.parametrize("mutate,message", DECODE_CASES + [
    (lambda d, m: d.update(qkv=d["qkv"].cpu()), "qkv must be CUDA BF16")])
def test_decode_kernel_validation_messages(gpu, mutate, message):
    """The same cases through torch.ops.lightdelta.decode on the GPU: the C++ kernel
    (csrc/torch_ops.cpp) raises the same messages, before any launch."""
    args = decode_args(gpu)
    mutate(args, gpu)
    with pytest.raises(RuntimeError, match=message):
        torch.ops.lightdelta.decode(*args.values())


@pytest.mark.gpu
def test_state_op_kernel_validation_messages(gpu):
    """The state-pool cases of test_state_io_validation_messages through the ops on the GPU:
    the C++ kernels (csrc/torch_ops.cpp) raise the same messages, before any launch."""
    ops_ = torch.ops.lightdelta
    pool = torch.zeros(8, 4, 128, 128, device=gpu)
    slots = torch.tensor([1, -1, 3], dtype=torch.int32, device=gpu)
    valid = torch.ones(3, dtype=torch.bool, device=gpu)
    packed = torch.zeros(3, 4, 128, 128, device=gpu)
    ops_.gather_state(pool, slots, valid, packed)
    ops_.scatter_state(packed, slots, pool)
    with pytest.raises(RuntimeError, match="pool must be CUDA FP32"):
        ops_.gather_state(pool.bfloat16(), slots, valid, packed.bfloat16())
    with pytest.raises(RuntimeError, match="pool must be CUDA FP32"):
        ops_.scatter_state(packed, slots, torch.zeros(8, 4, 128, 256, device=gpu)[..., :128])
    with pytest.raises(RuntimeError, match="slots must be a CUDA int32 vector"):
        ops_.gather_state(pool, slots.long(), valid, packed)
    with pytest.raises(RuntimeError, match="invalid packed layout"):
        ops_.scatter_state(packed[:2], slots, pool)
    with pytest.raises(RuntimeError, match="valid must be a CUDA bool vector"):
        ops_.gather_state(pool, slots, valid.int(), packed)
    conv = torch.zeros(8, 4, 8192, dtype=torch.bfloat16, device=gpu)
    conv_packed = torch.zeros(3, 4, 8192, dtype=torch.bfloat16, device=gpu)
    ops_.gather_slots(conv, slots, valid, conv_packed)
    ops_.scatter_slots(conv_packed, slots, conv)
    with pytest.raises(RuntimeError, match="invalid packed layout"):
        ops_.gather_slots(conv, slots, valid, torch.zeros(3, 4, 8192, device=gpu))
    with pytest.raises(RuntimeError, match="same length"):
        ops_.copy_state(pool, slots, slots[:2].contiguous())
    with pytest.raises(RuntimeError, match="src and dst must be contiguous CUDA int32 vectors"):
        ops_.copy_state(pool, slots.long(), slots)
    ops_.zero_slots(conv, slots)
    with pytest.raises(RuntimeError, match="slots must be a contiguous CUDA int32 vector"):
        ops_.zero_slots(pool, slots.long())
    with pytest.raises(RuntimeError, match="dense inner dimensions"):
        ops_.zero_slots(torch.zeros(8, 4, 128, 256, device=gpu)[..., :128], slots)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("mutate,message", CONV_CASES + [
    # a weight view 2 bytes into a buffer: contiguous, but not 8-byte aligned
    (lambda d, m: d.update(conv_weight=torch.zeros(CONV_DIM * 4 + 1, dtype=torch.bfloat16,
                                                   device=m)[1:].view(CONV_DIM, 4)),
     CONV_WEIGHT_MSG)])
def test_decode_conv_kernel_validation_messages(gpu, mutate, message):
    """The decode_conv cases through torch.ops.lightdelta.decode_conv on the GPU: the C++
    kernel (csrc/torch_ops.cpp) raises the same messages, before any launch (the metadata
    marks every request as padding, so even a launch would only zero the outputs)."""
    args = conv_args(gpu)
    mutate(args, gpu)
    with pytest.raises(RuntimeError, match=message):
        torch.ops.lightdelta.decode_conv(*args.values())
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_copy_state_checked_kernel_validation_messages(gpu):
    pool = torch.zeros(8, 4, 128, 128, device=gpu)
    src = torch.tensor([1, -1, 3], dtype=torch.int32, device=gpu)
    dst = torch.tensor([2, 4, -1], dtype=torch.int32, device=gpu)
    for bad in (torch.zeros(2, dtype=torch.int32, device=gpu),
                torch.zeros(3, dtype=torch.int64, device=gpu),
                torch.zeros(6, dtype=torch.int32, device=gpu)[::2]):
        with pytest.raises(RuntimeError, match="rejected must be a contiguous CUDA int32 vector"):
            torch.ops.lightdelta.copy_state_checked(pool, src, dst, bad)
    with pytest.raises(RuntimeError, match="same length"):
        torch.ops.lightdelta.copy_state_checked(pool, src, dst[:2].contiguous(),
                                                torch.zeros(3, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_packed_plan_kernel_validation_messages(gpu):
    i32 = dict(dtype=torch.int32, device=gpu)
    good = dict(slots=torch.zeros(4, 2, **i32), cu=torch.zeros(5, **i32),
                accepted=torch.zeros(4, **i32), source=torch.zeros(4, **i32),
                valid=torch.zeros(4, dtype=torch.bool, device=gpu),
                indices=torch.zeros(4, 2, **i32), destinations=torch.zeros(8, **i32))
    for name, bad, message in (
            ("slots", torch.zeros(4, 5, **i32), "slots must be a contiguous CUDA int32"),
            ("cu", torch.zeros(4, **i32), "packed_plan tensors must be"),
            ("destinations", torch.zeros(4, 2, **i32), "packed_plan tensors must be"),
            ("valid", torch.zeros(4, dtype=torch.uint8, device=gpu), "valid must be")):
        args = dict(good, **{name: bad})
        with pytest.raises(RuntimeError, match=message):
            torch.ops.lightdelta.packed_plan(*args.values())
    torch.cuda.synchronize()


def test_cpu_tensors_are_rejected():
    args = decode_args("cpu")
    with pytest.raises(RuntimeError, match="qkv must be CUDA BF16"):
        check(args)


def test_schemas_match_reference_strings():
    expected = {
        "decode": "decode(Tensor qkv, Tensor a, Tensor b, Tensor a_log, Tensor dt_bias, "
                  "Tensor indices, Tensor cu, Tensor accepted, Tensor(s!) state, Tensor gate, "
                  "Tensor weight, Tensor(o!) out, float eps) -> ()",
        "gather_state": "gather_state(Tensor pool, Tensor slots, Tensor valid, Tensor(o!) out) -> ()",
        "scatter_state": "scatter_state(Tensor packed, Tensor slots, Tensor(p!) pool) -> ()",
    }
    for name, schema in expected.items():
        assert ops.SCHEMAS[name] == schema
        assert str(getattr(torch.ops.lightdelta, name).default._schema) == "lightdelta::" + schema
