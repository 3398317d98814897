"""The chunked (WY) form of the delta rule that prefill_chunked.hip implements, restated in
float64 on the CPU and checked against the token-by-token recurrence of the oracle's
prepared inputs (oracle/gdn.py prepare: the reference's normalisation, decay and beta).

The restatement follows the kernels step for step: 64-token chunks with partial last
chunks, in-chunk cumulative log decay G, A = strict-lower(beta_i Gam_ij k_i.k_j), the four
16 x 16 diagonal blocks of I + A inverted and the blocked forward substitution for
W = (I+A)^-1 beta e^G k and U = (I+A)^-1 beta v, then per chunk
V_new = U - W S^T, O = (q e^G) S^T + P V_new, S' = e^G_last S + V_new^T (k e^(G_last - G)).
The 32-token form keeps T = (I+A)^-1 itself, built from its two diagonal blocks and
T10 = -T1 A10 T0, and forms V_new = T (diag(beta) v - diag(beta e^G) k S^T); its scan
multiplies the bf16 keys and queries by S (and by V_new's scaled rows) as three products
against an exact three-way bf16 split of the fp32 operand, which the split test pins.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn

C = 64
BLOCK = 16


def prepared_head(length: int, seed: int):
    """q, k, v [T, 128] (q scaled), log decay g [T] and beta [T] of one head, float64."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(1, length, 1, 128, generator=gen)
    k = torch.randn(1, length, 1, 128, generator=gen)
    v = torch.randn(1, length, 1, 128, generator=gen)
    a = torch.randn(1, length, 1, generator=gen)
    b = torch.randn(1, length, 1, generator=gen)
    p = gdn.prepare(q, k, v, a, b, torch.tensor([0.3]), torch.tensor([0.1]))
    as64 = lambda t: t[0, :, 0].double().numpy()  # noqa: E731
    return as64(p.q), as64(p.k), as64(p.v), np.log(as64(p.decay)), as64(p.beta)


def token_serial(q, k, v, g, beta, state):
    """The reference recurrence (gdn.py:110-116) in float64: outputs [T, 128], final state."""
    s = state.copy()
    out = np.empty((len(q), 128))
    for t in range(len(q)):
        s = s * np.exp(g[t])
        delta = (v[t] - s @ k[t]) * beta[t]
        s = s + np.outer(delta, k[t])
        out[t] = s @ q[t]
    return out, s


def lower_unit_inverse(a_block):
    """(I + A)^-1 for strictly lower A, one column at a time (the kernel's column form)."""
    n = len(a_block)
    t = np.eye(n)
    for m in range(n - 1):
        t[m + 1:] -= np.outer(a_block[m + 1:, m], t[m])
    return t


def chunked(q, k, v, g, beta, state, *, decay_state=True):
    """The kernels' chunked form in float64 (decay_state=False plants a mistake)."""
    s = state.copy()
    out = np.empty((len(q), 128))
    for t0 in range(0, len(q), C):
        n = min(C, len(q) - t0)
        # the kernels pad a partial chunk to 64 rows with beta = 0, q = k = 0, g = 0
        pad = lambda x, fill=0.0: np.concatenate([x[t0:t0 + n], np.full((C - n,) + x.shape[1:], fill)])  # noqa: E731
        qc, kc, vc, gc, bc = pad(q), pad(k), pad(v), pad(g), pad(beta)
        G = np.cumsum(gc)
        gam = np.exp(np.minimum(G[:, None] - G[None, :], 0.0))
        A = np.tril(bc[:, None] * gam * (kc @ kc.T), -1)
        P = np.tril(gam * (qc @ kc.T))
        rhs = np.concatenate([(bc * np.exp(G))[:, None] * kc, bc[:, None] * vc], axis=1)
        x = np.zeros_like(rhs)
        for rb in range(C // BLOCK):
            rows = slice(rb * BLOCK, (rb + 1) * BLOCK)
            y = rhs[rows] - A[rows, :rb * BLOCK] @ x[:rb * BLOCK]
            x[rows] = lower_unit_inverse(A[rows, rows]) @ y
        w, u = x[:, :128], x[:, 128:]
        vn = u - w @ s.T
        o = (qc * np.exp(G)[:, None]) @ s.T + P @ vn
        glast = G[n - 1]
        kd = kc * np.exp(glast - G)[:, None]
        s = (np.exp(glast) if decay_state else 1.0) * s + vn.T @ kd
        out[t0:t0 + n] = o[:n]
    return out, s


def chunked32(q, k, v, g, beta, state, *, t10_sign=-1.0):
    """The 32-token form in float64: T from the diagonal blocks' inverses and
    T10 = -T1 A10 T0 (t10_sign=+1 plants a sign mistake), V_new = T (beta v - beta e^G k S^T)."""
    c = 32
    s = state.copy()
    out = np.empty((len(q), 128))
    for t0 in range(0, len(q), c):
        n = min(c, len(q) - t0)
        pad = lambda x: np.concatenate([x[t0:t0 + n], np.zeros((c - n,) + x.shape[1:])])  # noqa: E731
        qc, kc, vc, gc, bc = pad(q), pad(k), pad(v), pad(g), pad(beta)
        G = np.cumsum(gc)
        gam = np.exp(np.minimum(G[:, None] - G[None, :], 0.0))
        A = np.tril(bc[:, None] * gam * (kc @ kc.T), -1)
        P = np.tril(gam * (qc @ kc.T))
        t_0 = lower_unit_inverse(A[:BLOCK, :BLOCK])
        t_1 = lower_unit_inverse(A[BLOCK:, BLOCK:])
        T = np.zeros((c, c))
        T[:BLOCK, :BLOCK] = t_0
        T[BLOCK:, BLOCK:] = t_1
        T[BLOCK:, :BLOCK] = t10_sign * t_1 @ A[BLOCK:, :BLOCK] @ t_0
        x = bc[:, None] * vc - (bc * np.exp(G))[:, None] * (kc @ s.T)
        vn = T @ x
        o = (qc * np.exp(G)[:, None]) @ s.T + P @ vn
        glast = G[n - 1]
        kd = kc * np.exp(glast - G)[:, None]
        s = np.exp(glast) * s + vn.T @ kd
        out[t0:t0 + n] = o[:n]
    return out, s


def bf16_rne(x):
    """float32 -> nearest bfloat16 (ties to even), returned as float32: the hardware's
    conversion the split uses."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def split3(x):
    """The kernel's split4 per value: s1 = RNE(x), s2 = RNE(x - s1), s3 = RNE(x - s1 - s2),
    each remainder taken in float32."""
    parts, r = [], np.asarray(x, np.float32)
    for _ in range(3):
        p = bf16_rne(r)
        parts.append(p)
        r = (r - p).astype(np.float32)
    return parts


@pytest.mark.parametrize("length", [1, 31, 32, 33, 100])
@pytest.mark.parametrize("from_zero", [True, False])
def test_32_token_form_equals_token_serial(length, from_zero):
    q, k, v, g, beta = prepared_head(length, seed=100 + length)
    rng = np.random.default_rng(length)
    state = np.zeros((128, 128)) if from_zero else rng.normal(0.0, 0.05, (128, 128))
    ref_out, ref_state = token_serial(q, k, v, g, beta, state)
    out, s = chunked32(q, k, v, g, beta, state)
    assert np.abs(out - ref_out).max() <= 1e-10 * np.abs(ref_out).max()
    assert np.abs(s - ref_state).max() <= 1e-10 * np.abs(ref_state).max()


def test_a_wrong_t10_sign_is_caught():
    """A planted mistake (T10 = +T1 A10 T0) breaks the 32-token form's agreement: the
    outputs of each chunk's second token tile move by about 1% (the final state, dominated
    by the last tokens' decayed contributions, by far less)."""
    q, k, v, g, beta = prepared_head(64, seed=7)
    state = np.random.default_rng(7).normal(0.0, 0.05, (128, 128))
    ref_out, ref_state = token_serial(q, k, v, g, beta, state)
    out, s = chunked32(q, k, v, g, beta, state, t10_sign=1.0)
    assert np.abs(out - ref_out).max() > 1e-3 * np.abs(ref_out).max()


def test_three_way_bf16_split_is_exact():
    """Every float32 of normal magnitude is the sum of its three bf16 parts, the sum in
    float32 as (s1 + s2) + s3 rejoins it exactly, and a product with an exact bf16 operand
    summed over the parts equals the float32 operand's product (float64 sums); a two-way
    split does not."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-40, 40, 200_000))).astype(np.float32)
    x = np.concatenate([x, np.float32([1.0, -1.0, 1 / 3, np.pi, 65504.0, 1.1754944e-38 * 2**20])])
    s1, s2, s3 = split3(x)
    assert np.all(bf16_rne(s1) == s1) and np.all(bf16_rne(s2) == s2) and np.all(bf16_rne(s3) == s3)
    assert np.array_equal(((s1 + s2).astype(np.float32) + s3).astype(np.float32), x)
    assert np.array_equal(s1.astype(np.float64) + s2 + s3, x.astype(np.float64))
    a = bf16_rne(rng.standard_normal(128).astype(np.float32)).astype(np.float64)
    rows = rng.standard_normal((64, 128)).astype(np.float32)
    parts = split3(rows)
    exact = rows.astype(np.float64) @ a
    assert np.array_equal(sum(p.astype(np.float64) @ a for p in parts), exact)
    two_way = (parts[0].astype(np.float64) + parts[1]) @ a
    assert np.abs(two_way - exact).max() > 0


@pytest.mark.parametrize("length", [1, 37, 64, 65, 200])
@pytest.mark.parametrize("from_zero", [True, False])
def test_chunked_form_equals_token_serial(length, from_zero):
    q, k, v, g, beta = prepared_head(length, seed=length)
    rng = np.random.default_rng(length)
    state = np.zeros((128, 128)) if from_zero else rng.normal(0.0, 0.05, (128, 128))
    ref_out, ref_state = token_serial(q, k, v, g, beta, state)
    out, s = chunked(q, k, v, g, beta, state)
    scale_o = np.abs(ref_out).max()
    scale_s = np.abs(ref_state).max()
    assert np.abs(out - ref_out).max() <= 1e-10 * scale_o
    assert np.abs(s - ref_state).max() <= 1e-10 * scale_s


def test_a_missing_state_decay_is_caught():
    """A planted mistake (no e^G_last on the carried state) breaks the agreement."""
    q, k, v, g, beta = prepared_head(130, seed=3)
    state = np.random.default_rng(3).normal(0.0, 0.05, (128, 128))
    ref_out, ref_state = token_serial(q, k, v, g, beta, state)
    out, s = chunked(q, k, v, g, beta, state, decay_state=False)
    assert np.abs(s - ref_state).max() > 1e-3 * np.abs(ref_state).max()
