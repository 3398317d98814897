"""The chunked (WY) form of the delta rule that prefill_chunked.hip implements, restated in
float64 on the CPU and checked against the token-by-token recurrence of the oracle's
prepared inputs (oracle/gdn.py prepare: the reference's normalisation, decay and beta).

The restatement follows the kernels step for step: 64-token chunks with partial last
chunks, in-chunk cumulative log decay G, A = strict-lower(beta_i Gam_ij k_i.k_j), the four
16 x 16 diagonal blocks of I + A inverted and the blocked forward substitution for
W = (I+A)^-1 beta e^G k and U = (I+A)^-1 beta v, then per chunk
V_new = U - W S^T, O = (q e^G) S^T + P V_new, S' = e^G_last S + V_new^T (k e^(G_last - G)).
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
