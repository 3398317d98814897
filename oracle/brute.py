"""fp64 per-element brute force of the post-conv GDN -- test infrastructure, tiny shapes.

Written from the delta-rule definition rather than from oracle/gdn.py (plain Python loops,
float64 throughout, no tensor broadcasting), so that a transposed operand, a dropped term, a
wrong sign or a misplaced decay in either one shows up as a disagreement:

    S_t = decay_t * S_{t-1} + beta_t * (v_t - (decay_t * S_{t-1}) k_t) k_t^T     (S is V x K)
    raw_t = round_bf16(S_t q_t)           out_t = raw_t / rms(raw_t) * w * silu(gate_t)

with q_t, k_t L2-normalised (+1e-6 inside the root), q_t scaled by K^-1/2, and
decay_t = exp(-exp(A_log) * softplus(a_t + dt_bias)), beta_t = sigmoid(b_t).
Inputs are numpy arrays (any float dtype); output rounding to bf16 is optional so callers can
compare before or after it.
"""

from __future__ import annotations

import math

import numpy as np


def bf16_round(x: float) -> float:
    """Round a float to the nearest bfloat16 (ties to even), via fp32."""
    f = np.array([x], dtype=np.float32).view(np.uint32)[0]
    if (int(f) & 0x7FFFFFFF) > 0x7F800000:
        return float("nan")
    f = (int(f) + 0x7FFF + ((int(f) >> 16) & 1)) & 0xFFFF0000
    return float(np.array([f], dtype=np.uint32).view(np.float32)[0])


def _softplus(x: float) -> float:
    return x if x > 20.0 else math.log1p(math.exp(x))


def _sigmoid(x: float) -> float:
    return 1.0 / (1.0 + math.exp(-x))


def run(q, k, v, a, b, a_log, dt_bias, gate, norm_weight, initial_state, lengths,
        *, norm_eps=1e-6, round_raw=True):
    """Shapes as oracle.gdn.run (numpy).  Returns (out [B,T,Hv,V] fp64 before the final cast,
    final_state [B,Hv,V,K] fp64, states [B,T+1,Hv,V,K] fp64)."""
    B, T, Hk, K = q.shape
    Hv, V = v.shape[2:]
    group = Hv // Hk
    out = np.zeros((B, T, Hv, V))
    states = np.zeros((B, T + 1, Hv, V, K))
    for r in range(B):
        for h in range(Hv):
            kh = h // group
            S = [[float(initial_state[r, h, i, j]) for j in range(K)] for i in range(V)]
            states[r, 0, h] = S
            for t in range(T):
                if t >= int(lengths[r]):
                    states[r, t + 1, h] = S
                    continue
                qv = [float(q[r, t, kh, j]) for j in range(K)]
                kv = [float(k[r, t, kh, j]) for j in range(K)]
                qn = 1.0 / math.sqrt(sum(x * x for x in qv) + 1e-6)
                kn = 1.0 / math.sqrt(sum(x * x for x in kv) + 1e-6)
                qv = [x * qn / math.sqrt(K) for x in qv]
                kv = [x * kn for x in kv]
                decay = math.exp(-math.exp(float(a_log[h])) *
                                 _softplus(float(a[r, t, h]) + float(dt_bias[h])))
                beta = _sigmoid(float(b[r, t, h]))
                for i in range(V):
                    row = [decay * S[i][j] for j in range(K)]
                    pred = sum(row[j] * kv[j] for j in range(K))
                    delta = beta * (float(v[r, t, h, i]) - pred)
                    S[i] = [row[j] + delta * kv[j] for j in range(K)]
                raw = [sum(S[i][j] * qv[j] for j in range(K)) for i in range(V)]
                if round_raw:
                    raw = [bf16_round(x) for x in raw]
                rstd = 1.0 / math.sqrt(sum(x * x for x in raw) / V + norm_eps)
                for i in range(V):
                    g = float(gate[r, t, h, i])
                    out[r, t, h, i] = raw[i] * rstd * float(norm_weight[i]) * g * _sigmoid(g)
                states[r, t + 1, h] = S
    return out, states[:, T], states
