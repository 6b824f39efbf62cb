"""Independent formulations used only to pin the oracle (test infrastructure).

None of these retypes the recurrence of mixer.selective_scan; each computes
the same mathematical quantity by a different route, in float64, so that a
dropped term, a wrong sign, an off-by-one in time or a transposed operand in
the oracle fails at least one check in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np


def scan_closed_form(u, dt, A, B, C, h0=None):
    """Unrolled solution of h_t = exp(dt_t A) h_{t-1} + dt_t B_t u_t:

        h_t = exp(A * S(0,t)) h0 + sum_{s<=t} exp(A * S(s,t)) dt_s B_s u_s,
        S(s,t) = sum_{r=s+1..t} dt_r   (cumulative sums, no products of exps)

    and y_t = <h_t, C_t>.  dt is the post-softplus step [b,D,l]; B, C [b,l,N];
    A [D,N].  O(l^2) per channel, float64.  Returns (y [b,D,l], h_last)."""
    u = np.asarray(u, np.float64)
    dt = np.asarray(dt, np.float64)
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    b, D, l = u.shape
    N = A.shape[1]
    cs = np.concatenate([np.zeros((b, D, 1)), np.cumsum(dt, axis=-1)], axis=-1)  # cs[t+1] = sum_{r<=t}
    y = np.zeros((b, D, l))
    h = None
    for t in range(l):
        # S(s,t) = cs[t+1] - cs[s+1] for s <= t
        S = cs[:, :, t + 1:t + 2] - cs[:, :, 1:t + 2]                      # [b,D,t+1]
        w = np.exp(S[..., None] * A[None, :, None, :])                     # [b,D,t+1,N]
        src = (dt[:, :, :t + 1] * u[:, :, :t + 1])[..., None] * B[:, None, :t + 1, :]
        h = (w * src).sum(axis=2)                                          # [b,D,N]
        if h0 is not None:
            h = h + np.exp(cs[:, :, t + 1][..., None] * A[None]) * np.asarray(h0, np.float64)
        y[:, :, t] = np.einsum("bdn,bn->bd", h, C[:, t])
    return y, h


def conv_by_np_convolve(x, w, bias=None, conv_state=None):
    """Causal depthwise conv via numpy.convolve per (batch, channel):
    F.conv1d is a cross-correlation, so convolve with the flipped taps and keep
    the 'valid' part of the history-prefixed sequence.  float64."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    b, D, l = x.shape
    K = w.shape[1]
    out = np.zeros((b, D, l))
    for i in range(b):
        for d in range(D):
            hist = np.zeros(K - 1) if conv_state is None else np.asarray(conv_state[i, d], np.float64)
            seq = np.concatenate([hist, x[i, d]])
            out[i, d] = np.convolve(seq, w[d][::-1], mode="valid")
            if bias is not None:
                out[i, d] += bias[d]
    return out


def scan_geometric(dt, a, bx, c, l, h0=0.0):
    """Constant inputs: h_t = r h_{t-1} + q with r = exp(dt*a), q = dt*bx gives
    h_t = r^t h0 + q (1 - r^t) / (1 - r) (t = 1..l) and y_t = c h_t.  float64
    scalars; returns y [l]."""
    r = np.exp(dt * a)
    q = dt * bx
    t = np.arange(1, l + 1, dtype=np.float64)
    h = r ** t * h0 + q * (1 - r ** t) / (1 - r)
    return c * h
