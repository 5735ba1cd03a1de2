# SPDX-License-Identifier: Apache-2.0
"""Float64 restatement of the chunked (WY / UT) form of the gated delta rule, the algorithm
the K2 kernel implements. TEST HELPER: it is checked against the sequential oracle
(tests/test_chunk_form.py), and its two diagonal conventions can be flipped to plant the
mistakes the chunked fixtures must catch:

    akk_diag=False  A_kk strictly lower (correct); True keeps its diagonal (wrong)
    aqk_diag=True   A_qk lower including the diagonal (correct); False drops it (wrong)

Per chunk, with G_t = cumsum of g within the chunk and q already scaled:
    A_kk[t,s] = beta_t sum_i k_ti k_si exp(G_ti - G_si)   s < t
    A_qk[t,s] =        sum_i q_ti k_si exp(G_ti - G_si)   s <= t
    Tm = inv(I + A_kk);  W = Tm diag(beta) (K*exp(G));  U = Tm diag(beta) V
    Vn = U - W S;  O = (Q*exp(G)) S + A_qk Vn;  S' = exp(G_last) S + (K*exp(G_last-G))^T Vn
"""
from __future__ import annotations

import numpy as np


def chunked(q, k, v, g, beta, S0, q_scale, C=64, akk_diag=False, aqk_diag=True):
    """q,k,v,g [T,H,D]; beta [T,H]; S0 [H,D,D]. Returns o [T,H,D], S [H,D,D] (float64)."""
    T, H, D = q.shape
    q = q.astype(np.float64) * q_scale
    k, v, g = k.astype(np.float64), v.astype(np.float64), g.astype(np.float64)
    beta = beta.astype(np.float64)
    S = S0.astype(np.float64).copy()
    o = np.zeros((T, H, D))
    for h in range(H):
        for t0 in range(0, T, C):
            t1 = min(T, t0 + C)
            n = t1 - t0
            G = np.cumsum(g[t0:t1, h], axis=0)                       # [n, D]
            K, Q, V, B = k[t0:t1, h], q[t0:t1, h], v[t0:t1, h], beta[t0:t1, h]
            E = np.exp(G[:, None, :] - G[None, :, :])                # [t, s, i]
            kk = np.einsum("ti,si,tsi->ts", K, K, E)
            qk = np.einsum("ti,si,tsi->ts", Q, K, E)
            low = np.tril(np.ones((n, n)), 0 if akk_diag else -1)
            Akk = B[:, None] * kk * low
            Aqk = qk * np.tril(np.ones((n, n)), 0 if aqk_diag else -1)
            Tm = np.linalg.inv(np.eye(n) + Akk)
            W = Tm @ (B[:, None] * K * np.exp(G))
            U = Tm @ (B[:, None] * V)
            Vn = U - W @ S[h]
            o[t0:t1, h] = (Q * np.exp(G)) @ S[h] + Aqk @ Vn
            S[h] = np.exp(G[-1])[:, None] * S[h] + (K * np.exp(G[-1] - G)).T @ Vn
    return o, S
