"""CPU check of the chunked (UT / WY) gated-delta algebra used by the gfx950
chunk_prep / chunk_scan kernels, restated here in numpy step for step, against
the token-sequential oracle (cpp/reference/qwen35.cpp:459-518 via
oracle.delta_core).  Catches an algebra slip (a dropped decay term, a wrong
triangle, a transposed operand) without a GPU."""
import numpy as np
import pytest

from helpers import normal, rng, rel_l2
from oracle import pyoracle as orc

C = 64


def chunked_numpy(q, k, v, beta, g, q_scale, state, dtype=np.float64):
    T, hk, dk = q.shape
    hv, dv = v.shape[1:]
    S = state.astype(dtype).copy()
    out = np.zeros((T, hv, dv), dtype)
    for h in range(hv):
        kh = h % hk
        for t0 in range(0, T, C):
            L = min(C, T - t0)
            Q = q[t0:t0 + L, kh].astype(dtype) * q_scale
            K = k[t0:t0 + L, kh].astype(dtype)
            V = v[t0:t0 + L, h].astype(dtype)
            b = beta[t0:t0 + L, h].astype(dtype)
            G = np.cumsum(g[t0:t0 + L, h].astype(dtype))
            diff = G[:, None] - G[None, :]
            lower = np.tril(np.ones((L, L), bool), -1)
            M = np.where(np.tril(np.ones((L, L), bool)), np.exp(np.where(lower | np.eye(L, dtype=bool), diff, 0)) * (Q @ K.T), 0)
            A = np.where(lower, b[:, None] * np.exp(np.where(lower, diff, 0)) * (K @ K.T), 0)
            Tm = np.linalg.inv(np.eye(L) + A)
            W = Tm @ (b[:, None] * np.exp(G)[:, None] * K)
            U = Tm @ (b[:, None] * V)
            S0 = S[h]
            Dl = U - W @ S0
            out[t0:t0 + L, h] = np.exp(G)[:, None] * (Q @ S0) + M @ Dl
            Kt = np.exp(G[-1] - G)[:, None] * K
            S[h] = np.exp(G[-1]) * S0 + Kt.T @ Dl
    return out, S


@pytest.mark.parametrize("T,hk,hv,d", [(64, 1, 2, 16), (150, 2, 4, 32), (512, 2, 2, 128)])
def test_chunked_algebra_matches_sequential_oracle(T, hk, hv, d):
    r = rng(T + d)
    q = normal(r, T, hk, d)
    k = normal(r, T, hk, d)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = normal(r, T, hv, d)
    beta = 1 / (1 + np.exp(-normal(r, T, hv)))
    g = -np.log1p(np.exp(normal(r, T, hv)))
    state = normal(r, hv, d, d, scale=0.1)
    qs = 1 / np.sqrt(d)
    ref_o, ref_s = orc.delta_core(q, k, v, beta, g, qs, state)
    o, s = chunked_numpy(q, k, v, beta, g, qs, state)
    assert rel_l2(s, ref_s) < 1e-5
    assert rel_l2(o, ref_o) < 1e-5
