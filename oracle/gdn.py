"""Gated-delta-rule oracle (test infrastructure only; float64).

``gdn_slot_step`` restates ``src/hs_guard/engine/fused_kernels.py:140-211`` (``gdn_slot_v8``), which has the
same recurrence as ``gdn_slot_kernel.py:10-73``. Per row n with ``lens[n] > 0`` and value head hv
(key head ``hv // (HV // H)``), for each real token t::

    q = l2norm(q) * K**-0.5,  k = l2norm(k)            (eps 1e-6 inside the sqrt, :170-171)
    g = -exp(A_log) * softplus(a + dt_bias)             (softplus threshold 20, :172-173)
    beta = sigmoid(b)                                   (:174)
    S *= exp(g);  v' = beta * (v - S^T k);  S += k v'^T;  o = S^T q       (:175-178)

Rows with ``lens == 0`` neither read nor write the state (:154, :194); padded positions of ``o`` are zero
(:189-193); ``sq = bf16(o)**2`` (:180-181).

``gdn_chunk`` is the WY/UT chunk form of the same recurrence (the algorithm behind FLA's
``chunk_gated_delta_rule``, called at ``runtime.py:80-89`` / ``bucketed_engine.py:109-111``; FLA 0.5.2 is
not vendored). It restates the published chunk algorithm, as also written out in transformers'
``torch_chunk_gated_delta_rule`` (qwen3_5/modeling_qwen3_5.py:249-327). ``gdn_slot_step_chunked`` is
``gdn_slot_step`` evaluated through ``gdn_chunk``.

Pinning (``tests/test_oracle_gdn.py``): transformers' ``torch_recurrent_gated_delta_rule`` and
``torch_chunk_gated_delta_rule`` (library routines); closed forms (beta=0 pure decay; zero state and one
token gives ``beta (k.q) v``; orthonormal keys written once are recalled exactly); affinity in the initial
state; chunked == recurrent for several chunk splits; the lens==0 / padding contract.
"""
import numpy as np

from .bf16 import bf16


def softplus_ref(x):
    """where(x > 20, x, log(1 + exp(x))) (fused_kernels.py:173)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log(1.0 + np.exp(np.minimum(x, 20.0))))


def l2norm(x, eps=1e-6):
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def gates(a, b, A_log, dt_bias):
    """(g, beta) of the kernel contract from raw projections a, b [..., HV]."""
    A = np.exp(np.asarray(A_log, dtype=np.float64))
    g = -A * softplus_ref(np.asarray(a, dtype=np.float64) + np.asarray(dt_bias, dtype=np.float64))
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, dtype=np.float64)))
    return g, beta


def gdn_slot_step(packed, key_dim, heads, head_k, value_heads, head_v, a, b, A_log, dt_bias, state, slots,
                  lens, scale=None):
    """packed [N, L, 2*key_dim + HV*V]; a, b [N, L, HV]; state [S, HV, K, V] (not modified).

    Returns (o [N, L, HV, V] float64 unrounded, sq [N, L, HV, V] = bf16(o)**2, new_state float64 copy).
    """
    packed = np.asarray(packed, dtype=np.float64)
    N, L, _ = packed.shape
    H, K, HV, V = heads, head_k, value_heads, head_v
    scale = K ** -0.5 if scale is None else scale
    st = np.array(state, dtype=np.float64, copy=True)
    slots = np.asarray(slots, dtype=np.int64)
    lens = np.asarray(lens, dtype=np.int64)
    o = np.zeros((N, L, HV, V))
    kh = np.arange(HV) // (HV // H)
    live = np.nonzero(lens > 0)[0]
    if len(live) == 0:
        return o, bf16(o).astype(np.float64) ** 2, st
    S = st[slots[live]]                                     # [R, HV, K, V]
    g_all, beta_all = gates(np.asarray(a)[live], np.asarray(b)[live], A_log, dt_bias)
    for t in range(int(lens[live].max())):
        on = np.nonzero(lens[live] > t)[0]                  # rows still running (only they are computed)
        rows = live[on]
        q = packed[rows, t, :key_dim].reshape(-1, H, K)[:, kh]
        k = packed[rows, t, key_dim:2 * key_dim].reshape(-1, H, K)[:, kh]
        v = packed[rows, t, 2 * key_dim:2 * key_dim + HV * V].reshape(-1, HV, V)
        q = l2norm(q) * scale
        k = l2norm(k)
        Sr = S[on] * np.exp(g_all[on, t])[:, :, None, None]
        kv = np.einsum('rhkv,rhk->rhv', Sr, k)
        vn = beta_all[on, t][:, :, None] * (v - kv)
        Sr += k[:, :, :, None] * vn[:, :, None, :]
        o[rows, t] = np.einsum('rhkv,rhk->rhv', Sr, q)
        S[on] = Sr
    st[slots[live]] = S
    return o, bf16(o).astype(np.float64) ** 2, st


def gdn_recurrent_seq(q, k, v, g, beta, S0, scale=None, normalize=True):
    """One sequence, all heads: q, k [T, H, K]; v [T, H, V]; g, beta [T, H]; S0 [H, K, V] -> (o [T,H,V], S)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    K = q.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    if normalize:
        q, k = l2norm(q), l2norm(k)
    q = q * scale
    S = np.array(S0, dtype=np.float64, copy=True)
    out = np.zeros(v.shape)
    for t in range(q.shape[0]):
        S *= np.exp(g[t])[:, None, None]
        vn = beta[t][:, None] * (v[t] - np.einsum('hkv,hk->hv', S, k[t]))
        S += k[t][:, :, None] * vn[:, None, :]
        out[t] = np.einsum('hkv,hk->hv', S, q[t])
    return out, S


def gdn_chunk(q, k, v, g, beta, S0, chunk=64, scale=None, normalize=True):
    """WY/UT chunk form. Shapes as ``gdn_recurrent_seq``. Returns (o [T, H, V], S [H, K, V]).

    Per chunk with in-chunk cumulative log-decay G (G_i = sum_{j<=i} g_j):
      A[i, j] = beta_i (k_i . k_j) exp(G_i - G_j)   for j < i      (strictly lower)
      T = (I + A)^-1                                                (unit lower triangular)
      W = T (beta * exp(G) * K),  U = T (beta * V)
      V' = U - W S
      O = (Q * exp(G)) S + ((Q K^T) * exp(G_i - G_j) [j <= i]) V'
      S <- exp(G_C) S + (K * exp(G_C - G))^T V'
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    beta = np.asarray(beta, dtype=np.float64)
    T, H, K = q.shape
    scale = K ** -0.5 if scale is None else scale
    if normalize:
        q, k = l2norm(q), l2norm(k)
    q = q * scale
    S = np.array(S0, dtype=np.float64, copy=True)          # [H, K, V]
    out = np.zeros(v.shape)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        C = c1 - c0
        Q = np.ascontiguousarray(q[c0:c1].transpose(1, 0, 2))      # [H, C, K]
        Kc = np.ascontiguousarray(k[c0:c1].transpose(1, 0, 2))
        Vc = np.ascontiguousarray(v[c0:c1].transpose(1, 0, 2))     # [H, C, V]
        G = np.cumsum(g[c0:c1].T, axis=1)                   # [H, C]
        bt = beta[c0:c1].T                                  # [H, C]
        diff = G[:, :, None] - G[:, None, :]                # [H, C, C]
        lower = np.tril(np.ones((C, C), dtype=bool), -1)
        causal = np.tril(np.ones((C, C), dtype=bool))
        KT = np.ascontiguousarray(Kc.transpose(0, 2, 1))
        KK = Kc @ KT
        A = np.where(lower, bt[:, :, None] * KK * np.exp(np.where(lower, diff, 0.0)), 0.0)
        Tm = np.linalg.inv(np.eye(C) + A)
        Wm = Tm @ ((bt * np.exp(G))[:, :, None] * Kc)
        Um = Tm @ (bt[:, :, None] * Vc)
        Vn = Um - Wm @ S
        P = np.where(causal, (Q @ KT) * np.exp(np.where(causal, diff, 0.0)), 0.0)
        out[c0:c1] = ((Q * np.exp(G)[:, :, None]) @ S + P @ Vn).transpose(1, 0, 2)
        Kd = np.ascontiguousarray((Kc * np.exp(G[:, -1:] - G)[:, :, None]).transpose(0, 2, 1))
        S = np.exp(G[:, -1])[:, None, None] * S + Kd @ Vn
    return out, S


def gdn_slot_step_chunked(packed, key_dim, heads, head_k, value_heads, head_v, a, b, A_log, dt_bias, state, slots,
                          lens, scale=None, chunk=64):
    """``gdn_slot_step`` (same arguments and returns) evaluated per live row in the chunk form ``gdn_chunk``.

    Both are float64 evaluations of one recurrence (fused_kernels.py:166-188), so they agree to float64
    rounding (``tests/test_oracle_gdn.py`` holds them to 1e-10); the chunk form replaces the per-token state
    updates of a long row by a few matrix products per 64 tokens, which is what makes full-geometry ticks of
    many-token rows affordable on the CPU."""
    packed = np.asarray(packed, dtype=np.float64)
    N, L, _ = packed.shape
    H, K, HV, V = heads, head_k, value_heads, head_v
    scale = K ** -0.5 if scale is None else scale
    st = np.array(state, dtype=np.float64, copy=True)
    slots = np.asarray(slots, dtype=np.int64)
    lens = np.asarray(lens, dtype=np.int64)
    o = np.zeros((N, L, HV, V))
    kh = np.arange(HV) // (HV // H)
    g_all, beta_all = gates(a, b, A_log, dt_bias)
    for n in np.nonzero(lens > 0)[0]:
        T = int(lens[n])
        q = packed[n, :T, :key_dim].reshape(T, H, K)[:, kh]
        k = packed[n, :T, key_dim:2 * key_dim].reshape(T, H, K)[:, kh]
        v = packed[n, :T, 2 * key_dim:2 * key_dim + HV * V].reshape(T, HV, V)
        o[n, :T], st[slots[n]] = gdn_chunk(q, k, v, g_all[n, :T], beta_all[n, :T], st[slots[n]], chunk=chunk,
                                           scale=scale)
    return o, bf16(o).astype(np.float64) ** 2, st
