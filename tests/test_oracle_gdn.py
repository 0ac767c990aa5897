"""Pins the GDN oracle (recurrent slot step and chunked WY/UT form) -- CPU only.

Anchors: transformers' torch_recurrent_gated_delta_rule / torch_chunk_gated_delta_rule (library routines
of the model family the reference builds on), closed forms and invariants of the recurrence.
"""
import numpy as np
import pytest

from oracle import gdn as ogdn

torch = pytest.importorskip("torch")


def _hf():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m
    return m


def _rand_seq(rng, T=37, H=3, K=16, V=8):
    q = rng.standard_normal((T, H, K))
    k = rng.standard_normal((T, H, K))
    v = rng.standard_normal((T, H, V))
    g = -np.log1p(np.exp(rng.standard_normal((T, H))))
    beta = 1 / (1 + np.exp(-rng.standard_normal((T, H))))
    S0 = rng.standard_normal((H, K, V)) * 0.1
    return q, k, v, g, beta, S0


def test_recurrent_matches_transformers():
    m = _hf()
    rng = np.random.default_rng(0)
    q, k, v, g, beta, S0 = _rand_seq(rng)
    o, S = ogdn.gdn_recurrent_seq(q, k, v, g, beta, S0)
    t = lambda x: torch.from_numpy(x)[None]
    o_hf, S_hf = m.torch_recurrent_gated_delta_rule(t(q), t(k), t(v), t(g), t(beta), initial_state=t(S0),
                                                    output_final_state=True, use_qk_l2norm_in_kernel=True)
    # transformers computes in float32 (it casts its inputs): compare at fp32 precision
    np.testing.assert_allclose(o, o_hf[0].numpy(), rtol=1e-5, atol=1e-6 * np.abs(o).max())
    np.testing.assert_allclose(S, S_hf[0].numpy(), rtol=1e-5, atol=1e-6 * np.abs(S).max())


@pytest.mark.parametrize("chunk", [64, 16, 5])
def test_chunk_matches_transformers_and_recurrent(chunk):
    m = _hf()
    rng = np.random.default_rng(1)
    q, k, v, g, beta, S0 = _rand_seq(rng, T=150)
    o_c, S_c = ogdn.gdn_chunk(q, k, v, g, beta, S0, chunk=chunk)
    o_r, S_r = ogdn.gdn_recurrent_seq(q, k, v, g, beta, S0)
    np.testing.assert_allclose(o_c, o_r, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(S_c, S_r, rtol=1e-9, atol=1e-11)
    t = lambda x: torch.from_numpy(x)[None]
    o_hf, S_hf = m.torch_chunk_gated_delta_rule(t(q), t(k), t(v), t(g), t(beta), chunk_size=chunk,
                                                initial_state=t(S0), output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    np.testing.assert_allclose(o_c, o_hf[0].numpy(), rtol=1e-4, atol=1e-5 * np.abs(o_c).max())
    np.testing.assert_allclose(S_c, S_hf[0].numpy(), rtol=1e-4, atol=1e-5 * np.abs(S_c).max())


def _slot_inputs(rng, N=3, L=4, H=2, HV=4, K=128):
    C = 2 * H * K + HV * K
    packed = rng.standard_normal((N, L, C))
    a = rng.standard_normal((N, L, HV))
    b = rng.standard_normal((N, L, HV))
    A_log = rng.standard_normal(HV) * 0.3
    dt = rng.standard_normal(HV) * 0.3
    state = rng.standard_normal((N + 2, HV, K, K)) * 0.05
    return packed, a, b, A_log, dt, state


def test_slot_step_matches_per_sequence_recurrence():
    """gdn_slot_step (the kernel contract: packed layout, raw a/b, GQA head map) equals the sequence form
    with g, beta from the gate formula, and touches only the rows' slots."""
    rng = np.random.default_rng(2)
    H, HV, K = 2, 4, 128
    packed, a, b, A_log, dt, state = _slot_inputs(rng, H=H, HV=HV)
    slots, lens = np.array([3, 0, 4]), np.array([4, 2, 0])
    o, sq, st = ogdn.gdn_slot_step(packed, H * K, H, K, HV, K, a, b, A_log, dt, state, slots, lens)
    g, beta = ogdn.gates(a, b, A_log, dt)
    kh = np.arange(HV) // (HV // H)
    for n in range(3):
        T = lens[n]
        q = packed[n, :T, :H * K].reshape(T, H, K)[:, kh]
        k = packed[n, :T, H * K:2 * H * K].reshape(T, H, K)[:, kh]
        v = packed[n, :T, 2 * H * K:].reshape(T, HV, K)
        o_s, S_s = ogdn.gdn_recurrent_seq(q, k, v, g[n, :T], beta[n, :T], state[slots[n]])
        np.testing.assert_allclose(o[n, :T], o_s, rtol=1e-12, atol=1e-14)
        assert (o[n, T:] == 0).all()
        np.testing.assert_allclose(st[slots[n]], S_s, rtol=1e-12, atol=1e-14)
    for s in (1, 2):
        np.testing.assert_array_equal(st[s], state[s])


def test_closed_forms():
    rng = np.random.default_rng(3)
    T, H, K, V = 5, 2, 16, 8
    q = rng.standard_normal((T, H, K))
    k = rng.standard_normal((T, H, K))
    v = rng.standard_normal((T, H, V))
    g = -np.abs(rng.standard_normal((T, H)))
    S0 = rng.standard_normal((H, K, V))
    # beta = 0: pure decay, o_t = S_t^T q_t with S_t = exp(sum g) S0
    o, S = ogdn.gdn_recurrent_seq(q, k, v, g, np.zeros((T, H)), S0)
    decay = np.exp(np.cumsum(g, 0))
    qn = ogdn.l2norm(q) * K ** -0.5
    for t in range(T):
        np.testing.assert_allclose(o[t], np.einsum('hkv,hk->hv', S0 * decay[t][:, None, None], qn[t]), rtol=1e-12)
    np.testing.assert_allclose(S, S0 * decay[-1][:, None, None], rtol=1e-12)
    # zero state, one token: o = beta (k.q) v
    beta = rng.uniform(0.1, 0.9, (1, H))
    o1, _ = ogdn.gdn_recurrent_seq(q[:1], k[:1], v[:1], g[:1], beta, np.zeros((H, K, V)))
    kn = ogdn.l2norm(k[:1])
    expect = beta[0][:, None] * (kn[0] * qn[0]).sum(-1)[:, None] * v[0]
    np.testing.assert_allclose(o1[0], expect, rtol=1e-12)
    # g = 0, beta = 1, orthonormal keys written once: recall S^T k_i = v_i / sqrt(1 + eps) (the l2norm eps
    # sits inside the square root, fused_kernels.py:171)
    Q, _ = np.linalg.qr(rng.standard_normal((K, K)))
    keys = Q[:4].reshape(4, 1, K)
    vals = rng.standard_normal((4, 1, V))
    _, S = ogdn.gdn_recurrent_seq(keys, keys, vals, np.zeros((4, 1)), np.ones((4, 1)), np.zeros((1, K, V)))
    for i in range(4):
        np.testing.assert_allclose(S[0].T @ keys[i, 0], vals[i, 0] / np.sqrt(1 + 1e-6), rtol=1e-12, atol=1e-13)


def test_affine_in_initial_state():
    """For fixed inputs the map S0 -> (o, S) is affine: f(S0 + d) - f(S0) is linear in d."""
    rng = np.random.default_rng(4)
    q, k, v, g, beta, S0 = _rand_seq(rng, T=9)
    d1 = rng.standard_normal(S0.shape)
    d2 = rng.standard_normal(S0.shape)
    f = lambda s: ogdn.gdn_recurrent_seq(q, k, v, g, beta, s)
    o0, s0 = f(S0)
    o1, s1 = f(S0 + d1)
    o2, s2 = f(S0 + d2)
    o12, s12 = f(S0 + d1 + d2)
    np.testing.assert_allclose(o12 - o0, (o1 - o0) + (o2 - o0), atol=1e-10)
    np.testing.assert_allclose(s12 - s0, (s1 - s0) + (s2 - s0), atol=1e-10)


def test_tick_size_invariance():
    """Running a row as 1-token ticks or as one multi-token tick gives the same outputs and state."""
    rng = np.random.default_rng(5)
    H, HV, K = 2, 2, 128
    packed, a, b, A_log, dt, state = _slot_inputs(rng, N=1, L=6, H=H, HV=HV)
    o_all, _, st_all = ogdn.gdn_slot_step(packed, H * K, H, K, HV, K, a, b, A_log, dt, state, [1], [6])
    st = state
    for t in range(6):
        o_t, _, st = ogdn.gdn_slot_step(packed[:, t:t + 1], H * K, H, K, HV, K, a[:, t:t + 1], b[:, t:t + 1],
                                        A_log, dt, st, [1], [1])
        np.testing.assert_allclose(o_t[0, 0], o_all[0, t], rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(st, st_all, rtol=1e-12, atol=1e-14)


def test_chunked_slot_step_equals_recurrent_slot_step():
    """gdn_slot_step_chunked (the chunk form per row, used for full-geometry ticks) gives gdn_slot_step's outputs
    and state to float64 rounding: rows longer than one chunk, a row shorter than its tick, an empty row, the
    GQA head map (HV > H), untouched other slots."""
    rng = np.random.default_rng(6)
    H, HV, K = 2, 4, 128
    packed, a, b, A_log, dt, state = _slot_inputs(rng, N=4, L=70, H=H, HV=HV)
    packed[..., :2 * H * K] *= 0.2          # raw q, k of conv-output scale
    slots, lens = np.array([3, 0, 5, 1]), np.array([70, 9, 0, 1])
    o_r, sq_r, st_r = ogdn.gdn_slot_step(packed, H * K, H, K, HV, K, a, b, A_log, dt, state, slots, lens)
    o_c, sq_c, st_c = ogdn.gdn_slot_step_chunked(packed, H * K, H, K, HV, K, a, b, A_log, dt, state, slots, lens)
    scale = np.abs(o_r).max()
    np.testing.assert_allclose(o_c, o_r, rtol=1e-10, atol=1e-12 * scale)
    np.testing.assert_allclose(st_c, st_r, rtol=1e-10, atol=1e-12 * np.abs(st_r).max())
    assert (o_c[1, 9:] == 0).all() and (o_c[2] == 0).all()
    for s in (2, 4):
        np.testing.assert_array_equal(st_c[s], state[s])
