"""Pins the ring-attention oracle -- CPU only.

Anchors: torch scaled_dot_product_attention with an explicit boolean mask built from a brute-force
enumeration of the window predicate, closed forms (only the new key visible; all keys equal).
"""
import numpy as np
import pytest

from oracle import ring as oring
from oracle.bf16 import bf16, sigmoid

torch = pytest.importorskip("torch")


def _setup(rng, N=3, Hkv=2, G=2, Lb=3, D=8, W=16, S=5):
    q = rng.standard_normal((N, Hkv, G * Lb, D))
    ring_k = rng.standard_normal((S, Hkv, W + 1, D))
    ring_v = rng.standard_normal((S, Hkv, W + 1, D))
    new_k = rng.standard_normal((N, Hkv, Lb, D))
    new_v = rng.standard_normal((N, Hkv, Lb, D))
    slots = rng.permutation(S - 1)[:N]
    starts = rng.integers(0, 40, N)
    lens = rng.integers(0, Lb + 1, N)
    ring_pos = np.full((S, W + 1), -1, dtype=np.int64)
    for s, st in zip(slots, starts):
        fill = int(rng.integers(0, W + 1))
        for p in range(max(0, st - fill), st):
            ring_pos[s, p % W] = p
    return q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, W


def test_matches_sdpa_with_bruteforce_mask():
    rng = np.random.default_rng(0)
    for trial in range(5):
        q, rk, rv, nk, nv, rp, slots, starts, lens, W = _setup(rng)
        N, Hkv, M, D = q.shape
        Lb = nk.shape[2]
        out = oring.ring_attention_reference(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.3, W)
        for n in range(N):
            keys = np.concatenate([rk[slots[n], :, :W], nk[n]], 1)
            vals = np.concatenate([rv[slots[n], :, :W], nv[n]], 1)
            kpos = [rp[slots[n], c] for c in range(W)] + [starts[n] + j if j < lens[n] else -1 for j in range(Lb)]
            for r in range(M):
                l = r % Lb
                qpos = starts[n] + l
                mask = np.array([l < lens[n] and 0 <= kp <= qpos and kp > qpos - W for kp in kpos])
                if not mask.any():
                    assert (out[n, :, r] == 0).all()
                    continue
                ref = torch.nn.functional.scaled_dot_product_attention(
                    torch.from_numpy(q[n, :, r:r + 1]), torch.from_numpy(keys), torch.from_numpy(vals),
                    attn_mask=torch.from_numpy(mask)[None, None], scale=0.3)
                np.testing.assert_allclose(out[n, :, r], ref[:, 0].numpy(), rtol=1e-10, atol=1e-12)


def test_only_new_key_visible_gives_gated_value():
    """Empty ring, one new token: out = bf16(v_new) * bf16(sigmoid(gate)) (fill 0 + self only)."""
    rng = np.random.default_rng(1)
    N, Hkv, G, D, W = 2, 2, 2, 8, 16
    q = rng.standard_normal((N, Hkv, G, D))
    rk = rng.standard_normal((N + 1, Hkv, W + 1, D))
    rv = rng.standard_normal((N + 1, Hkv, W + 1, D))
    nk = rng.standard_normal((N, Hkv, 1, D))
    value = bf16(rng.standard_normal((N, 1, Hkv * D)))
    gate = rng.standard_normal((N, 1, Hkv * G * 2 * D))
    rp = np.full((N + 1, W + 1), -1, dtype=np.int64)
    out, _, rk2, _ = oring.ring_attention_v8(q, rk, rv, nk, value, gate, rp, np.arange(N), np.array([5, 0]),
                                             np.ones(N, np.int64), 1.0, W, True)
    v = value.reshape(N, 1, Hkv, 1, D).repeat(G, 3).reshape(N, 1, Hkv * G * D)
    sig = bf16(sigmoid(gate.reshape(N, 1, Hkv * G, 2 * D)[..., D:])).reshape(N, 1, -1)
    np.testing.assert_allclose(out, bf16(v * sig), rtol=0, atol=0)
    np.testing.assert_array_equal(rk2[0, :, 5], nk[0, :, 0])   # ring write at start % W
    np.testing.assert_array_equal(rk2[1, :, 0], nk[1, :, 0])


def test_equal_keys_give_mean_of_visible_values():
    rng = np.random.default_rng(2)
    q, rk, rv, nk, nv, rp, slots, starts, lens, W = _setup(rng, N=2, Lb=1)
    rk[:] = 0.7
    nk[:] = 0.7
    lens[:] = 1
    out = oring.ring_attention_reference(q, rk, rv, nk, nv, rp, slots, starts, lens, 1.0, W)
    for n in range(2):
        vis = [c for c in range(W) if 0 <= rp[slots[n], c] <= starts[n] and rp[slots[n], c] > starts[n] - W]
        vals = np.concatenate([rv[slots[n], :, vis], nv[n, :, :1].transpose(1, 0, 2)], 0)   # [k, Hkv, D]
        np.testing.assert_allclose(out[n, :, 0], vals.mean(0), rtol=1e-12)


def test_blockwise_equals_exact_without_rounding_and_is_within_bf16_p_bound():
    from oracle.bf16 import exact
    rng = np.random.default_rng(3)
    for lb in (1, 3, 40):
        q, rk, rv, nk, nv, rp, slots, starts, lens, W = _setup(rng, N=3, Lb=lb, W=64, D=16)
        ref = oring.ring_attention_reference(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.4, W)
        with exact():
            blk = oring.attend_blockwise(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.4, W)
        np.testing.assert_allclose(blk, ref, rtol=1e-10, atol=1e-12)
        rounded = oring.attend_blockwise(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.4, W)
        # bf16 p: each weight moves by at most 2**-8 relative, so the output by at most 2**-8 * sum|p v| / l
        bound = 2.0 ** -8 * np.abs(nv).max() * 2 + 1e-12
        assert np.abs(rounded - ref).max() <= bound


def test_closed_form_equals_online_loop():
    """attend_blockwise (the rescale chain multiplied out) equals the reference kernels' block-by-block loop with
    bf16 probabilities, to float64 rounding: decode and multi-step ticks, partly filled and empty rings."""
    rng = np.random.default_rng(8)
    for lb in (1, 3, 40):
        q, rk, rv, nk, nv, rp, slots, starts, lens, W = _setup(rng, N=4, Lb=lb, W=64, D=16)
        a = oring.attend_blockwise(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.4, W)
        b = oring.attend_blockwise_online(q, rk, rv, nk, nv, rp, slots, starts, lens, 0.4, W)
        np.testing.assert_allclose(a, b, rtol=1e-11, atol=1e-13)
