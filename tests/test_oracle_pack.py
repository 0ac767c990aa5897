"""Pins the integer bookkeeping of the oracle (pack layout, ring columns, ring_pos) -- CPU only."""
import numpy as np
import pytest

from oracle import pack as opack
from oracle.bf16 import bf16


def test_padding_uses_scratch_slot():
    """The reference's own known-answer vector (tests/test_contract.py:14-18): one 3-token request, nb=2,
    lb=4, length=[7], max_slots=1."""
    out = np.empty(2 * 4 + 3 * 2, dtype=np.int64)
    lens = opack.pack_inputs([[4, 5, 6]], [0], 2, 4, np.array([7]), 1, out)
    assert lens.tolist() == [3]
    assert out[:8].tolist() == [4, 5, 6, 0, 0, 0, 0, 0]
    assert out[8:10].tolist() == [3, 0]
    assert out[10:12].tolist() == [0, 1]
    assert out[12:].tolist() == [7, 0]


def test_bucket():
    assert opack.bucket(1, (1, 2, 4)) == 1
    assert opack.bucket(3, (1, 2, 4)) == 4
    with pytest.raises(ValueError):
        opack.bucket(5, (1, 2, 4))


def test_ring_pos_matches_window_model():
    """Random tick sequences: after every tick, ring_pos holds exactly the last min(len, W) positions of
    each slot at column pos % W (a dictionary model of the window), and column W stays -1."""
    rng = np.random.default_rng(0)
    W, S = 16, 5
    ring_pos = np.full((S + 1, W + 1), -1, dtype=np.int64)
    length = np.zeros(S, dtype=np.int64)
    for _ in range(200):
        n = int(rng.integers(1, S + 1))
        slots = rng.permutation(S)[:n]
        lb = int(rng.choice([1, 2, 4, 8]))
        lens = rng.integers(1, lb + 1, size=n)
        nb = n + int(rng.integers(0, 2))
        slots_b = np.concatenate([slots, np.full(nb - n, S)])
        lens_b = np.concatenate([lens, np.zeros(nb - n, np.int64)])
        starts_b = np.concatenate([length[slots], np.zeros(nb - n, np.int64)])
        opack.ring_pos_update(ring_pos, slots_b, starts_b, lens_b, lb, W)
        length[slots] += lens
        for s in range(S):
            expect = np.full(W, -1, dtype=np.int64)
            for p in range(max(0, length[s] - W), length[s]):
                expect[p % W] = p
            np.testing.assert_array_equal(ring_pos[s, :W], expect)
        assert (ring_pos[:, W] == -1).all()


def test_bf16_matches_torch_cast():
    torch = pytest.importorskip("torch")
    x = np.concatenate([np.random.default_rng(1).standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-40], dtype=np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16(x), ref)


def test_bf16_perturbed_flips_exactly_the_values_near_a_tie():
    """Inside perturbed(k) the values within k fp32 ulps of a bf16 rounding tie take the other bf16 neighbour
    and every other value rounds as torch's cast does."""
    from oracle.bf16 import perturbed
    torch = pytest.importorskip("torch")
    base = np.random.default_rng(2).standard_normal(4000).astype(np.float32)
    hi = base.view(np.uint32) & np.uint32(0xFFFF0000)
    offsets = np.arange(-6, 7, dtype=np.int64)            # distance (fp32 ulps) to the tie at low half 0x8000
    u = (hi[:, None].astype(np.int64) + 0x8000 + offsets[None]).astype(np.uint32)
    x = u.view(np.float32).ravel()
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    with perturbed(3):
        got = bf16(x)
    flipped = (got != ref).reshape(u.shape)
    np.testing.assert_array_equal(flipped, np.broadcast_to(np.abs(offsets) <= 3, u.shape))
    near = np.broadcast_to(np.abs(offsets) <= 3, u.shape)
    lo = np.minimum(got, ref).reshape(u.shape)[near]
    hi_ = np.maximum(got, ref).reshape(u.shape)[near]
    xs = x.reshape(u.shape)[near]
    assert np.all((lo < xs) & (xs < hi_)) or np.all((lo > xs) & (xs > hi_))   # the two neighbours of each value
    np.testing.assert_array_equal(bf16(x), ref)              # outside the context: plain rounding again
