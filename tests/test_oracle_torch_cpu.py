"""Pins the PyTorch-CPU float32 restatement (oracle/torch_cpu.py, the benchmark's CPU baseline) against the float64
oracle with its bf16 rounding switched off -- CPU only.

Both restate the same step (slot_engine_v8.py:30-89) without bf16 rounding, so they agree to float32 round-off:
class probabilities, recurrent state, conv history and rings, and bit for bit on ring_pos and length. The ticks
cover padded rows, single- and multi-step rows in one tick, a row shorter than its tick, and rings that wrap.
"""
import numpy as np
import pytest

from oracle.backbone import StreamOracle
from oracle.bf16 import exact

torch = pytest.importorskip("torch")


def _cfg():
    from hs_guard.model import GuardConfig
    return GuardConfig(vocab_size=50, hidden_size=64, num_hidden_layers=4, intermediate_size=96,
                       linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=16,
                       linear_value_head_dim=16, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                       window_tokens=16, head_hidden=32)


def test_torch_cpu_step_matches_oracle():
    from hs_guard.model import GuardModel
    from oracle.torch_cpu import TorchStream
    cfg = _cfg()
    m = GuardModel.random(cfg, seed=2, device="cpu", std=0.2)
    w = {k: v.float().numpy() for k, v in m.weights.items()}
    ts = TorchStream(m.weights, cfg, 4)
    orc = StreamOracle(w, cfg, 4)
    rng = np.random.default_rng(0)
    ticks = [[(0, rng.integers(0, 50, 9).tolist()), (2, rng.integers(0, 50, 3).tolist())],
             [(1, [4]), (0, rng.integers(0, 50, 12).tolist()), (3, [7])],
             [(2, rng.integers(0, 50, 20).tolist())]] + \
            [[(s, rng.integers(0, 50, int(rng.choice([1, 1, 2, 5]))).tolist()) for s in (0, 1, 2, 3)] for _ in range(5)]
    for t, tick in enumerate(ticks):
        got = ts.tick(tick).numpy()
        with exact():
            ref, _ = orc.tick(tick)
        for r, (_, ids) in enumerate(tick):
            np.testing.assert_allclose(got[:, r, :len(ids)], ref[:, r, :len(ids)], rtol=0, atol=2e-5,
                                       err_msg=f"tick {t} row {r}")
    np.testing.assert_array_equal(ts.length, orc.length)
    np.testing.assert_array_equal(ts.ring_pos.numpy(), orc.ring_pos)
    assert (orc.ring_pos[:4, :16] >= 0).sum() > 40                       # rings filled and wrapped
    rel = np.linalg.norm(ts.rec.numpy() - orc.rec) / np.linalg.norm(orc.rec)
    assert rel < 1e-5, rel
    for name in ("conv", "ring_k", "ring_v"):
        a, b = getattr(ts, name).numpy()[:, :4], getattr(orc, name)[:, :4]
        if name != "conv":
            a, b = a[..., :16, :], b[..., :16, :]
        assert np.linalg.norm(a - b) <= 1e-5 * np.linalg.norm(b), name


def test_gdn_step_and_ring_decode_match_oracle():
    """The config-1 and config-2 legs of the CPU baseline: one GDN token per row and one decode step of the window
    attention with its ring write, against the oracle's functions (float64, rounding off)."""
    from oracle import gdn as ogdn
    from oracle import ring as oring
    from oracle.torch_cpu import gdn_step_torch, ring_decode_torch
    rng = np.random.default_rng(3)
    H, HV, K = 2, 4, 128
    N, S = 3, 5
    packed = rng.standard_normal((N, 2 * H * K + HV * K)).astype(np.float32)
    a, b = rng.standard_normal((N, HV)).astype(np.float32), rng.standard_normal((N, HV)).astype(np.float32)
    A_log, dt = (rng.standard_normal(HV) * 0.3).astype(np.float32), (rng.standard_normal(HV) * 0.3).astype(np.float32)
    state = (rng.standard_normal((S, HV, K, K)) * 0.05).astype(np.float32)
    slots = np.array([4, 0, 2])
    with exact():
        o_ref, _, st_ref = ogdn.gdn_slot_step(packed[:, None], H * K, H, K, HV, K, a[:, None], b[:, None], A_log, dt,
                                              state, slots, np.ones(N, np.int64))
    st = torch.from_numpy(state.copy())
    t = torch.from_numpy
    o = gdn_step_torch(t(packed), H * K, H, K, HV, K, t(a), t(b), t(A_log), t(dt), st, t(slots))
    np.testing.assert_allclose(o.numpy(), o_ref[:, 0], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(st.numpy(), st_ref, rtol=1e-4, atol=1e-6)
    Hkv, G, D, W = 2, 4, 32, 64
    q = rng.standard_normal((N, Hkv, G, D)).astype(np.float32)
    rk = rng.standard_normal((S, Hkv, W + 1, D)).astype(np.float32)
    rv = rng.standard_normal((S, Hkv, W + 1, D)).astype(np.float32)
    nk = rng.standard_normal((N, Hkv, D)).astype(np.float32)
    nv = rng.standard_normal((N, Hkv, D)).astype(np.float32)
    gate = rng.standard_normal((N, Hkv, G, D)).astype(np.float32)
    starts = np.array([700, 5, 64])
    rp = np.full((S, W + 1), -1, np.int64)
    for s, st_, f in zip(slots, starts, (64, 5, 30)):
        for p_ in range(st_ - f, st_):
            rp[s, p_ % W] = p_
    with exact():
        ref = oring.ring_attention_reference(q, rk, rv, nk[:, :, None], nv[:, :, None], rp, slots, starts,
                                             np.ones(N, np.int64), D ** -0.5, W)
    ref = ref * (1 / (1 + np.exp(-gate.astype(np.float64))))
    rkt, rvt = t(rk.copy()), t(rv.copy())
    out = ring_decode_torch(t(q), rkt, rvt, t(nk), t(nv), t(gate), t(rp), t(slots), t(starts), D ** -0.5, W)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-4, atol=1e-5)
    for n, s in enumerate(slots):
        np.testing.assert_array_equal(rkt[s, :, starts[n] % W].numpy(), nk[n])
        np.testing.assert_array_equal(rvt[s, :, starts[n] % W].numpy(), nv[n])
