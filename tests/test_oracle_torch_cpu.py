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
