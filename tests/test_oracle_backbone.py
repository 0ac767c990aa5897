"""Pins the composition of the whole-step oracle -- CPU only.

The streamed oracle (ticks of several sizes over per-slot pools) must reproduce transformers'
Qwen3_5TextModel forward over the whole sequence (the complete-message path, docs/ENGINE.md:13) when the
sequence fits the window. With the oracle's bf16 rounding switched off (``oracle.bf16.exact``) and
transformers in float64 the two agree to the pools' fp32 storage round-off (~1e-6), which pins the composition (layer order, norm
placement and offsets, head maps, RoPE, gates, conv history, recurrent state, ring). With rounding on they
agree at bf16-noise level. Planted mistakes (a dropped attention gate, a wrong RMSNorm offset) move the
result by orders of magnitude more.
"""
import numpy as np
import pytest

from oracle.backbone import StreamOracle
from oracle.bf16 import exact

torch = pytest.importorskip("torch")


def _tiny_cfg():
    from hs_guard.model import GuardConfig
    return GuardConfig(vocab_size=50, hidden_size=64, num_hidden_layers=4, intermediate_size=96,
                       linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=16,
                       linear_value_head_dim=16, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                       window_tokens=16, head_hidden=32)


def _weights(cfg, seed=0):
    from hs_guard.model import GuardModel
    m = GuardModel.random(cfg, seed=seed, device="cpu", std=0.2)
    return {k: v.float().numpy() for k, v in m.weights.items()}


def _hf_hidden(cfg, w, ids):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextModel
    hc = Qwen3_5TextConfig(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                           num_hidden_layers=cfg.num_hidden_layers, intermediate_size=cfg.intermediate_size,
                           linear_num_key_heads=cfg.linear_num_key_heads,
                           linear_num_value_heads=cfg.linear_num_value_heads,
                           linear_key_head_dim=cfg.linear_key_head_dim, linear_value_head_dim=cfg.linear_value_head_dim,
                           num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                           head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps,
                           rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                                            "partial_rotary_factor": cfg.partial_rotary_factor,
                                            "mrope_section": [1, 1, 2]})
    hc._attn_implementation = "eager"
    model = Qwen3_5TextModel(hc).double().eval()
    sd = {k[len("backbone."):]: torch.from_numpy(v).double() for k, v in w.items() if k.startswith("backbone.")}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    with torch.no_grad():
        out = model(input_ids=torch.tensor([ids]), use_cache=False).last_hidden_state[0]
    return out.numpy()


def _stream_hidden(oracle, slot, ids, ticks):
    hid = []
    at = 0
    for size in ticks:
        _, normed = oracle.tick([(slot, ids[at:at + size])])
        hid.append(normed[0, :size])
        at += size
    return np.concatenate(hid)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_streamed_oracle_matches_transformers_forward():
    cfg = _tiny_cfg()
    w = _weights(cfg)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, cfg.vocab_size, 15).tolist()          # < window: windowed == causal attention
    ref = _hf_hidden(cfg, w, ids)
    with exact():
        oracle = StreamOracle(w, cfg, max_slots=3)
        got = _stream_hidden(oracle, 1, ids, [5, 1, 7, 2])
        assert _rel(got, ref) < 1e-5, _rel(got, ref)   # pools store fp32: ~1e-6 round-off
        # a second slot streamed with other tick sizes agrees too (slot 1's state does not leak into it)
        got2 = _stream_hidden(oracle, 2, ids, [1] * 15)
        assert _rel(got2, ref) < 1e-5
    rounded = _stream_hidden(StreamOracle(w, cfg, max_slots=3), 1, ids, [5, 1, 7, 2])
    assert _rel(rounded, ref) < 0.1


def test_planted_mistakes_are_detected():
    cfg = _tiny_cfg()
    w = _weights(cfg)
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, 12).tolist()
    ref = _hf_hidden(cfg, w, ids)
    import oracle.ring as oring
    orig = oring.ring_attention_v8

    def no_gate(q, rk, rv, nk, value, gate, *a, **k):
        return orig(q, rk, rv, nk, value, np.full_like(gate, 30.0), *a, **k)   # sigmoid ~ 1: gate dropped
    oring.ring_attention_v8 = no_gate
    try:
        with exact():
            bad = _stream_hidden(StreamOracle(w, cfg, 2), 0, ids, [4, 8])
    finally:
        oring.ring_attention_v8 = orig
    assert _rel(bad, ref) > 1e-2
    w2 = dict(w)
    w2["backbone.layers.1.post_attention_layernorm.weight"] = w["backbone.layers.1.post_attention_layernorm.weight"] - 1.0
    with exact():
        bad = _stream_hidden(StreamOracle(w2, cfg, 2), 0, ids, [4, 8])
    assert _rel(bad, ref) > 1e-2


def _floor(cfg, seed, slots, ctx, decode_ticks, ulps=1, std=0.02):
    """Largest per-token |d(1 - p(safe))| between the oracle and the oracle with fp32-level rounding freedom
    (oracle.bf16.perturbed(4): the roughly 1.4e-4 of bf16 roundings that lie within 4 fp32 ulps of a tie go the
    other way) everywhere except in the GEMM outputs, which stay one fixed function of their inputs as in the
    matched-GEMM engine tests; over a tick of ``ctx`` tokens per slot and ``decode_ticks`` single-token ticks."""
    from hs_guard.model import GuardModel
    from oracle.bf16 import perturbed
    from oracle.glue import linear_bf16

    def gemm(x, wt, bias, lens):
        with perturbed(0):
            return linear_bf16(x, wt, bias)
    m = GuardModel.random(cfg, seed=seed, device="cpu", std=std)
    w = {k: v.float().numpy() for k, v in m.weights.items()}
    rng = np.random.default_rng(seed)
    ticks = [[(s, rng.integers(0, cfg.vocab_size, ctx).tolist()) for s in range(slots)]]
    ticks += [[(s, [int(rng.integers(0, cfg.vocab_size))]) for s in range(slots)] for _ in range(decode_ticks)]
    a, b = StreamOracle(w, cfg, slots, gdn="chunk"), StreamOracle(w, cfg, slots, gdn="chunk")
    worst = 0.0
    for tick in ticks:
        pa, _ = a.tick(tick, gemm=gemm)
        with perturbed(ulps):
            pb, _ = b.tick(tick, gemm=gemm)
        worst = max(worst, float(np.abs(pa[..., 0] - pb[..., 0]).max()))
    return worst


def test_noise_floor_at_benchmark_depth():
    """At the 24-layer benchmark geometry (GuardConfig.baseline(), random-init N(0, 0.02) weights) the oracle's
    own fp32-level noise floor exceeds the 2e-3 end-to-end bar: letting the values within one fp32 ulp of a bf16
    rounding tie round the other way -- a freedom any fp32 evaluation has, the reference's kernels included --
    moves cut scores by several times 2e-3. A full-geometry comparison is therefore held to this floor,
    measured on identical inputs (tests/test_full_geometry_gpu.py); the 2e-3 bar is kept for the 2-layer
    matched-GEMM tests (tests/test_engine_gpu.py)."""
    from hs_guard.model import GuardConfig
    f24 = _floor(GuardConfig.baseline(), 0, 2, 64, 1)
    print(f"noise floor at 24 layers: {f24:.2e}")
    assert f24 > 2e-3


def test_noise_floor_scales_with_weights():
    """The floor is a property of the random-init net, not of any implementation: each bf16 rounding turns a small
    difference of its inputs into sparse one-ulp flips whose norm is about sqrt(difference x ulp), so a few
    rounding stages carry any fp32-level difference up to about one bf16 ulp of the hidden state (~1%), and the
    heads turn that into a cut-score change proportional to their logits' scale, which grows with the weights'.
    At N(0, 0.0025) the 24-layer floor is below 1e-3, so the 2e-3 bar can be held at the benchmark depth
    (tests/test_full_geometry_gpu.py::test_benchmark_depth_at_north_star_bar); at N(0, 0.005) the 2-layer floor is
    below 1e-3 (the 2e-3 tests of tests/test_engine_gpu.py and tests/test_contract_gpu.py)."""
    from hs_guard.model import GuardConfig
    two = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=2,
                      layer_types=["linear_attention", "full_attention"], intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    f2_small, f2 = _floor(two, 0, 4, 32, 2, std=0.005), _floor(two, 0, 4, 32, 2)
    f24_small = _floor(GuardConfig.baseline(), 0, 2, 64, 1, std=0.0025)
    print(f"noise floor: 2 layers {f2_small:.2e} (std 0.005) / {f2:.2e} (std 0.02); 24 layers {f24_small:.2e} "
          f"(std 0.0025)")
    assert f2_small < 1e-3 and f24_small < 1e-3
    assert f2 > 2 * f2_small
