"""Parity of the streaming step at the benchmark geometry (config 3) and the released v10 geometry against the CPU
oracle.

Geometry: GuardConfig.baseline() -- 24 layers [GDN, GDN, GDN, attention] x 6, hidden 1024, GDN 16 heads x 128,
attention 16 q / 4 kv heads of 256 with a 512-token window, MLP 3584, vocab 151,936, random-init bf16 weights
N(0, 0.02), seed 0. Eight slots receive contexts of 520-597 tokens in 64-token ticks (the reference's tick cut),
so every slot's 512-column ring wraps, then four single-token ticks for every slot and one mixed tick of 1-64
tokens per slot. The oracle's GEMMs are the engine's own products (tests/parity_helpers.py), so everything else
-- conv, recurrence, norms, RoPE, window attention with its ring, heads, ring and length bookkeeping -- is the
float64 CPU restatement; its GDN layers use the chunk form for multi-token ticks (the same recurrence,
tests/test_oracle_gdn.py).

Bar. At this depth a random-init net amplifies last-bit differences: the oracle run a second time with the
values within one fp32 ulp of a bf16 rounding tie rounded the other way (oracle.bf16.perturbed(1), a freedom
every fp32 evaluation has, the reference's Triton kernels included) moves per-token cut scores by up to ~1e-2
(tests/test_oracle_backbone.py::test_noise_floor_at_benchmark_depth), five times the north star's 2e-3. The
engine is held to that floor measured here on the same inputs: the median, 99th percentile and maximum of its
per-token |d(1 - p(safe))| against the oracle must each be at most 1.5 times the perturbed oracle's. Integer
bookkeeping (ring_pos, length) is bit-exact.
"""
import numpy as np
import pytest
from parity_helpers import matched_gemm

pytestmark = pytest.mark.gpu

FLOOR_FACTOR = 1.5


@pytest.fixture(scope="module", params=["baseline", "v10"])
def full(request):
    """The benchmark geometry at 8 slots, and the released v10 geometry (8 q / 2 kv heads, vocab 248,320,
    docs/evaluation.json:623) at 4 slots."""
    from hs_guard.model import GuardConfig, GuardModel
    print(f"[full] random-init {request.param} model", flush=True)
    cfg = getattr(GuardConfig, request.param)()
    model_cpu = GuardModel.random(cfg, seed=0, device="cpu")
    weights = {k: v.float().numpy() for k, v in model_cpu.weights.items()}
    return cfg, model_cpu.to("cuda:0"), weights, (8 if request.param == "baseline" else 4)


def _ticks(rng, vocab, slots=8):
    ctx = [rng.integers(0, vocab, 520 + 11 * s).tolist() for s in range(slots)]
    ticks = []
    for t0 in range(0, max(len(c) for c in ctx), 64):
        ticks.append([(s, c[t0:t0 + 64]) for s, c in enumerate(ctx) if t0 < len(c)])
    for _ in range(4):
        ticks.append([(s, [int(rng.integers(0, vocab))]) for s in range(slots)])
    ticks.append([(s, rng.integers(0, vocab, n).tolist()) for s, n in enumerate((1, 2, 5, 17, 64, 1, 3, 9)[:slots])])
    return ticks


def _cut_diffs(got, ref):
    """Per-token |d(1 - p(safe))| over both roles and all requests of a tick, as one flat array."""
    return np.concatenate([np.abs(np.asarray(g)[:, 0] - np.asarray(e)[:, 0]) for role in ("user", "assistant")
                           for g, e in zip(got[role], ref[role])])


def test_baseline_geometry_matches_oracle(full):
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from oracle.backbone import StreamOracle
    from oracle.bf16 import perturbed
    cfg, model, weights, slots = full
    eng = SlotStreamEngine(model, slots, use_graphs=False)
    orc = StreamOracle(weights, cfg, slots, gdn="chunk")
    twin = StreamOracle(weights, cfg, slots, gdn="chunk")
    gemm = matched_gemm(eng)
    hip, floor = [], []
    for t, tick in enumerate(_ticks(np.random.default_rng(0), cfg.vocab_size, slots)):
        got = eng.step(tick)
        ref = orc.step(tick, gemm=gemm)
        with perturbed(1):
            alt = twin.step(tick, gemm=gemm)
        hip.append(_cut_diffs({r: [x.numpy() for x in v] for r, v in got.items()}, ref))
        floor.append(_cut_diffs(alt, ref))
        print(f"[full] tick {t}: {len(tick)} rows, {sum(len(i) for _, i in tick)} tokens, max |d cut| engine "
              f"{hip[-1].max():.2e}, perturbed oracle {floor[-1].max():.2e}", flush=True)
    W = cfg.window_tokens
    np.testing.assert_array_equal(eng.length, orc.length)
    np.testing.assert_array_equal(eng.ring_pos.cpu().numpy(), orc.ring_pos)
    assert (orc.ring_pos[:slots, :W] >= 0).all() and (orc.length > W).all()     # every ring has wrapped
    rec = eng.rec.double().cpu().numpy()
    rel = [np.linalg.norm(rec[:, s] - orc.rec[:, s]) / np.linalg.norm(orc.rec[:, s]) for s in range(slots)]
    rel_twin = [np.linalg.norm(twin.rec[:, s] - orc.rec[:, s]) / np.linalg.norm(orc.rec[:, s])
                for s in range(slots)]
    print(f"[full] state rel err: engine {max(rel):.1e}, perturbed oracle {max(rel_twin):.1e}", flush=True)
    hip, floor = np.concatenate(hip), np.concatenate(floor)
    stats = {name: (fn(hip), fn(floor)) for name, fn in (("p50", np.median), ("p99", lambda x: np.quantile(x, 0.99)),
                                                          ("max", np.max))}
    print("[full] |d cut| engine vs perturbed oracle: " +
          ", ".join(f"{k} {a:.2e} / {b:.2e}" for k, (a, b) in stats.items()), flush=True)
    for k, (a, b) in stats.items():
        assert a <= FLOOR_FACTOR * b, f"{k}: engine {a:.2e} > {FLOOR_FACTOR} x floor {b:.2e}"
    assert max(rel) <= FLOOR_FACTOR * max(rel_twin)


@pytest.mark.parametrize("geometry", ["baseline", "v10"])
def test_benchmark_depth_at_north_star_bar(geometry):
    """The 2e-3 bar itself at the benchmark depth: GuardConfig.baseline() (24 layers; and the released v10
    geometry, 8 q / 2 kv heads, vocab 248,320) with random-init weights
    N(0, 0.0025), where the oracle's fp32-level noise floor is below 1e-3 (measured here on the same inputs, and on
    the CPU by tests/test_oracle_backbone.py::test_noise_floor_scales_with_weights). Four slots receive contexts of
    520-553 tokens in 64-token ticks (every ring wraps), then four single-token ticks and a mixed tick; every
    per-token |d(1 - p(safe))| against the oracle with matched GEMMs must be within 2e-3. The recurrent state, whose
    inputs carry the ~1% bf16 noise of the hidden state at this depth (the perturbed oracle's own state moves by
    ~1e-2), is held to 1.5x the perturbed oracle's deviation."""
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    from oracle.backbone import StreamOracle
    from oracle.bf16 import perturbed
    print(f"[full] benchmark depth, {geometry} geometry, N(0, 0.0025), 2e-3 bar", flush=True)
    cfg = getattr(GuardConfig, geometry)()
    model_cpu = GuardModel.random(cfg, seed=0, device="cpu", std=0.0025)
    weights = {k: v.float().numpy() for k, v in model_cpu.weights.items()}
    slots = 4
    eng = SlotStreamEngine(model_cpu.to("cuda:0"), slots, use_graphs=False)
    del model_cpu
    orc = StreamOracle(weights, cfg, slots, gdn="chunk")
    twin = StreamOracle(weights, cfg, slots, gdn="chunk")
    gemm = matched_gemm(eng)
    worst = floor = 0.0
    cuts = []
    for t, tick in enumerate(_ticks(np.random.default_rng(1), cfg.vocab_size, slots)):
        got = eng.step(tick)
        cuts.extend(x.numpy()[:, 0] for v in got.values() for x in v)
        ref = orc.step(tick, gemm=gemm)
        with perturbed(1):
            alt = twin.step(tick, gemm=gemm)
        d = _cut_diffs({r: [x.numpy() for x in v] for r, v in got.items()}, ref).max()
        f = _cut_diffs(alt, ref).max()
        worst, floor = max(worst, d), max(floor, f)
        print(f"[full] tick {t}: {len(tick)} rows, {sum(len(i) for _, i in tick)} tokens, max |d cut| engine "
              f"{d:.2e}, perturbed oracle {f:.2e}", flush=True)
        assert d <= 2e-3, f"tick {t}: cut-score diff {d:.2e}"
    W = cfg.window_tokens
    np.testing.assert_array_equal(eng.length, orc.length)
    np.testing.assert_array_equal(eng.ring_pos.cpu().numpy(), orc.ring_pos)
    assert (orc.ring_pos[:slots, :W] >= 0).all() and (orc.length > W).all()
    assert floor < 1e-3, f"noise floor {floor:.2e}: the bar would not be meaningful on these inputs"
    # and the bar discriminates: at this weight scale the cut scores still move with the input far beyond 2e-3
    cuts = np.concatenate(cuts)
    spread = float(np.percentile(cuts, 95) - np.percentile(cuts, 5))
    print(f"[full] cut scores: 5-95 percentile spread {spread:.2e} over {cuts.size} tokens", flush=True)
    assert spread > 10 * 2e-3
    rec = eng.rec.double().cpu().numpy()
    rel = max(np.linalg.norm(rec[:, s] - orc.rec[:, s]) / np.linalg.norm(orc.rec[:, s]) for s in range(slots))
    rel_twin = max(np.linalg.norm(twin.rec[:, s] - orc.rec[:, s]) / np.linalg.norm(orc.rec[:, s])
                   for s in range(slots))
    print(f"[full] worst |d cut| {worst:.2e} (floor {floor:.2e}); state rel err {rel:.1e} (perturbed oracle "
          f"{rel_twin:.1e})", flush=True)
    assert rel <= FLOOR_FACTOR * rel_twin
