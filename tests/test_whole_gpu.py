"""GPU parity of the complete-message scorer (hs_guard.engine.whole: chunked GDN prefill, gated RMSNorm and the
segment-ring window attention) against the CPU oracle and against the streaming engine.

The oracle is the streaming restatement (oracle.backbone.StreamOracle) fed the same sequence in ticks: the
recurrence and the window mask are the same functions whether a sequence arrives at once or in ticks (the
oracle's own tick-split invariance is pinned in tests/test_oracle_backbone.py). GEMMs are independent
(hipBLASLt at the whole sequence's M against numpy fp32), so the bound is the engine test's 1e-2 on per-token
class probabilities (see tests/test_engine_gpu.py for why deeper random nets need it); geometry: hidden 1024,
GDN heads 128 wide, attention head_dim 256, a 32-token window so that sequences of a few hundred tokens cross
many windows and 64-token segments.
"""
import numpy as np
import pytest
import torch
from parity_helpers import oracle_whole, whole_matched_gemm

pytestmark = pytest.mark.gpu

PROB_TOL = 2e-3
PROB_TOL_INDEPENDENT = 1e-2


@pytest.fixture(scope="module")
def setup():
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    model_cpu = GuardModel.random(cfg, seed=3, device="cpu")
    weights = {k: v.float().numpy() for k, v in model_cpu.weights.items()}
    return cfg, model_cpu.to("cuda:0"), weights


@pytest.mark.parametrize("T", [1, 63, 200])
def test_whole_sequence_matches_oracle(setup, T):
    from hs_guard.engine.whole import WholeSequenceScorer
    cfg, model, weights = setup
    print(f"[whole] T={T} vs oracle", flush=True)
    ids = np.random.default_rng(T).integers(0, cfg.vocab_size, T).tolist()
    got = WholeSequenceScorer(model).forward(ids).cpu().numpy()
    ref = oracle_whole(weights, cfg, ids)
    for i, role in enumerate(("user", "assistant")):
        diff = np.abs(got[i] - ref[i]).max()
        print(f"[whole] T={T} {role}: max prob diff {diff:.2e}", flush=True)
        assert diff <= PROB_TOL_INDEPENDENT, f"{role}: {diff:.2e}"


def test_whole_sequence_matched_gemms():
    """On the 2-layer [GDN, attention] net with the oracle's projections computed by the scorer's own product
    (tests/parity_helpers.py), every other kernel of the complete-message path -- conv, chunked GDN prefill,
    gated RMSNorm, window attention over gathered segment rings, the fp32 risk heads -- is held to the north
    star's 2e-3 on 1 - p(safe) against the float64 oracle read out in fp32 (runtime.py:70-73,141)."""
    from hs_guard.engine.whole import WholeSequenceScorer
    from hs_guard.model import GuardConfig, GuardModel
    print("[whole] matched GEMMs, 2 layers", flush=True)
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=2,
                      layer_types=["linear_attention", "full_attention"], intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    model_cpu = GuardModel.random(cfg, seed=1, device="cpu")
    weights = {k: v.float().numpy() for k, v in model_cpu.weights.items()}
    model = model_cpu.to("cuda:0")
    for T in (50, 200):
        ids = np.random.default_rng(T + 1).integers(0, cfg.vocab_size, T).tolist()
        got = WholeSequenceScorer(model).forward(ids).cpu().numpy()
        ref = oracle_whole(weights, cfg, ids, gemm=whole_matched_gemm(cfg))
        diff = float(np.abs(got[:, :, 0] - ref[:, :, 0]).max())
        print(f"[whole] T={T}: max |d cut| {diff:.2e}", flush=True)
        assert diff <= PROB_TOL, f"T={T}: {diff:.2e}"


def test_attention_segment_batches_agree(setup, monkeypatch):
    """Splitting the attention's segments over several launches (as sequences longer than 8192 tokens do) gives
    the same result as one launch."""
    import hs_guard.engine.whole as whole
    cfg, model, _ = setup
    print("[whole] attention segment batches", flush=True)
    ids = np.random.default_rng(9).integers(0, cfg.vocab_size, 300).tolist()
    one = whole.WholeSequenceScorer(model).forward(ids)
    monkeypatch.setattr(whole, "MAX_ATT_SEGMENTS", 2)
    split = whole.WholeSequenceScorer(model).forward(ids)
    torch.testing.assert_close(split, one, rtol=0, atol=0)


def test_stream_vs_whole_selfcheck(setup):
    """The readiness check of examples/demo/server.py:500-524: the sequence streamed 3 tokens per tick equals one
    whole forward (the reference fails it above 0.05)."""
    from hs_guard.runtime import selfcheck
    cfg, model, _ = setup
    print("[whole] stream vs whole", flush=True)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, 130).tolist()
    res = selfcheck(model, ids, piece=3)
    print(f"[whole] selfcheck {res}", flush=True)
    assert res["tokens"] == 130 and res["stream_positions"] == 130
    assert res["max_prob_diff_stream_vs_whole"] <= PROB_TOL_INDEPENDENT


def test_score_ids_record(setup):
    """score_ids readout (src/hs_guard/runtime.py:136-145): user -> last cut score, assistant -> largest, over
    the given positions; flagged iff above the role's threshold."""
    from hs_guard.engine.whole import WholeSequenceScorer
    from hs_guard.runtime import random_metadata, score_ids
    cfg, model, _ = setup
    print("[whole] score_ids record", flush=True)
    meta = random_metadata()
    ids = np.random.default_rng(2).integers(0, cfg.vocab_size, 90).tolist()
    positions = list(range(40, 90))
    probs = WholeSequenceScorer(model).forward(ids).cpu().numpy()
    cut_user = 1 - probs[0, positions, 0]
    cut_asst = 1 - probs[1, positions, 0]
    rec_u = score_ids(model, meta, ids, positions, "user")
    rec_a = score_ids(model, meta, ids, positions, "assistant")
    assert rec_u["role"] == "user" and rec_a["role"] == "assistant" and rec_u["head"] == "redline"
    assert abs(rec_u["score"] - cut_user[-1]) < 1e-6
    assert abs(rec_a["score"] - cut_asst.max()) < 1e-6
    assert rec_u["threshold"] == meta["thresholds"]["user"]
    assert rec_u["flagged"] == (rec_u["score"] > rec_u["threshold"])
    with pytest.raises(ValueError):
        score_ids(model, meta, [], None, "user")
    with pytest.raises(ValueError):
        score_ids(model, meta, [cfg.vocab_size], None, "user")


def test_selfcheck_full_geometry():
    """The readiness self-check on the benchmark geometry (24 layers, 16q/4kv, window 512, random-init): streamed
    in 3-token ticks vs one whole forward, against the reference's bound of 0.05 (examples/demo/server.py:483)."""
    from hs_guard.model import GuardConfig, GuardModel
    from hs_guard.runtime import selfcheck
    print("[whole] full-geometry selfcheck", flush=True)
    cfg = GuardConfig.baseline()
    model = GuardModel.random(cfg, seed=0, device=torch.device("cuda:0"), gen_device=torch.device("cuda:0"))
    ids = np.random.default_rng(7).integers(0, cfg.vocab_size, 160).tolist()
    res = selfcheck(model, ids, piece=3)
    print(f"[whole] full-geometry selfcheck {res}", flush=True)
    assert res["stream_positions"] == 160
    assert res["max_prob_diff_stream_vs_whole"] <= 0.05


def test_local_bundle_end_to_end(tmp_path):
    """load_model on a synthetic local bundle (tests/conftest.py:write_bundle), then score_messages through its
    tokenizer and StreamingGuard on the same ids: the loaded model scores exactly like the same weights built
    directly, and streaming agrees with the whole forward."""
    from conftest import write_bundle
    from hs_guard.model import GuardConfig, GuardModel
    from hs_guard.runtime import StreamingGuard, encode_messages, load_model, score_ids, score_messages
    print("[whole] local bundle end to end", flush=True)
    cfg = GuardConfig(vocab_size=64, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    root, state = write_bundle(tmp_path / "b", cfg)
    model, tok, meta = load_model(str(root))
    msgs = [{"role": "user", "content": " ".join(f"w{i % 60}" for i in range(40))},
            {"role": "assistant", "content": " ".join(f"w{(7 * i) % 60}" for i in range(50))}]
    rec = score_messages(model, tok, meta, msgs)
    ids, positions, role = encode_messages(tok, msgs)
    assert role == "assistant" and len(ids) == 92 and positions == list(range(42, 92))   # the 50 content tokens
    direct = GuardModel(cfg, {k: v.to("cuda:0") for k, v in state.items() if k in cfg.parameter_shapes()})
    assert rec == score_ids(direct, meta, ids, positions, role)
    guard = StreamingGuard(model, meta, max_slots=2)
    cuts = []
    for a in range(0, len(ids), 7):
        cuts += guard.step([(1, ids[a:a + 7])], role="assistant")[0]["cut_scores"]
    streamed = max(cuts[p] for p in positions)
    assert abs(streamed - rec["score"]) <= PROB_TOL_INDEPENDENT
