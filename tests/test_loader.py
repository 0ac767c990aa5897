"""Local bundle loading (src/hs_guard/runtime.py:19-41,92-125) on a synthetic bundle -- CPU only.

The bundle has the released layout (tests/conftest.py:write_bundle). Pinned: manifest checks (format, labels,
required assets, path safety, SHA-256), the config.json geometry mapping, strict checkpoint names and shapes,
the general-head swap, and that the loaded tensors are the written ones bit for bit.
"""
import json
import os

import pytest
import torch

from conftest import write_bundle


def _cfg():
    from hs_guard.model import GuardConfig
    return GuardConfig(vocab_size=64, hidden_size=1024, num_hidden_layers=4, intermediate_size=256,
                       linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                       num_key_value_heads=2, window_tokens=32, rope_theta=12345.0)


@pytest.fixture(scope="module")
def bundle(tmp_path_factory):
    return write_bundle(tmp_path_factory.mktemp("bundle") / "b", _cfg())


def test_bundle_loads_bit_exact(bundle):
    from hs_guard.runtime import load_bundle
    root, state = bundle
    model, tok, meta = load_bundle(root, device="cpu")
    cfg = model.config
    assert (cfg.vocab_size, cfg.num_hidden_layers, cfg.num_attention_heads, cfg.window_tokens) == (64, 4, 8, 32)
    assert cfg.layer_types == _cfg().layer_types and cfg.rope_theta == 12345.0 and cfg.rotary_dim == 64
    assert set(model.weights) == set(cfg.parameter_shapes())
    for name, t in model.weights.items():
        want = torch.float32 if name.startswith("heads.") else torch.bfloat16
        assert t.dtype == want and torch.equal(t, state[name]), name
    assert meta["head"] == "redline" and meta["thresholds"] == {"user": 0.07, "assistant": 0.11}
    assert meta["window_tokens"] == 32
    enc = tok.encode("USER:\nw3 w5", add_special_tokens=False)
    assert enc.ids == [1, 7, 9] and enc.offsets[1] == (6, 8)


def test_general_head_swaps_projection_and_risk(bundle):
    from hs_guard.runtime import load_bundle
    root, state = bundle
    model, _, meta = load_bundle(root, head="general", device="cpu")
    assert meta["thresholds"] == {"user": 0.5, "assistant": 0.5}
    for role in ("user", "assistant"):
        assert torch.equal(model[f"heads.{role}.projection.0.weight"], state[f"heads.{role}.general_projection.0.weight"])
        assert torch.equal(model[f"heads.{role}.risk.bias"], state[f"heads.{role}.general.bias"])
    assert torch.equal(model["backbone.norm.weight"], state["backbone.norm.weight"])


def test_manifest_checks(tmp_path):
    from hs_guard.runtime import verify_model
    root, _ = write_bundle(tmp_path / "b", _cfg(), extra_heads=False)
    verify_model(root)
    man = json.loads((root / "hs_guard.json").read_text())

    def with_manifest(**changes):
        m = dict(man, **changes)
        (root / "hs_guard.json").write_text(json.dumps(m))

    with_manifest(files={k: v for k, v in man["files"].items() if k != "tokenizer.json"})
    with pytest.raises(ValueError, match="missing required assets"):
        verify_model(root)
    with_manifest(files=dict(man["files"], **{"../escape.bin": "0"}))
    with pytest.raises(ValueError, match="Invalid model asset"):
        verify_model(root)
    outside = tmp_path / "outside.bin"
    outside.write_bytes(b"x")
    os.symlink(outside, root / "link.bin")
    with_manifest(files=dict(man["files"], **{"link.bin": "0"}))
    with pytest.raises(ValueError, match="Invalid model asset: link.bin"):
        verify_model(root)
    with_manifest(risk_labels=["unsafe", "safe", "controversial"])
    with pytest.raises(ValueError, match="risk-label order"):
        verify_model(root)
    with_manifest()
    (root / "config.json").write_text((root / "config.json").read_text() + " ")
    with pytest.raises(ValueError, match="checksum mismatch: config.json"):
        verify_model(root)


def test_checkpoint_names_and_shapes_are_strict():
    from hs_guard.model import GuardModel
    cfg = _cfg()
    state = dict(GuardModel.random(cfg, seed=1, device="cpu").weights)
    GuardModel.from_state_dict(cfg, state, device="cpu")
    with pytest.raises(ValueError, match="Unexpected keys"):
        GuardModel.from_state_dict(cfg, dict(state, **{"backbone.extra.weight": torch.zeros(1)}), device="cpu")
    missing = dict(state)
    del missing["backbone.layers.3.self_attn.q_norm.weight"]
    with pytest.raises(ValueError, match="Missing key"):
        GuardModel.from_state_dict(cfg, missing, device="cpu")
    bad = dict(state, **{"backbone.norm.weight": torch.zeros(7, dtype=torch.bfloat16)})
    with pytest.raises(ValueError, match="Shape mismatch"):
        GuardModel.from_state_dict(cfg, bad, device="cpu")
    with pytest.raises(ValueError, match="Missing key"):   # general head requested, checkpoint has none
        GuardModel.from_state_dict(cfg, state, head="general", device="cpu")


def test_head_parameters_reach_the_readouts_unrounded(bundle):
    """The heads' float32 checkpoint values (values bf16 cannot hold) reach both readouts as the reference uses
    them: the streaming readout casts the Linear weights to bf16 and keeps the LayerNorm float32
    (slot_engine_v7.py:44-61); the complete-message readout keeps every head tensor float32 (runtime.py:70-73)."""
    from hs_guard.engine.slot_engine import PreparedWeights
    from hs_guard.engine.whole import fp32_heads
    from hs_guard.runtime import load_bundle
    root, state = bundle
    model, _, _ = load_bundle(root, device="cpu")
    ln_w = torch.stack([state[f"heads.{r}.projection.1.weight"] for r in ("user", "assistant")])
    assert not torch.equal(ln_w, ln_w.to(torch.bfloat16).float())       # not representable in bf16
    pw = PreparedWeights.of(model)
    assert pw.head_ln_w.dtype == torch.float32 and torch.equal(pw.head_ln_w, ln_w)
    assert torch.equal(pw.head_ln_b, torch.stack([state[f"heads.{r}.projection.1.bias"] for r in ("user", "assistant")]))
    assert pw.head_w1.dtype == torch.bfloat16 and pw.head_w2.dtype == torch.bfloat16
    assert torch.equal(pw.head_w1[:512], state["heads.user.projection.0.weight"].to(torch.bfloat16))
    h = fp32_heads(model)
    assert all(t.dtype == torch.float32 for t in h.values())
    assert torch.equal(h["ln_w"], ln_w) and torch.equal(h["w1"][512:], state["heads.assistant.projection.0.weight"])
    assert torch.equal(h["w2"][1], state["heads.assistant.risk.weight"])
