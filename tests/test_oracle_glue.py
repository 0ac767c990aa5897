"""Pins the glue oracle against transformers' Qwen3.5 modules and torch functionals -- CPU only.

The transformers modules are the model-family definitions the reference builds its backbone from; on
inputs that are exact bf16 values they fix each formula (the oracle's explicit rounding points are
compared with the module run in float64 and rounded once, or in bf16 where the module itself rounds).
"""
import numpy as np
import pytest

from oracle import glue as oglue
from oracle.bf16 import bf16

torch = pytest.importorskip("torch")


def _m():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m
    return m


def test_rmsnorm_matches_qwen3_5_rmsnorm():
    m = _m()
    rng = np.random.default_rng(0)
    x = bf16(rng.standard_normal((7, 64)))
    w = bf16(rng.standard_normal(64) * 0.1)
    mod = m.Qwen3_5RMSNorm(64, eps=1e-6)
    mod.weight.data = torch.from_numpy(w)
    ref = mod(torch.from_numpy(x).to(torch.bfloat16)).detach().float().numpy()
    got = oglue.rmsnorm(x, 1.0 + w.astype(np.float32), 1e-6)
    # torch computes in fp32 (one rounding difference at most)
    assert np.mean(got != ref) < 0.01
    np.testing.assert_allclose(got, ref, rtol=2 ** -7)


def test_gated_rmsnorm_matches_module():
    m = _m()
    rng = np.random.default_rng(1)
    x = bf16(rng.standard_normal((9, 128)))
    z = bf16(rng.standard_normal((9, 128)))
    w = bf16(1 + 0.1 * rng.standard_normal(128))
    mod = m.Qwen3_5RMSNormGated(128, eps=1e-6)
    mod.weight.data = torch.from_numpy(w).to(torch.bfloat16)
    ref = mod(torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(z).to(torch.bfloat16)).detach().float().numpy()
    got = oglue.gated_rmsnorm(x, z, w, 1e-6)
    assert np.mean(got != ref) < 0.02
    np.testing.assert_allclose(got, ref, rtol=2 ** -6)


def test_conv_update_matches_causal_conv1d_update():
    m = _m()
    rng = np.random.default_rng(2)
    N, L, C, KS = 2, 5, 12, 4
    qkv = bf16(rng.standard_normal((N, L, C)))
    pool = bf16(rng.standard_normal((3, KS - 1, C)))
    w = bf16(rng.standard_normal((C, 1, KS)) * 0.5)
    slots, lens = np.array([2, 0]), np.array([5, 2])
    out, pool2 = oglue.conv_silu_update(qkv, pool, w, slots, lens)
    for n in range(N):
        state = torch.from_numpy(pool[slots[n]].T.copy()).double()[None]       # [1, C, KS-1]
        h = torch.from_numpy(qkv[n].T.copy()).double()[None]                   # [1, C, L]
        ref = m.causal_conv1d_update(h, state, torch.from_numpy(w[:, 0]).double(), None, None)
        # the oracle rounds the conv to bf16 before SiLU and SiLU's output again (fused_kernels.py:113-115)
        exp = bf16(oglue.silu(bf16(ref[0].T.detach().numpy())))
        np.testing.assert_array_equal(out[n], exp)
        T = lens[n]
        ext = np.concatenate([pool[slots[n]], qkv[n]], 0)
        np.testing.assert_array_equal(pool2[slots[n]], ext[T:T + KS - 1])
    np.testing.assert_array_equal(pool2[1], pool[1])


def test_rope_matches_apply_rotary_pos_emb():
    m = _m()
    rng = np.random.default_rng(3)
    T, Hh, D, rot = 5, 3, 32, 8
    x = bf16(rng.standard_normal((T, Hh, D)))
    w1 = np.ones(D, dtype=np.float32)
    pos = np.array([0, 1, 7, 511, 8000])
    cos, sin = oglue.rope_cos_sin(pos, oglue.inv_freq(rot, 10000.0))
    got = oglue.norm_rope(x, w1, 1e-6, cos, sin)
    normed = oglue.rmsnorm(x, w1, 1e-6)
    qt = torch.from_numpy(normed).to(torch.bfloat16).transpose(0, 1)[None]        # [1, H, T, D]
    ct = torch.from_numpy(cos).to(torch.bfloat16)[None]
    st = torch.from_numpy(sin).to(torch.bfloat16)[None]
    ref, _ = m.apply_rotary_pos_emb(qt, qt, ct, st)
    np.testing.assert_array_equal(got, ref[0].transpose(0, 1).detach().float().numpy())


def test_rope_cos_sin_matches_rotary_embedding():
    m = _m()
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(hidden_size=64, num_attention_heads=2, num_key_value_heads=1, head_dim=32,
                            num_hidden_layers=1, rope_parameters={"rope_type": "default", "rope_theta": 10000.0,
                                                                  "partial_rotary_factor": 0.25,
                                                                  "mrope_section": [1, 1, 2]})
    emb = m.Qwen3_5TextRotaryEmbedding(cfg)
    pos = torch.tensor([[0, 3, 100, 8191]])
    cos, sin = emb(torch.zeros(1, dtype=torch.bfloat16), pos)
    c2, s2 = oglue.rope_cos_sin(pos.numpy()[0], emb.inv_freq.numpy())
    np.testing.assert_array_equal(c2, cos[0].detach().float().numpy())
    np.testing.assert_array_equal(s2, sin[0].detach().float().numpy())
    np.testing.assert_array_equal(oglue.inv_freq(8, 10000.0), emb.inv_freq.numpy())


def test_silu_mul_and_risk_head_match_torch():
    rng = np.random.default_rng(4)
    g = bf16(rng.standard_normal((4, 32)) * 3)
    u = bf16(rng.standard_normal((4, 32)))
    gt, ut = torch.from_numpy(g).to(torch.bfloat16), torch.from_numpy(u).to(torch.bfloat16)
    ref = (torch.nn.functional.silu(gt.float()).to(torch.bfloat16).float() * ut.float()).to(torch.bfloat16)
    np.testing.assert_array_equal(oglue.silu_mul(g, u), ref.detach().float().numpy())
    h = bf16(rng.standard_normal((6, 16)))
    w1, b1 = bf16(rng.standard_normal((8, 16)) * 0.3), bf16(rng.standard_normal(8) * 0.1)
    lw, lb = bf16(1 + 0.1 * rng.standard_normal(8)), bf16(0.1 * rng.standard_normal(8))
    w2, b2 = bf16(rng.standard_normal((3, 8))), bf16(rng.standard_normal(3) * 0.1)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double()
    y = torch.nn.functional.linear(t(h), t(w1), t(b1)).to(torch.bfloat16).double()
    y = torch.nn.functional.silu(torch.nn.functional.layer_norm(y, (8,), t(lw), t(lb)))
    logits = torch.nn.functional.linear(y.to(torch.bfloat16).double(), t(w2), t(b2)).to(torch.bfloat16).double()
    ref = torch.softmax(logits, -1).numpy()
    np.testing.assert_allclose(oglue.risk_probs(h, w1, b1, lw, lb, w2, b2), ref, rtol=1e-6, atol=1e-6)


def test_risk_head_f32_matches_torch_modules():
    """risk_probs_f32 (the complete-message readout) equals the reference's head modules -- nn.Linear,
    nn.LayerNorm, nn.SiLU, nn.Linear in float64 -- applied to hidden.float(), with no bf16 rounding; and it
    differs from the streaming readout (risk_probs) by the three bf16 roundings that readout makes."""
    rng = np.random.default_rng(5)
    h = bf16(rng.standard_normal((7, 16)))
    w1, b1 = rng.standard_normal((8, 16)) * 0.3, rng.standard_normal(8) * 0.1      # fp32 values, not bf16
    lw, lb = 1 + 0.1 * rng.standard_normal(8), 0.1 * rng.standard_normal(8)
    w2, b2 = rng.standard_normal((3, 8)), rng.standard_normal(3) * 0.1
    proj = torch.nn.Sequential(torch.nn.Linear(16, 8), torch.nn.LayerNorm(8), torch.nn.SiLU()).double()
    risk = torch.nn.Linear(8, 3).double()
    with torch.no_grad():
        for p_, v in zip((proj[0].weight, proj[0].bias, proj[1].weight, proj[1].bias, risk.weight, risk.bias),
                         (w1, b1, lw, lb, w2, b2)):
            p_.copy_(torch.from_numpy(v))
        ref = torch.softmax(risk(proj(torch.from_numpy(h).double())), -1).numpy()
    got = oglue.risk_probs_f32(h, w1, b1, lw, lb, w2, b2)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)
    assert np.abs(oglue.risk_probs(h, w1, b1, lw, lb, w2, b2) - got).max() > 1e-6
