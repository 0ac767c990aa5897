"""GPU parity of the kernel wrappers with the reference engine's own contracts (hs_guard.engine.kernels).

The reference engine imports nine kernel functions (src/hs_guard/engine/slot_engine_v8.py:6-7). Each wrapper is
checked here against its oracle function on the same bf16 inputs (bit-exact where the formula has one rounding,
otherwise the bf16 bars of the glue tests), and then all nine are composed into a two-layer [GDN, attention] step
in the order the reference's _forward / _gdn8 / _attention8 call them (slot_engine_v8.py:30-89), with the
reference's padded [n, lb] layout, plain torch GEMMs and torch's own mean for every variance. That step is held to
the north-star bar (per-token 1 - p(safe) within 2e-3) against the CPU oracle whose products are made bitwise the
composition's (the same torch.mm call on the same rows), with ring_pos and lengths bit-exact.
"""
import numpy as np
import pytest
import torch
from parity_helpers import close_bf16 as _close

from oracle import glue as oglue
from oracle.bf16 import bf16

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PROB_TOL = 2e-3


def _np(t):
    return t.detach().float().cpu().numpy()


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("rows,width", [(37, 1024), (5, 1001)])
def test_add_square(rows, width):
    """bf16(res + mix) and its fp32 squares bit for bit (one rounding each); mixed None returns residual itself."""
    from hs_guard.engine.kernels import add_square
    print(f"[contract] add_square {rows}x{width}", flush=True)
    rng = np.random.default_rng(10)
    res, mix = bf16(rng.standard_normal((rows, width))), bf16(rng.standard_normal((rows, width)) * 0.3)
    res_d = _bf(res).view(1, rows, width)
    out, sq = add_square(res_d, _bf(mix).view(1, rows, width))
    h = bf16(res + mix)
    np.testing.assert_array_equal(_np(out)[0], h)
    assert sq.dtype == torch.float32 and sq.shape == res_d.shape
    np.testing.assert_array_equal(_np(sq)[0], (h.astype(np.float64) ** 2).astype(np.float32))
    same, sq0 = add_square(res_d)
    assert same is res_d
    np.testing.assert_array_equal(_np(sq0)[0], (res.astype(np.float64) ** 2).astype(np.float32))


@pytest.mark.parametrize("rows,width", [(37, 1024), (5, 1001)])
def test_rms_finish(rows, width):
    """Given var = sq.mean(-1) as the reference engine computes it (torch, on the GPU)."""
    from hs_guard.engine.kernels import add_square, rms_finish
    print(f"[contract] rms_finish {rows}x{width}", flush=True)
    rng = np.random.default_rng(11)
    x = bf16(rng.standard_normal((rows, width)))
    w1 = (1.0 + bf16(rng.standard_normal(width) * 0.02)).astype(np.float32)
    x_d = _bf(x)
    _, sq = add_square(x_d)
    var = sq.mean(-1, keepdim=True)
    out = rms_finish(x_d, var, torch.from_numpy(w1).to(DEV), 1e-6)
    _close(_np(out), oglue.rms_finish(x, _np(var), w1, 1e-6), "rms_finish", ulps=1)


@pytest.mark.parametrize("shape", [(2, 11, 3584), (7, 1001)])
def test_silu_mul(shape):
    from hs_guard.engine.kernels import silu_mul
    print(f"[contract] silu_mul {shape}", flush=True)
    rng = np.random.default_rng(12)
    g, u = bf16(rng.standard_normal(shape) * 2), bf16(rng.standard_normal(shape))
    out = silu_mul(_bf(g), _bf(u))
    assert out.shape == shape and out.dtype == torch.bfloat16
    _close(_np(out), oglue.silu_mul(g, u), "silu_mul")


def test_conv_silu_update():
    """The reference's padded layout: every position of every row computed, pools updated only where lens > 0,
    bit-exact."""
    from hs_guard.engine.kernels import conv_silu_update
    print("[contract] conv_silu_update", flush=True)
    rng = np.random.default_rng(13)
    N, L, C, S = 5, 9, 2048, 7
    slots, lens = np.array([4, 0, 6, 2, 1]), np.array([9, 3, 0, 1, 9])
    qkv = bf16(rng.standard_normal((N, L, C)))
    pool = bf16(rng.standard_normal((S, 3, C)))
    w = bf16(rng.standard_normal((C, 1, 4)) * 0.5)
    ref, ref_pool = oglue.conv_silu_update(qkv, pool, w, slots, lens)
    pool_d = _bf(pool)
    out = conv_silu_update(_bf(qkv), pool_d, _bf(w), torch.from_numpy(slots).to(DEV), torch.from_numpy(lens).to(DEV))
    atol = 16 * 2.0 ** -24 * float(np.abs(w).max()) * float(max(np.abs(qkv).max(), np.abs(pool).max()))
    _close(_np(out), ref, "conv_silu_update", atol=atol, ulps=2)
    np.testing.assert_array_equal(_np(pool_d), ref_pool)


@pytest.mark.parametrize("rows,width", [(29 * 4, 128), (3, 250)])
def test_gated_finish(rows, width):
    from hs_guard.engine.kernels import gated_finish
    print(f"[contract] gated_finish {rows}x{width}", flush=True)
    rng = np.random.default_rng(14)
    x, z = bf16(rng.standard_normal((rows, width))), bf16(rng.standard_normal((rows, width)))
    w = bf16(1.0 + rng.standard_normal(width) * 0.1)
    x_d = _bf(x)
    var = (x_d.float() ** 2).mean(-1, keepdim=True)
    out = gated_finish(x_d, var, _bf(w), _bf(z), 1e-6)
    _close(_np(out), oglue.gated_finish(x, _np(var), w, z, 1e-6), "gated_finish")


def test_square_rows_and_norm_rope_layouts():
    """square_rows reads the q heads out of the q|gate projection rows (bit-exact squares); norm_rope writes q in
    the grouped [N, Hkv, G*Lb, D] layout and k in [N, Hkv, Lb, D], each head at its reference position."""
    from hs_guard.engine.kernels import norm_rope, square_rows
    print("[contract] square_rows + norm_rope", flush=True)
    rng = np.random.default_rng(15)
    n, lb, hq, hkv, D, rot = 3, 5, 8, 2, 256, 64
    G = hq // hkv
    qp = bf16(rng.standard_normal((n, lb, hq * 2 * D)))
    kp = bf16(rng.standard_normal((n, lb, hkv * D)))
    pos = np.array([0, 511, 8000])[:, None] + np.arange(lb)[None]
    cos, sin = oglue.rope_cos_sin(pos, oglue.inv_freq(rot, 10000.0))
    qw1 = (1.0 + bf16(rng.standard_normal(D) * 0.02)).astype(np.float32)
    kw1 = (1.0 + bf16(rng.standard_normal(D) * 0.02)).astype(np.float32)
    qp_d, kp_d, cos_d, sin_d = _bf(qp), _bf(kp), _bf(cos), _bf(sin)
    sq_q = square_rows(qp_d, n * lb, hq, hq * 2 * D, 2 * D, D)
    q_heads = qp.reshape(n, lb, hq, 2 * D)[..., :D]
    np.testing.assert_array_equal(_np(sq_q).reshape(n, lb, hq, D), (q_heads.astype(np.float64) ** 2).astype(np.float32))
    var_q = sq_q.view(n, lb, hq, D).mean(-1, keepdim=True)
    sq_k = square_rows(kp_d, n * lb, hkv, hkv * D, D, D)
    var_k = sq_k.view(n, lb, hkv, D).mean(-1, keepdim=True)
    q = norm_rope(qp_d, var_q, torch.from_numpy(qw1).to(DEV), cos_d, sin_d, 1e-6, n, lb, hq, G, hq * 2 * D, 2 * D, D)
    k = norm_rope(kp_d, var_k, torch.from_numpy(kw1).to(DEV), cos_d, sin_d, 1e-6, n, lb, hkv, 1, hkv * D, D, D)
    assert q.shape == (n, hkv, G * lb, D) and k.shape == (n, hkv, lb, D)
    q_ref = oglue.norm_rope_given(q_heads, _np(var_q), qw1, 1e-6, cos, sin)            # [n, lb, hq, D]
    k_ref = oglue.norm_rope_given(kp.reshape(n, lb, hkv, D), _np(var_k), kw1, 1e-6, cos, sin)
    # head h*G + g of step l sits at row g*lb + l of kv head h
    q_ref = q_ref.reshape(n, lb, hkv, G, D).transpose(0, 2, 3, 1, 4).reshape(n, hkv, G * lb, D)
    _close(_np(q), q_ref, "norm_rope q (grouped layout)")
    _close(_np(k), k_ref.transpose(0, 2, 1, 3), "norm_rope k")


# ---------------------------------------------------------------------------------------------------------------
# The nine wrappers composed as the reference engine composes them
# ---------------------------------------------------------------------------------------------------------------
def _lin(x, w, bias=None):
    """The composition's product (and, through _oracle_gemm, the oracle's): one torch.mm over the [n*lb, K] rows."""
    x2 = x.reshape(-1, x.shape[-1])
    y = torch.mm(x2, w.t()) if bias is None else torch.addmm(bias, x2, w.t())
    return y.view(*x.shape[:-1], w.shape[0])


class ContractStep:
    """One tick of the reference engine's program (slot_engine_v8.py:30-89) on this library's contract wrappers:
    embedding, rotary cos/sin, add_square + rms_finish around every layer, the GDN mixer as conv_silu_update ->
    gdn_slot_v8 -> gated_finish, the attention mixer as square_rows -> norm_rope -> ring_attention_v8 (with the
    Lb > 1 ring scatter in torch), silu_mul in the MLP, the risk heads, and the ring_pos update, all in the padded
    [n, lb] layout of pack_inputs. Test code: it exists to exercise the wrappers the way a swapped import would."""

    def __init__(self, model, max_slots):
        cfg = model.config
        self.cfg, self.w = cfg, model.weights
        self.max_slots = max_slots
        S = max_slots + 1
        types = list(cfg.layer_types)
        self.kind = [(t, types[:i].count(t)) for i, t in enumerate(types)]
        n_gdn, n_att = types.count("linear_attention"), types.count("full_attention")
        W, D = cfg.window_tokens, cfg.head_dim
        self.rec = torch.zeros(n_gdn, S, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                               cfg.linear_value_head_dim, device=DEV)
        self.conv = torch.zeros(n_gdn, S, cfg.linear_conv_kernel_dim - 1, cfg.conv_dim, dtype=torch.bfloat16,
                                device=DEV)
        self.ring_k = torch.zeros(n_att, S, cfg.num_key_value_heads, W + 1, D, dtype=torch.bfloat16, device=DEV)
        self.ring_v = torch.zeros_like(self.ring_k)
        self.ring_pos = torch.full((S, W + 1), -1, dtype=torch.long, device=DEV)
        self.length = np.zeros(max_slots, dtype=np.int64)
        rot = cfg.rotary_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))).to(DEV)
        self.w1 = lambda name: (1.0 + self.w[name].float()).contiguous()

    def tick(self, requests):
        from hs_guard._lib import check, lib
        from hs_guard.engine import kernels as K
        cfg, w = self.cfg, self.w
        n = len(requests)
        lb = max(len(ids) for _, ids in requests)
        ids = np.zeros((n, lb), dtype=np.int64)
        lens = np.array([len(t) for _, t in requests], dtype=np.int64)
        for r, (_, t) in enumerate(requests):
            ids[r, :len(t)] = t
        slots_np = np.array([s for s, _ in requests], dtype=np.int64)
        starts_np = self.length[slots_np]
        ids_d, lens_d = torch.from_numpy(ids).to(DEV), torch.from_numpy(lens).to(DEV)
        slots, starts = torch.from_numpy(slots_np).to(DEV), torch.from_numpy(starts_np).to(DEV)
        W, eps = cfg.window_tokens, cfg.rms_norm_eps
        steps = torch.arange(lb, device=DEV)
        valid = steps[None] < lens_d[:, None]
        pos = starts[:, None] + steps[None]
        hidden = w["backbone.embed_tokens.weight"][ids_d]
        freqs = pos.float()[..., None] * self.inv_freq
        emb = torch.cat([freqs, freqs], -1)
        cos, sin = emb.cos().to(torch.bfloat16).contiguous(), emb.sin().to(torch.bfloat16).contiguous()
        ring_col = torch.where(valid, pos % W, W)
        _, sq = K.add_square(hidden)
        normed = K.rms_finish(hidden, sq.mean(-1, keepdim=True), self.w1("backbone.layers.0.input_layernorm.weight"),
                              eps)
        nl = len(self.kind)
        for i, (kind, idx) in enumerate(self.kind):
            p = f"backbone.layers.{i}."
            if kind == "linear_attention":
                mixed = self._gdn(p + "linear_attn.", normed, idx, slots, lens_d)
            else:
                mixed = self._attention(p + "self_attn.", normed, idx, slots, starts, lens_d, cos, sin, ring_col)
            hidden, sq = K.add_square(hidden, mixed)
            normed = K.rms_finish(hidden, sq.mean(-1, keepdim=True), self.w1(p + "post_attention_layernorm.weight"),
                                  eps)
            act = K.silu_mul(_lin(normed, w[p + "mlp.gate_proj.weight"]), _lin(normed, w[p + "mlp.up_proj.weight"]))
            hidden, sq = K.add_square(hidden, _lin(act, w[p + "mlp.down_proj.weight"]))
            nxt = f"backbone.layers.{i + 1}.input_layernorm.weight" if i + 1 < nl else "backbone.norm.weight"
            normed = K.rms_finish(hidden, sq.mean(-1, keepdim=True), self.w1(nxt), eps)
        # risk heads: each role's first Linear as its own biased product, then the library's head kernel
        roles = ("user", "assistant")
        E = cfg.head_hidden
        y = torch.cat([_lin(normed, w[f"heads.{r}.projection.0.weight"].to(torch.bfloat16),
                            w[f"heads.{r}.projection.0.bias"].to(torch.bfloat16)) for r in roles], -1).contiguous()
        ln_w = torch.stack([w[f"heads.{r}.projection.1.weight"] for r in roles]).float().contiguous()
        ln_b = torch.stack([w[f"heads.{r}.projection.1.bias"] for r in roles]).float().contiguous()
        w2 = torch.stack([w[f"heads.{r}.risk.weight"] for r in roles]).to(torch.bfloat16).contiguous()
        b2 = torch.stack([w[f"heads.{r}.risk.bias"] for r in roles]).to(torch.bfloat16).contiguous()
        probs = torch.empty(len(roles), n * lb, 3, dtype=torch.float32, device=DEV)
        check(lib().hsg_risk_head(y.data_ptr(), len(roles) * E, ln_w.data_ptr(), ln_b.data_ptr(), w2.data_ptr(),
                                  b2.data_ptr(), cfg.layer_norm_eps, len(roles), E, probs.data_ptr(), n * lb,
                                  torch.cuda.current_stream(DEV).cuda_stream), "hsg_risk_head")
        self.ring_pos[slots[:, None], ring_col] = torch.where(valid, pos, -1)
        self.length[slots_np] += lens
        return probs.view(len(roles), n, lb, 3).cpu().numpy(), lens

    def _gdn(self, a, x, g, slots, lens):
        from hs_guard.engine import kernels as K
        cfg, w = self.cfg, self.w
        nb, lb, _ = x.shape
        V = cfg.linear_value_head_dim
        qkv = _lin(x, w[a + "in_proj_qkv.weight"])
        z = _lin(x, w[a + "in_proj_z.weight"])
        b, av = _lin(x, w[a + "in_proj_b.weight"]), _lin(x, w[a + "in_proj_a.weight"])
        packed = K.conv_silu_update(qkv, self.conv[g], w[a + "conv1d.weight"], slots, lens)
        o, sq = K.gdn_slot_v8(packed, cfg.key_dim, cfg.linear_num_key_heads, cfg.linear_key_head_dim,
                              cfg.linear_num_value_heads, V, av, b, w[a + "A_log"], w[a + "dt_bias"], self.rec[g],
                              slots, lens)
        out = K.gated_finish(o.view(-1, V), sq.view(-1, V).mean(-1, keepdim=True), w[a + "norm.weight"],
                             z.view(-1, V), cfg.rms_norm_eps)
        return _lin(out.view(nb, lb, -1), w[a + "out_proj.weight"])

    def _attention(self, a, x, idx, slots, starts, lens, cos, sin, ring_col):
        from hs_guard.engine import kernels as K
        cfg, w = self.cfg, self.w
        nb, lb, _ = x.shape
        D, hq, hkv, eps = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.rms_norm_eps
        qp, kp, vp = _lin(x, w[a + "q_proj.weight"]), _lin(x, w[a + "k_proj.weight"]), _lin(x, w[a + "v_proj.weight"])
        var_q = K.square_rows(qp, nb * lb, hq, hq * 2 * D, 2 * D, D).view(nb, lb, hq, D).mean(-1, keepdim=True)
        var_k = K.square_rows(kp, nb * lb, hkv, hkv * D, D, D).view(nb, lb, hkv, D).mean(-1, keepdim=True)
        q = K.norm_rope(qp, var_q, self.w1(a + "q_norm.weight"), cos, sin, eps, nb, lb, hq, hq // hkv, hq * 2 * D,
                        2 * D, D)
        k = K.norm_rope(kp, var_k, self.w1(a + "k_norm.weight"), cos, sin, eps, nb, lb, hkv, 1, hkv * D, D, D)
        write = lb == 1
        out = K.ring_attention_v8(q, self.ring_k[idx], self.ring_v[idx], k, vp, qp, self.ring_pos, slots, starts, lens,
                                  D ** -0.5, cfg.window_tokens, write)
        if not write:
            self.ring_k[idx, slots[:, None], :, ring_col] = k.transpose(1, 2)
            self.ring_v[idx, slots[:, None], :, ring_col] = vp.view(nb, lb, hkv, D)
        return _lin(out, w[a + "o_proj.weight"])


def _oracle_gemm(cfg):
    """The oracle's products made bitwise the composition's: its fused projections are split back into the
    reference's separate Linears and each runs as _lin on the GPU over the same [n*lb, K] rows."""
    C, VD, HV = cfg.conv_dim, cfg.value_dim, cfg.linear_num_value_heads
    hq, hkv, D, I, E = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size,
                        cfg.head_hidden)
    splits = {C + VD + 2 * HV: [C, VD, HV, HV], hq * 2 * D + 2 * hkv * D: [hq * 2 * D, hkv * D, hkv * D],
              2 * I: [I, I]}
    cache = {}

    def parts(w, sizes):
        key = (id(w), w.shape)
        if key not in cache:
            cuts = np.cumsum([0] + sizes)
            cache[key] = (w, [_bf(w[cuts[j]:cuts[j + 1]]).contiguous() for j in range(len(sizes))])
        return cache[key][1]

    def gemm(x, w, bias, lens):
        xd = _bf(x)
        if bias is not None:
            ws = parts(w, [E] * (w.shape[0] // E))
            bs = [_bf(bias[j * E:(j + 1) * E]) for j in range(len(ws))]
            y = torch.cat([_lin(xd, wj, bj) for wj, bj in zip(ws, bs)], -1)
        elif w.shape[0] in splits and w.shape[1] == cfg.hidden_size:
            y = torch.cat([_lin(xd, wj) for wj in parts(w, splits[w.shape[0]])], -1)
        else:
            y = _lin(xd, parts(w, [w.shape[0]])[0])
        return y.float().cpu().numpy()
    return gemm


def _schedule(rng, vocab):
    """Ticks of at most 32 tokens (the window) over 4 slots: prefill-like rows, single-token (Lb == 1, the
    reference's in-kernel ring write) and mixed ticks, wrapping every ring."""
    ticks = [[(0, rng.integers(0, vocab, 20).tolist()), (3, rng.integers(0, vocab, 7).tolist())],
             [(3, [5]), (1, rng.integers(0, vocab, 30).tolist()), (0, [7])],
             [(2, rng.integers(0, vocab, 32).tolist())],
             [(s, [int(rng.integers(0, vocab))]) for s in (0, 1, 2, 3)]]
    for _ in range(5):
        ticks.append([(s, rng.integers(0, vocab, int(rng.choice([1, 1, 3, 9]))).tolist()) for s in (0, 1, 3)])
    ticks.append([(s, [int(rng.integers(0, vocab))]) for s in (3, 1)])
    ticks.append([(1, [1]), (2, rng.integers(0, vocab, 25).tolist())])
    return ticks


def _small_net():
    """Two layers [GDN, attention] with random-init weights N(0, 0.005). At this scale the oracle's own fp32-level
    noise floor (oracle.bf16.perturbed(1) against the plain oracle, on this schedule) is 4.2e-4, so the 2e-3 bar
    has a margin of about 5x; at N(0, 0.02) the same floor is 3.0e-3 and no fp32 evaluation can be held to 2e-3
    (tests/test_oracle_backbone.py::test_noise_floor_scales_with_weights). A dropped attention gate moves cut scores
    by 1.1e-2 at this scale."""
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=2,
                      layer_types=["linear_attention", "full_attention"], intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    model_cpu = GuardModel.random(cfg, seed=0, device="cpu", std=0.005)
    return cfg, model_cpu, {k: v.float().numpy() for k, v in model_cpu.weights.items()}


def _cut_diff(got, lens, ref):
    return max(float(np.abs(got[:, r, :lens[r], 0] - ref[:, r, :lens[r], 0]).max()) for r in range(len(lens)))


def test_reference_composition_matches_oracle():
    """A [GDN, attention] net run tick by tick through the nine wrappers in the reference engine's order: per-token
    cut scores within 2e-3 of the oracle (same products), ring_pos and lengths bit-exact, the recurrent state within
    1e-3 relative, the conv history (raw projections, so one bf16 flip of an input row moves a few) within two bf16
    ulps on all but 1% of its values. A planted mistake in the oracle (attention gate dropped) fails the bar by more
    than 4x."""
    import oracle.ring as oring
    from oracle.backbone import StreamOracle
    print("[contract] nine wrappers composed as the reference engine vs oracle", flush=True)
    cfg, model_cpu, weights = _small_net()
    model = model_cpu.to("cuda:0")
    step = ContractStep(model, 4)
    orc = StreamOracle(weights, cfg, 4)
    gemm = _oracle_gemm(cfg)
    worst = 0.0
    for t, tick in enumerate(_schedule(np.random.default_rng(0), cfg.vocab_size)):
        got, lens = step.tick(tick)
        ref, _ = orc.tick(tick, gemm=gemm)
        d = _cut_diff(got, lens, ref)
        worst = max(worst, d)
        assert d <= PROB_TOL, f"tick {t}: cut-score diff {d:.2e}"
    print(f"[contract] worst cut-score diff {worst:.2e}", flush=True)
    orig = oring.ring_attention_v8
    oring.ring_attention_v8 = lambda q, rk, rv, nk, value, gate, *a, **k: orig(q, rk, rv, nk, value,
                                                                               np.full_like(gate, 30.0), *a, **k)
    try:
        tick = _schedule(np.random.default_rng(0), cfg.vocab_size)[0]
        got, lens = ContractStep(model, 4).tick(tick)
        bad, _ = StreamOracle(weights, cfg, 4).tick(tick, gemm=gemm)
        assert _cut_diff(got, lens, bad) > 4 * PROB_TOL
    finally:
        oring.ring_attention_v8 = orig
    np.testing.assert_array_equal(step.length, orc.length)
    np.testing.assert_array_equal(step.ring_pos.cpu().numpy(), orc.ring_pos)
    _close(_np(step.conv), orc.conv, "conv history", frac=1e-2, ulps=2)
    rec = step.rec.double().cpu().numpy()
    for s in range(4):
        rel = np.linalg.norm(rec[:, s] - orc.rec[:, s]) / np.linalg.norm(orc.rec[:, s])
        assert rel < 1e-3, f"slot {s} state rel err {rel:.2e}"
