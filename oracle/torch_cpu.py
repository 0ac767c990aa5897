"""PyTorch-CPU float32 restatement of the streaming step -- TEST INFRASTRUCTURE ONLY (the CPU baseline).

The reference has no CPU path (it needs CUDA, Triton and FLA: src/hs_guard/runtime.py:101-102,
src/hs_guard/engine/bucketed_engine.py:24), so the baseline the benchmark reports next to the GPU numbers is this
restatement of the same step in PyTorch on the host's cores, in float32 with no bf16 rounding. ``bench.py`` times
it (its ``cpu_baseline`` leg); ``tests/test_oracle_torch_cpu.py`` pins it against the float64 oracle
(``oracle.backbone.StreamOracle`` with rounding off). Nothing in ``hs-guard_amd/`` imports it.

``TorchStream.tick`` follows ``SlotStreamEngineV8._forward`` (src/hs_guard/engine/slot_engine_v8.py:30-89) with
per-slot pools (bucketed_engine.py:37-45) and the reference's separate projections (slot_engine_v8.py:60-72,
74-89):
* GDN layers: in_proj_qkv / z / b / a -> causal conv + SiLU with the pool update (fused_kernels.py:94-136) ->
  the gated delta rule (fused_kernels.py:140-211): token 0 of every row by one batched recurrent update, the
  further tokens of longer rows by the WY/UT chunk form (``gdn_chunk_torch``, the same recurrence; positions
  past a row's length carry beta = 0 and g = 0, which leave the state as it is) -> gated RMSNorm
  (fused_kernels.py:215-233) -> out_proj;
* attention layers: q (with its gate) / k / v projections -> per-head RMSNorm(1 + w) and partial RoPE
  (fused_kernels.py:237-284) -> window-W attention over the ring and the tick's keys
  (ring_attention_kernel.py:7-26; step 0 of every row, then the further steps of longer rows) -> sigmoid(gate)
  -> ring write at pos % W (slot_engine_v8.py:86-88) -> o_proj;
* residual adds, RMSNorm(1 + w), SiLU MLP, final norm; both roles' risk heads (slot_engine_v7.py:58-61);
  ring_pos[slot, pos % W] = pos after all layers (slot_engine_v8.py:41,57).
The tick is held packed (its real tokens only; the reference pads every row to the tick's longest,
pack_inputs, slot_engine_v7.py:7-25), so this baseline spends no work on padding.
"""
import numpy as np
import torch
import torch.nn.functional as F

ROLES = ("user", "assistant")


def _rms(x, w1, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w1


def _span(slots):
    """slots as a slice when they are one ascending run (pool rows then work in place), else the index tensor."""
    if len(slots) and bool((slots[1:] - slots[:-1] == 1).all()):
        return slice(int(slots[0]), int(slots[-1]) + 1)
    return slots


def gdn_chunk_torch(q, k, v, g, beta, S, chunk=64):
    """WY/UT chunk form of the gated delta rule for a batch: q, k [B, T, K] (already l2-normalised, q scaled),
    v [B, T, V], g, beta [B, T], S [B, K, V] (updated in place). Returns o [B, T, V]."""
    B, T, K = q.shape
    out = torch.empty(B, T, v.shape[-1], dtype=q.dtype)
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        C = c1 - c0
        Q, Kc, Vc = q[:, c0:c1], k[:, c0:c1], v[:, c0:c1]
        G = torch.cumsum(g[:, c0:c1], 1)
        bt = beta[:, c0:c1]
        diff = G[:, :, None] - G[:, None, :]
        low = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
        causal = torch.tril(torch.ones(C, C, dtype=torch.bool))
        KT = Kc.transpose(1, 2)
        A = torch.where(low, bt[:, :, None] * (Kc @ KT) * torch.exp(torch.where(low, diff, 0.0)), 0.0)
        Tm = torch.linalg.solve_triangular(torch.eye(C) + A, torch.eye(C).expand(B, C, C), upper=False,
                                           unitriangular=True)
        Wm = Tm @ ((bt * torch.exp(G))[:, :, None] * Kc)
        Um = Tm @ (bt[:, :, None] * Vc)
        Vn = Um - Wm @ S
        P = torch.where(causal, (Q @ KT) * torch.exp(torch.where(causal, diff, 0.0)), 0.0)
        out[:, c0:c1] = (Q * torch.exp(G)[:, :, None]) @ S + P @ Vn
        Kd = (Kc * torch.exp(G[:, -1:] - G)[:, :, None]).transpose(1, 2)
        S.mul_(torch.exp(G[:, -1])[:, None, None]).add_(Kd @ Vn)
    return out


def gdn_step_torch(packed, key_dim, H, K, HV, V, a, b, A_log, dt_bias, state, slots, scale=None):
    """One token per row of the gated delta rule (config 1; fused_kernels.py:140-211 at L = 1): packed
    [N, 2*key_dim + HV*V] (q, k, v after the conv), a, b [N, HV] raw, state [S, HV, K, V] updated in place at rows
    ``slots``. Returns o [N, HV, V]."""
    N = packed.shape[0]
    kh = torch.arange(HV) // (HV // H)
    scale = K ** -0.5 if scale is None else scale
    q = packed[:, :key_dim].reshape(N, H, K)[:, kh]
    k = packed[:, key_dim:2 * key_dim].reshape(N, H, K)[:, kh]
    v = packed[:, 2 * key_dim:].reshape(N, HV, V)
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * scale
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    g = -torch.exp(A_log) * F.softplus(a + dt_bias, threshold=20.0)
    beta = torch.sigmoid(b)
    S = state[slots]
    S.mul_(torch.exp(g)[:, :, None, None])
    vn = beta[..., None] * (v - (k[:, :, None, :] @ S)[:, :, 0])
    S.add_(k[..., :, None] * vn[..., None, :])
    state[slots] = S
    return (q[:, :, None, :] @ S)[:, :, 0]


def ring_decode_torch(q, ring_k, ring_v, new_k, new_v, gate, ring_pos, slots, starts, scale, window):
    """Decode step of the window attention with the ring write (config 2; ring_attention_kernel.py:7-26 at Lb = 1
    with the v8 gate and write, fused_kernels.py:288-356): q [N, Hkv, G, D], ring_k / ring_v [S, Hkv, W+1, D]
    (written in place at column start % W), new_k / new_v [N, Hkv, D], gate [N, Hkv, G, D] (pre-sigmoid),
    ring_pos [S, W+1]. Returns out [N, Hkv, G, D] = softmax attention * sigmoid(gate)."""
    N, hkv, G, D = q.shape
    W = window
    keys = torch.cat([ring_k[slots, :, :W], new_k[:, :, None]], 2)       # [N, Hkv, W + 1, D]
    vals = torch.cat([ring_v[slots, :, :W], new_v[:, :, None]], 2)
    kpos = torch.cat([ring_pos[slots, :W], starts[:, None]], 1)          # [N, W + 1]
    ok = (kpos >= 0) & (kpos <= starts[:, None]) & (kpos > starts[:, None] - W)
    scores = (q @ keys.transpose(2, 3)) * scale
    scores = scores.masked_fill(~ok[:, None, None], float("-inf"))
    out = (torch.softmax(scores, -1) @ vals) * torch.sigmoid(gate)
    col = starts % W
    ring_k[slots, :, col] = new_k
    ring_v[slots, :, col] = new_v
    return out


class TorchStream:
    """Per-slot pools for ``max_slots`` streams (row ``max_slots`` is the scratch slot of padded rows)."""

    def __init__(self, weights, cfg, max_slots, roles=ROLES):
        """weights: name -> tensor (any float dtype, any device); kept as float32 CPU copies."""
        self.w = {k: v.detach().float().cpu().contiguous() for k, v in weights.items()}
        self.cfg, self.roles, self.max_slots = cfg, tuple(roles), max_slots
        types = list(cfg.layer_types)
        self.kind = [(t, sum(1 for u in types[:i] if u == t)) for i, t in enumerate(types)]
        n_gdn, n_att = types.count("linear_attention"), types.count("full_attention")
        S, W = max_slots + 1, cfg.window_tokens
        f32 = torch.float32
        self.rec = torch.zeros(n_gdn, S, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                               cfg.linear_value_head_dim, dtype=f32)
        self.conv = torch.zeros(n_gdn, S, cfg.linear_conv_kernel_dim - 1, cfg.conv_dim, dtype=f32)
        self.ring_k = torch.zeros(n_att, S, cfg.num_key_value_heads, W + 1, cfg.head_dim, dtype=f32)
        self.ring_v = torch.zeros_like(self.ring_k)
        self.ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
        self.length = np.zeros(max_slots, dtype=np.int64)
        rot = cfg.rotary_dim
        self.inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=f32) / rot))

    def fill_synthetic(self, lengths, seed=0):
        """Pools as after contexts of ``lengths`` tokens (state, conv history and ring keys/values random, ring
        positions and lengths exact), for timing steps without prefilling long contexts on the CPU: a step's
        work does not depend on the values of its pools."""
        gen = torch.Generator().manual_seed(seed)
        W = self.cfg.window_tokens
        for t, std in ((self.rec, 0.02), (self.conv, 1.0), (self.ring_k, 1.0), (self.ring_v, 1.0)):
            block = torch.randn(t[:, :1].shape, generator=gen) * std      # one slot's worth, copied to all
            t.copy_(block.expand_as(t))
        cols = torch.arange(W)
        for s, n in enumerate(lengths):
            self.length[s] = n
            # column c holds the latest position p < n with p % W == c, or nothing
            p = n - 1 - torch.remainder(n - 1 - cols, W)
            self.ring_pos[s, :W] = torch.where(p >= 0, p, -1)
            self.ring_pos[s, W] = -1

    # ------------------------------------------------------------------------------------------------
    # A tick is held packed: its T real tokens in request order, token j of row r at index off[r] + j. ``tk``
    # carries the per-token index vectors: row, step, position and the rows' slots, lengths and offsets.

    def _padded(self, x, tk, rows, L):
        """Rows ``rows`` of the packed [T, ...] tensor x as [len(rows), L, ...] (zeros past each row's length)."""
        out = x.new_zeros((len(rows), L) + x.shape[1:])
        j = torch.arange(L)
        ok = j[None] < tk["lens"][rows, None]
        src = (tk["off"][rows, None] + j[None])[ok]
        out[ok] = x[src]
        return out, ok

    def _gdn(self, a, x, idx, tk):
        cfg, w = self.cfg, self.w
        T = x.shape[0]
        H, HV, K, V = (cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                       cfg.linear_value_head_dim)
        C = cfg.conv_dim
        qkv = F.linear(x, w[a + "in_proj_qkv.weight"])
        z = F.linear(x, w[a + "in_proj_z.weight"])
        bb = F.linear(x, w[a + "in_proj_b.weight"])
        aa = F.linear(x, w[a + "in_proj_a.weight"])
        # causal depthwise conv over [history; tick]: tap i of token (r, j) reads time j - 3 + i of row r, from the
        # tick when >= 0, else from the slot's history (pool row j + i)
        pool = self.conv[idx]
        slots, lens, off, row, step = tk["slots"], tk["lens"], tk["off"], tk["row"], tk["step"]
        n = len(slots)
        cw = w[a + "conv1d.weight"].reshape(C, -1)
        ks = cw.shape[1]
        hist = pool[slots].reshape(n * (ks - 1), C)
        src = torch.cat([hist, qkv])
        acc = 0
        for i in range(ks):
            tm = step - (ks - 1) + i
            at = torch.where(tm >= 0, n * (ks - 1) + off[row] + tm, row * (ks - 1) + step + i)
            acc = acc + src[at] * cw[:, i]
        conv = F.silu(acc)
        # history update: times len - 3 .. len - 1 of every row
        j = torch.arange(ks - 1)
        tm = lens[:, None] - (ks - 1) + j[None]
        at = torch.where(tm >= 0, n * (ks - 1) + off[:, None] + tm, torch.arange(n)[:, None] * (ks - 1) + lens[:, None] + j)
        pool[slots] = src[at]
        # gated delta rule
        kh = torch.arange(HV) // (HV // H)
        q = conv[:, :cfg.key_dim].reshape(T, H, K)[:, kh]
        k = conv[:, cfg.key_dim:2 * cfg.key_dim].reshape(T, H, K)[:, kh]
        v = conv[:, 2 * cfg.key_dim:].reshape(T, HV, V)
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * K ** -0.5
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        g = -torch.exp(w[a + "A_log"]) * F.softplus(aa + w[a + "dt_bias"], threshold=20.0)
        beta = torch.sigmoid(bb)
        o = torch.empty(T, HV, V)
        rec = self.rec[idx]
        # token 0 of every row: one recurrent step, in place when the rows' slots form one run
        sel = _span(slots)
        S = rec[sel]                                                      # [n, HV, K, V]
        t0 = off
        k0 = k[t0]
        S.mul_(torch.exp(g[t0])[:, :, None, None])
        vn = beta[t0][..., None] * (v[t0] - (k0[:, :, None, :] @ S)[:, :, 0])
        S.add_(k0[..., :, None] * vn[..., None, :])
        o[t0] = (q[t0][:, :, None, :] @ S)[:, :, 0]
        if not isinstance(sel, slice):
            rec[sel] = S
        # the further tokens of longer rows in the chunk form (padded positions: beta = 0, g = 0, no change)
        multi = torch.nonzero(lens > 1)[:, 0]
        if len(multi):
            L = int(lens.max()) - 1
            m = len(multi)
            sub = {"lens": lens[multi] - 1, "off": off[multi] + 1}
            pq, ok = self._padded(q, sub, torch.arange(m), L)
            pk, _ = self._padded(k, sub, torch.arange(m), L)
            pv, _ = self._padded(v, sub, torch.arange(m), L)
            pg, _ = self._padded(g, sub, torch.arange(m), L)
            pb, _ = self._padded(beta, sub, torch.arange(m), L)
            sm = _span(slots[multi])
            Sf = rec[sm].reshape(m * HV, K, V)
            flat = lambda t: t.transpose(1, 2).reshape(m * HV, L, -1)
            out = gdn_chunk_torch(flat(pq), flat(pk), flat(pv), pg.transpose(1, 2).reshape(m * HV, L),
                                  pb.transpose(1, 2).reshape(m * HV, L), Sf)
            o[(sub["off"][:, None] + torch.arange(L)[None])[ok]] = out.reshape(m, HV, L, V).transpose(1, 2)[ok]
            if not isinstance(sm, slice):
                rec[sm] = Sf.reshape(m, HV, K, V)
        # gated RMSNorm and out_proj
        normed = o * torch.rsqrt((o * o).mean(-1, keepdim=True) + cfg.rms_norm_eps) * w[a + "norm.weight"]
        gated = (normed * F.silu(z.reshape(T, HV, V))).reshape(T, HV * V)
        return F.linear(gated, w[a + "out_proj.weight"])

    def _attention(self, a, x, idx, tk, cos, sin):
        cfg, w = self.cfg, self.w
        T = x.shape[0]
        hq, hkv, D, W = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.window_tokens
        G = hq // hkv
        slots, lens, off, pos = tk["slots"], tk["lens"], tk["off"], tk["pos"]
        n = len(slots)
        qp = F.linear(x, w[a + "q_proj.weight"]).reshape(T, hq, 2 * D)
        q, gate = qp[..., :D], qp[..., D:]
        k = F.linear(x, w[a + "k_proj.weight"]).reshape(T, hkv, D)
        v = F.linear(x, w[a + "v_proj.weight"]).reshape(T, hkv, D)

        def norm_rope(t, w1):
            t = _rms(t, w1, cfg.rms_norm_eps)
            rot = cos.shape[-1]
            tr = t[..., :rot]
            half = rot // 2
            rh = torch.cat([-tr[..., half:], tr[..., :half]], -1)
            return torch.cat([tr * cos[:, None] + rh * sin[:, None], t[..., rot:]], -1)
        q = norm_rope(q, 1.0 + w[a + "q_norm.weight"])
        k = norm_rope(k, 1.0 + w[a + "k_norm.weight"])
        rk, rv = self.ring_k[idx], self.ring_v[idx]
        scale = D ** -0.5
        rpos = self.ring_pos[slots, :W]

        def attend(qg, ring_k, ring_v, kt, vt, kpos, qpos, qvalid):
            """qg [m, hkv, G*L, D] of query steps qpos / qvalid [m, L] over the ring and the keys kt, vt
            [m, hkv, L', D] at kpos [m, W + L']."""
            m, L = qpos.shape
            ok = (kpos[:, None] >= 0) & (kpos[:, None] <= qpos[..., None]) & (kpos[:, None] > qpos[..., None] - W)
            ok = ok & qvalid[..., None]
            sc = torch.cat([qg @ ring_k.transpose(2, 3), qg @ kt.transpose(2, 3)], -1) * scale
            mask = ok[:, None, None].expand(m, hkv, G, L, kpos.shape[1]).reshape(m, hkv, G * L, -1)
            pr = torch.softmax(sc.masked_fill(~mask, float("-inf")), -1).nan_to_num(0.0)
            return pr[..., :W] @ ring_v + pr[..., W:] @ vt

        att = torch.empty(T, hq, D)
        # step 0 of every row over the ring and its own key, on the pool rows in place when the slots form a run
        sel = _span(slots)
        t0 = off
        a0 = attend(q[t0].reshape(n, hkv, G, D), rk[sel, :, :W], rv[sel, :, :W], k[t0][:, :, None],
                    v[t0][:, :, None], torch.cat([rpos, pos[t0][:, None]], 1), pos[t0][:, None],
                    torch.ones(n, 1, dtype=torch.bool))
        att[t0] = a0.reshape(n, hq, D)
        # the further steps of longer rows, over the ring and the tick's keys
        multi = torch.nonzero(lens > 1)[:, 0]
        if len(multi):
            L = int(lens.max())
            m = len(multi)
            pq, ok = self._padded(q, tk, multi, L)
            pk, _ = self._padded(k, tk, multi, L)
            pv, _ = self._padded(v, tk, multi, L)
            ppos = off[multi, None] + torch.arange(L)[None]
            qpos = pos[off[multi]][:, None] + torch.arange(L)[None]
            qg = pq.reshape(m, L, hkv, G, D).permute(0, 2, 3, 1, 4).reshape(m, hkv, G * L, D)
            kpos = torch.cat([rpos[multi], torch.where(ok, qpos, -1)], 1)
            sm = _span(slots[multi])
            am = attend(qg, rk[sm, :, :W], rv[sm, :, :W], pk.transpose(1, 2), pv.transpose(1, 2), kpos, qpos, ok)
            am = am.reshape(m, hkv, G, L, D).permute(0, 3, 1, 2, 4).reshape(m, L, hq, D)
            later = ok.clone()
            later[:, 0] = False
            att[ppos[later]] = am[later]
        att = att * torch.sigmoid(gate)
        # ring write of every token at pos % W after all reads (a tick's steps own distinct columns)
        rk[slots[tk["row"]], :, pos % W] = k
        rv[slots[tk["row"]], :, pos % W] = v
        return F.linear(att.reshape(T, hq * D), w[a + "o_proj.weight"])

    @torch.inference_mode()
    def tick(self, requests):
        """requests: [(slot, ids)] with unique slots, each with 1 to min(64, W) ids. Returns probs
        [roles, n, lb, 3] (lb the longest request; zeros past each row's length)."""
        cfg, w = self.cfg, self.w
        n = len(requests)
        slots = torch.tensor([s for s, _ in requests], dtype=torch.long)
        lens = torch.tensor([len(ids) for _, ids in requests], dtype=torch.long)
        off = torch.cumsum(lens, 0) - lens
        T = int(lens.sum())
        row = torch.repeat_interleave(torch.arange(n), lens)
        step = torch.arange(T) - off[row]
        starts = torch.as_tensor(self.length[slots.numpy()])
        pos = starts[row] + step
        tk = {"slots": slots, "lens": lens, "off": off, "row": row, "step": step, "pos": pos}
        ids = torch.as_tensor([i for _, t in requests for i in t], dtype=torch.long)
        freqs = pos[:, None].float() * self.inv_freq
        emb = torch.cat([freqs, freqs], -1)
        cos, sin = emb.cos(), emb.sin()
        eps = cfg.rms_norm_eps
        hidden = w["backbone.embed_tokens.weight"][ids]
        for i, (kind, idx) in enumerate(self.kind):
            p = f"backbone.layers.{i}."
            x = _rms(hidden, 1.0 + w[p + "input_layernorm.weight"], eps)
            if kind == "linear_attention":
                mix = self._gdn(p + "linear_attn.", x, idx, tk)
            else:
                mix = self._attention(p + "self_attn.", x, idx, tk, cos, sin)
            hidden = hidden + mix
            x = _rms(hidden, 1.0 + w[p + "post_attention_layernorm.weight"], eps)
            gu = F.silu(F.linear(x, w[p + "mlp.gate_proj.weight"])) * F.linear(x, w[p + "mlp.up_proj.weight"])
            hidden = hidden + F.linear(gu, w[p + "mlp.down_proj.weight"])
        final = _rms(hidden, 1.0 + w["backbone.norm.weight"], eps)
        lb = int(lens.max())
        probs = torch.zeros(len(self.roles), n, lb, 3)
        for ri, r in enumerate(self.roles):
            h = f"heads.{r}."
            y = F.linear(final, w[h + "projection.0.weight"], w[h + "projection.0.bias"])
            y = F.silu(F.layer_norm(y, (y.shape[-1],), w[h + "projection.1.weight"], w[h + "projection.1.bias"],
                                    cfg.layer_norm_eps))
            probs[ri, row, step] = torch.softmax(F.linear(y, w[h + "risk.weight"], w[h + "risk.bias"]), -1)
        self.ring_pos[slots[row], pos % cfg.window_tokens] = pos
        self.length[slots.numpy()] += lens.numpy()
        return probs
