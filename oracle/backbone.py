"""Whole streaming step on the CPU (test infrastructure only).

``StreamOracle.tick`` restates ``SlotStreamEngineV8._forward`` (src/hs_guard/engine/slot_engine_v8.py:30-89)
in the reference's padded [n, lb] layout of ``pack_inputs`` (slot_engine_v7.py:7-25), with its per-slot
pools (bucketed_engine.py:37-45, slot_engine.py:14-17): GDN layers run conv_silu_update -> gdn_slot_step
-> gated RMSNorm -> out_proj; attention layers run q/k RMSNorm + RoPE -> ring attention with gate -> ring
scatter -> o_proj; every layer ends with add+RMSNorm -> SiLU-MLP -> add+RMSNorm; after the last layer both
risk heads are read out and ring_pos is updated. GEMMs are fp32 products of bf16 values rounded to bf16
(autocast semantics); the recurrent state is float64.

Each piece is the oracle function pinned in its own test module; the composition is pinned by
``tests/test_oracle_backbone.py`` against transformers' Qwen3_5TextModel forward over the whole sequence
(the complete-message path the streaming engine must reproduce, docs/ENGINE.md:13).

The projections of one input are computed as one product with the weights concatenated (GDN
qkv|z|b|a, attention q|k|v, MLP gate|up, both heads' first Linear): each output column is its own dot
product, so this equals the separate products. ``tick(requests, gemm=...)`` takes the product as a
parameter -- ``gemm(x [n, lb, K], w [N, K], bias or None, lens) -> [n, lb, N]`` -- so a test can make the
oracle's products bitwise those of the engine under test and compare everything else exactly.
"""
import numpy as np

from . import gdn as ogdn
from . import glue as oglue
from . import pack as opack
from . import ring as oring
from .bf16 import bf16

ROLES = ("user", "assistant")


class StreamOracle:
    def __init__(self, weights, cfg, max_slots, roles=ROLES, gdn="recurrent", state_dtype="float64"):
        """weights: name -> float32 numpy array of the bf16 weights (reference parameter names). gdn: "recurrent"
        (``gdn_slot_step``, token by token) or "chunk" (``gdn_slot_step_chunked`` for ticks of more than one
        step: the same float64 recurrence in the chunk form, for full-geometry ticks of long rows).
        state_dtype "float16": the recurrent state is stored in fp16 between ticks, as the reference's
        StreamingGuard keeps it (runtime.py:157, ``state_dtype='float16'``): each tick runs from the stored
        fp16 values in float64 and rounds the pool to fp16 when it stores it back."""
        if gdn not in ("recurrent", "chunk"):
            raise ValueError("gdn must be 'recurrent' or 'chunk'")
        if state_dtype not in ("float64", "float16"):
            raise ValueError("state_dtype must be 'float64' or 'float16'")
        self.gdn = gdn
        self.state_dtype = state_dtype
        self.w = weights
        self._fused = {}
        self.cfg = cfg
        self.roles = roles
        self.max_slots = max_slots
        S = max_slots + 1
        types = list(cfg.layer_types)
        self.kind = [(t, sum(1 for u in types[:i] if u == t)) for i, t in enumerate(types)]
        n_gdn, n_att = types.count("linear_attention"), types.count("full_attention")
        W = cfg.window_tokens
        self.rec = np.zeros((n_gdn, S, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                             cfg.linear_value_head_dim))
        self.conv = np.zeros((n_gdn, S, cfg.linear_conv_kernel_dim - 1, cfg.conv_dim), dtype=np.float32)
        self.ring_k = np.zeros((n_att, S, cfg.num_key_value_heads, W + 1, cfg.head_dim), dtype=np.float32)
        self.ring_v = np.zeros_like(self.ring_k)
        self.ring_pos = np.full((S, W + 1), -1, dtype=np.int64)
        self.length = np.zeros(max_slots, dtype=np.int64)
        rot = cfg.rotary_dim
        self.inv_freq = oglue.inv_freq(rot, cfg.rope_theta)

    def reset(self, slots=None):
        """Zero every slot (the reference's reset, bucketed_engine.py:51-55) or only ``slots``."""
        if slots is None:
            self.__init__(self.w, self.cfg, self.max_slots, self.roles, self.gdn, self.state_dtype)
            return
        idx = np.asarray(list(slots), dtype=np.int64)
        self.rec[:, idx] = 0
        self.conv[:, idx] = 0
        self.ring_k[:, idx] = 0
        self.ring_v[:, idx] = 0
        self.ring_pos[idx] = -1
        self.length[idx] = 0

    def _cat(self, prefix, names):
        key = (prefix,) + tuple(names)
        if key not in self._fused:
            self._fused[key] = np.concatenate([self.w[prefix + n + ".weight"] for n in names])
        return self._fused[key]

    def tick(self, requests, gemm=None):
        """requests: [(slot, ids)] with unique slots, each <= 64 ids. Returns probs [R, n, lb, 3] float64
        and the final normed hidden [n, lb, hidden]."""
        cfg, w = self.cfg, self.w
        if gemm is None:
            gemm = lambda x, wt, bias, lens: oglue.linear_bf16(x, wt, bias)
        n = len(requests)
        lb = max(len(ids) for _, ids in requests)
        slots = np.array([s for s, _ in requests], dtype=np.int64)
        out = np.empty(n * lb + 3 * n, dtype=np.int64)
        lens = opack.pack_inputs([list(ids) for _, ids in requests], slots, n, lb, self.length, self.max_slots, out)
        ids = out[:n * lb].reshape(n, lb)
        starts = out[n * lb + 2 * n:]
        pos = starts[:, None] + np.arange(lb)[None]
        W, eps = cfg.window_tokens, cfg.rms_norm_eps
        hq, hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        G = hq // hkv
        H, HV, K, V = (cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim,
                       cfg.linear_value_head_dim)
        hidden = w["backbone.embed_tokens.weight"][ids].astype(np.float32)
        normed = oglue.rmsnorm(hidden, 1.0 + w["backbone.layers.0.input_layernorm.weight"], eps)
        cos, sin = oglue.rope_cos_sin(pos, self.inv_freq)
        nl = len(self.kind)
        for i, (kind, idx) in enumerate(self.kind):
            p = f"backbone.layers.{i}."
            if kind == "linear_attention":
                a = p + "linear_attn."
                C, VD = cfg.conv_dim, cfg.value_dim
                proj = gemm(normed, self._cat(a, ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")), None, lens)
                qkv, z = proj[..., :C], proj[..., C:C + VD]
                bb, aa = proj[..., C + VD:C + VD + HV], proj[..., C + VD + HV:C + VD + 2 * HV]
                conv_out, self.conv[idx] = oglue.conv_silu_update(qkv, self.conv[idx], w[a + "conv1d.weight"],
                                                                  slots, lens)
                step = ogdn.gdn_slot_step_chunked if self.gdn == "chunk" and lb > 1 else ogdn.gdn_slot_step
                o, _, self.rec[idx] = step(conv_out, cfg.key_dim, H, K, HV, V, aa, bb, w[a + "A_log"],
                                           w[a + "dt_bias"], self.rec[idx], slots, lens)
                if self.state_dtype == "float16":
                    self.rec[idx] = self.rec[idx].astype(np.float16).astype(np.float64)
                gated = oglue.gated_rmsnorm(bf16(o), z.reshape(n, lb, HV, V), w[a + "norm.weight"], eps)
                mix = gemm(gated.reshape(n, lb, HV * V), w[a + "out_proj.weight"], None, lens)
            else:
                a = p + "self_attn."
                proj = gemm(normed, self._cat(a, ("q_proj", "k_proj", "v_proj")), None, lens)
                qp = proj[..., :hq * 2 * D]
                kp = proj[..., hq * 2 * D:hq * 2 * D + hkv * D]
                vp = proj[..., hq * 2 * D + hkv * D:]
                q = qp.reshape(n, lb, hq, 2 * D)[..., :D]
                qr = oglue.norm_rope(q, 1.0 + w[a + "q_norm.weight"], eps, cos, sin)
                kr = oglue.norm_rope(kp.reshape(n, lb, hkv, D), 1.0 + w[a + "k_norm.weight"], eps, cos, sin)
                qg = qr.reshape(n, lb, hkv, G, D).transpose(0, 2, 3, 1, 4).reshape(n, hkv, G * lb, D)
                new_k = kr.transpose(0, 2, 1, 3)
                att, _, _, _ = oring.ring_attention_v8(qg, self.ring_k[idx], self.ring_v[idx], new_k, vp, qp,
                                                       self.ring_pos, slots, starts, lens, D ** -0.5, W, False)
                new_v = vp.reshape(n, lb, hkv, D).transpose(0, 2, 1, 3)
                oring.ring_scatter(self.ring_k[idx], self.ring_v[idx], new_k, new_v, slots, starts, lens, W)
                mix = gemm(att, w[a + "o_proj.weight"], None, lens)
            hidden, normed = oglue.add_rmsnorm(hidden, mix, 1.0 + w[p + "post_attention_layernorm.weight"], eps)
            I = cfg.intermediate_size
            gu = gemm(normed, self._cat(p + "mlp.", ("gate_proj", "up_proj")), None, lens)
            mix = gemm(oglue.silu_mul(gu[..., :I], gu[..., I:]), w[p + "mlp.down_proj.weight"], None, lens)
            nxt = (f"backbone.layers.{i + 1}.input_layernorm.weight" if i + 1 < nl else "backbone.norm.weight")
            hidden, normed = oglue.add_rmsnorm(hidden, mix, 1.0 + w[nxt], eps)
        E = cfg.head_hidden
        y = gemm(normed, np.concatenate([w[f"heads.{r}.projection.0.weight"] for r in self.roles]),
                 np.concatenate([w[f"heads.{r}.projection.0.bias"] for r in self.roles]), lens)
        probs = np.stack([oglue.risk_probs_from_projection(
            y[..., i * E:(i + 1) * E].reshape(n * lb, E), w[f"heads.{r}.projection.1.weight"],
            w[f"heads.{r}.projection.1.bias"], w[f"heads.{r}.risk.weight"], w[f"heads.{r}.risk.bias"],
            cfg.layer_norm_eps).reshape(n, lb, 3) for i, r in enumerate(self.roles)])
        opack.ring_pos_update(self.ring_pos, slots, starts, lens, lb, W)
        self.length[slots] += lens
        return probs, normed

    def step(self, requests, gemm=None):
        """Like the engine's step (slot_engine_v7.py:147-167): splits each request into ticks of at most
        min(64, window) tokens. Returns {role: [[L_i, 3]]}."""
        cut = min(64, self.cfg.window_tokens)
        results = {r: [[] for _ in requests] for r in self.roles}
        pending = [(i, s, list(ids)) for i, (s, ids) in enumerate(requests)]
        while pending:
            probs, _ = self.tick([(s, ids[:cut]) for _, s, ids in pending], gemm=gemm)
            for ri, role in enumerate(self.roles):
                for row, (i, _, ids) in enumerate(pending):
                    results[role][i].append(probs[ri, row, :min(cut, len(ids))])
            pending = [(i, s, ids[cut:]) for i, s, ids in pending if len(ids) > cut]
        return {r: [np.concatenate(c) for c in rows] for r, rows in results.items()}
