"""Complete-message scoring on the MI355X kernels: one forward over a whole token sequence.

Replaces the reference's whole forward behind ``score_messages`` (src/hs_guard/runtime.py:136-145): the
Qwen3.5 backbone with FLA's ``chunk_gated_delta_rule`` in the GDN layers (runtime.py:76-89) and the tiled
512-token window attention (src/hs_guard/window_attention.py:34-53, 56-72) in the attention layers, then both
roles' risk heads (runtime.py:71-74).

* GDN layers: fused projection GEMM -> causal conv + SiLU -> ``hsg_gdn_chunk_prefill`` from a zero state (the
  WY/UT chunk form on MFMA) -> ``hsg_gated_rmsnorm`` -> out_proj.
* Attention layers: fused q|k|v GEMM -> q/k RMSNorm + RoPE at positions 0 .. T-1 -> window attention ->
  sigmoid(gate) -> o_proj.
* Risk heads in float32, as the reference's readout on ``hidden.float()`` outside autocast (runtime.py:70-73,
  141): an fp32 GEMM with the heads' fp32 weights, then ``hsg_risk_head_f32`` (LayerNorm, SiLU, logits and
  softmax, nothing rounded to bf16).
* The sequence is cut into 64-token segments for the conv and the attention. Segment s is given, as its conv
  history, the 3 tokens before it and, as its "ring", the keys and values of the W positions before it
  (positions [64 s - W, 64 s) at columns p mod W, ring_pos = p, or -1 before the sequence start), gathered on
  the device. ``hsg_conv_silu_update`` and ``hsg_ring_attention`` (no ring write) then compute exactly the
  whole sequence's causal conv and window mask (0 <= p <= q, p > q - W). No per-slot state of the streaming
  engine is read or written.

GEMMs run at the whole sequence's M, so results differ from the streaming path's in the last bits of some
products; the two agree within the tolerances the tests state (the reference's own stream-vs-whole check
allows 0.05, examples/demo/server.py:483).
"""
from __future__ import annotations

import math

import torch

from .._lib import check, lib
from .slot_engine import ROLES, PreparedWeights, gdn_proj_width

SEG = 64                  # tokens per conv / attention segment (the tiled ring kernel's row limit)
MAX_ATT_SEGMENTS = 128    # segments per attention launch: bounds the gathered rings to ~270 MB at W = 512


def fp32_heads(model, roles=ROLES):
    """Both roles' risk heads for the complete-message readout, float32 and unrounded (runtime.py:70-73): the first
    Linear fused over the roles (w1 [roles*E, hidden], b1), the LayerNorm (ln_w, ln_b [roles, E]) and the risk
    Linear (w2 [roles, 3, E], b2 [roles, 3])."""
    m, f32 = model, torch.float32
    return {"w1": torch.cat([m[f"heads.{r}.projection.0.weight"] for r in roles]).to(f32).contiguous(),
            "b1": torch.cat([m[f"heads.{r}.projection.0.bias"] for r in roles]).to(f32).contiguous(),
            "ln_w": torch.stack([m[f"heads.{r}.projection.1.weight"] for r in roles]).to(f32).contiguous(),
            "ln_b": torch.stack([m[f"heads.{r}.projection.1.bias"] for r in roles]).to(f32).contiguous(),
            "w2": torch.stack([m[f"heads.{r}.risk.weight"] for r in roles]).to(f32).contiguous(),
            "b2": torch.stack([m[f"heads.{r}.risk.bias"] for r in roles]).to(f32).contiguous()}


class WholeSequenceScorer(PreparedWeights):
    """Scores whole token sequences with the kernels of libhsg.so. ``shared``: a SlotStreamEngine (or another
    scorer) whose prepared weights are reused instead of building a second copy."""

    def __init__(self, model, roles=ROLES, shared=None):
        lib()  # fail loudly if the HIP library is missing
        self.model, self.cfg = model, model.config
        self.roles = tuple(roles)
        self.device = model.device
        types = list(self.cfg.layer_types)
        self.kind = [(t, sum(1 for u in types[:i] if u == t)) for i, t in enumerate(types)]
        self.window = self.cfg.window_tokens
        if shared is not None and tuple(shared.roles) == self.roles:
            for name in ("layers", "final_w1", "emb", "inv_freq", "head_w1", "head_b1", "head_ln_w", "head_ln_b",
                         "head_w2", "head_b2"):
                setattr(self, name, getattr(shared, name))
        else:
            self._prepare_weights()
        self.head32 = fp32_heads(model, self.roles)

    @torch.inference_mode()
    def forward(self, ids):
        """Class probabilities of every position of the token sequence ``ids``: float32 [roles, T, 3] on the
        device (the softmax of each role's risk head)."""
        L = lib()
        cfg, dev = self.cfg, self.device
        T = len(ids)
        if T == 0:
            raise ValueError("The sequence is empty")
        st = torch.cuda.current_stream(dev).cuda_stream
        bf16 = torch.bfloat16
        H, eps, W = cfg.hidden_size, cfg.rms_norm_eps, self.window
        hq, hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        G = hq // hkv
        nh, hv, kd, vd = cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim, \
            cfg.linear_value_head_dim
        C = cfg.conv_dim
        gdn_in = gdn_proj_width(cfg)       # row stride of the GDN projection (zero-padded weight rows)
        att_in = hq * 2 * D + 2 * hkv * D
        i64 = dict(dtype=torch.long, device=dev)

        ids_d = torch.tensor(list(ids), **i64)
        pos = torch.arange(T, **i64)
        nseg = math.ceil(T / SEG)
        seg_off = torch.arange(nseg, **i64) * SEG
        seg_len = torch.clamp(T - seg_off, max=SEG)
        seg_slot = torch.arange(nseg, **i64)
        # conv history of segment s: tokens 64 s - 3 .. 64 s - 1 (zero before the sequence start)
        K1 = cfg.linear_conv_kernel_dim - 1
        hist = seg_off[:, None] - K1 + torch.arange(K1, **i64)[None, :]
        hist_ok = (hist >= 0)[..., None]
        hist = hist.clamp(min=0)
        # window ring of segment s: column c holds position 64 s - W + ((c - 64 s) mod W)
        cols = torch.arange(W, **i64)[None, :]
        ring_p = seg_off[:, None] - W + torch.remainder(cols - seg_off[:, None], W)
        ring_pos_all = torch.full((nseg, W + 1), -1, **i64)
        ring_pos_all[:, :W] = torch.where(ring_p >= 0, ring_p, torch.full_like(ring_p, -1))
        ring_src = ring_p.clamp(min=0)

        hidden = torch.empty(T, H, dtype=bf16, device=dev)
        normed = torch.empty_like(hidden)
        mix = torch.empty_like(hidden)
        check(L.hsg_embed_rmsnorm(ids_d.data_ptr(), self.emb.data_ptr(), cfg.vocab_size,
                                  self.layers[0]["in_w1"].data_ptr(), eps, hidden.data_ptr(), normed.data_ptr(), T, H,
                                  st), "hsg_embed_rmsnorm")
        ws = state = None
        row0 = torch.zeros(1, **i64)
        row_len = torch.full((1,), T, **i64)
        for i, ((kind, _), Lw) in enumerate(zip(self.kind, self.layers)):
            if kind == "linear_attention":
                proj = torch.mm(normed, Lw["w_in"].t())
                pools = torch.where(hist_ok, proj[:, :C][hist], torch.zeros((), dtype=bf16, device=dev)).contiguous()
                conv = torch.empty(T, C, dtype=bf16, device=dev)
                check(L.hsg_conv_silu_update(proj.data_ptr(), gdn_in, pools.data_ptr(), nseg,
                                             Lw["conv_w"].data_ptr(), cfg.linear_conv_kernel_dim, seg_slot.data_ptr(),
                                             seg_len.data_ptr(), seg_off.data_ptr(), nseg, 0, C, conv.data_ptr(), C,
                                             st), "hsg_conv_silu_update")
                if ws is None:
                    ws = torch.empty(max(int(L.hsg_gdn_chunk_workspace_bytes(1, T, hv)), 256), dtype=torch.uint8,
                                     device=dev)
                    state = torch.empty(1, hv, kd, vd, dtype=torch.float32, device=dev)
                state.zero_()
                o = torch.empty(T, hv, vd, dtype=bf16, device=dev)
                base = proj.data_ptr()
                check(L.hsg_gdn_chunk_prefill(
                    conv.data_ptr(), C, 0, cfg.key_dim, 2 * cfg.key_dim,
                    base + 2 * (C + cfg.value_dim + hv), base + 2 * (C + cfg.value_dim), gdn_in,
                    Lw["A_log"].data_ptr(), Lw["dt_bias"].data_ptr(), state.data_ptr(), 0, 1, row0.data_ptr(),
                    row_len.data_ptr(), row0.data_ptr(), 1, T, nh, hv, kd, vd, kd ** -0.5, o.data_ptr(), None, 0,
                    ws.data_ptr(), ws.numel(), st), "hsg_gdn_chunk_prefill")
                gated = torch.empty(T, cfg.value_dim, dtype=bf16, device=dev)
                check(L.hsg_gated_rmsnorm(o.data_ptr(), cfg.value_dim, base + 2 * C, gdn_in, Lw["norm_w"].data_ptr(),
                                          eps, gated.data_ptr(), cfg.value_dim, T, hv, vd, st), "hsg_gated_rmsnorm")
                torch.mm(gated, Lw["w_out"].t(), out=mix)
            else:
                proj = torch.mm(normed, Lw["w_in"].t())
                q = torch.empty(T, hq * D, dtype=bf16, device=dev)
                k = torch.empty(T, hkv * D, dtype=bf16, device=dev)
                base = proj.data_ptr()
                check(L.hsg_norm_rope(base, att_in, 2 * D, hq, Lw["q_w1"].data_ptr(), eps, q.data_ptr(), hq * D, D,
                                      base + 2 * hq * 2 * D, att_in, D, hkv, Lw["k_w1"].data_ptr(), eps,
                                      k.data_ptr(), hkv * D, D, pos.data_ptr(), self.inv_freq.data_ptr(),
                                      cfg.rotary_dim, T, D, st), "hsg_norm_rope")
                v = proj[:, hq * 2 * D + hkv * D:].view(T, hkv, D)
                kh = k.view(T, hkv, D)
                att = torch.empty(T, hq * D, dtype=bf16, device=dev)
                for s0 in range(0, nseg, MAX_ATT_SEGMENTS):
                    s1 = min(nseg, s0 + MAX_ATT_SEGMENTS)
                    n = s1 - s0
                    ring_k = torch.zeros(n, hkv, W + 1, D, dtype=bf16, device=dev)
                    ring_v = torch.zeros_like(ring_k)
                    ring_k[:, :, :W] = kh[ring_src[s0:s1]].permute(0, 2, 1, 3)
                    ring_v[:, :, :W] = v[ring_src[s0:s1]].permute(0, 2, 1, 3)
                    rpos = ring_pos_all[s0:s1].contiguous()
                    offs = seg_off[s0:s1].contiguous()
                    lens = seg_len[s0:s1].contiguous()
                    slots = torch.arange(n, **i64)
                    check(L.hsg_ring_attention(
                        q.data_ptr(), 0, hq * D, G * D, D, ring_k.data_ptr(), ring_v.data_ptr(), n, W,
                        k.data_ptr(), 0, hkv * D, D, base + 2 * (hq * 2 * D + hkv * D), 0, att_in, D,
                        base, 0, att_in, G * 2 * D, 2 * D, D, rpos.data_ptr(), slots.data_ptr(), offs.data_ptr(),
                        lens.data_ptr(), offs.data_ptr(), n, SEG, hkv, G, D, D ** -0.5, 0, 0,
                        att.data_ptr(), 0, hq * D, G * D, D, st), "hsg_ring_attention")
                torch.mm(att, Lw["w_out"].t(), out=mix)
            check(L.hsg_add_rmsnorm(hidden.data_ptr(), mix.data_ptr(), Lw["post_w1"].data_ptr(), eps,
                                    normed.data_ptr(), T, H, st), "hsg_add_rmsnorm")
            I = cfg.intermediate_size
            gu = torch.mm(normed, Lw["w_gu"].t())
            act = torch.empty(T, I, dtype=bf16, device=dev)
            check(L.hsg_silu_mul(gu.data_ptr(), 2 * I, I, act.data_ptr(), T, st), "hsg_silu_mul")
            torch.mm(act, Lw["w_down"].t(), out=mix)
            nxt = self.layers[i + 1]["in_w1"] if i + 1 < len(self.layers) else self.final_w1
            check(L.hsg_add_rmsnorm(hidden.data_ptr(), mix.data_ptr(), nxt.data_ptr(), eps, normed.data_ptr(), T, H,
                                    st), "hsg_add_rmsnorm")
        R, E = len(self.roles), cfg.head_hidden
        h32 = self.head32
        y = torch.addmm(h32["b1"], normed.float(), h32["w1"].t())
        probs = torch.empty(R, T, 3, dtype=torch.float32, device=dev)
        check(L.hsg_risk_head_f32(y.data_ptr(), R * E, h32["ln_w"].data_ptr(), h32["ln_b"].data_ptr(),
                                  h32["w2"].data_ptr(), h32["b2"].data_ptr(), cfg.layer_norm_eps, R, E,
                                  probs.data_ptr(), T, st), "hsg_risk_head_f32")
        return probs
