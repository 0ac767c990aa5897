"""Helpers shared by the engine-vs-oracle GPU tests (imported by them; holds no tests itself).

``matched_gemm(engine)`` gives the oracle (``StreamOracle.tick(..., gemm=...)``) the engine's own bf16 product:
the engine's ``mm`` (hsg_gemm_bf16 with the same committed hipBLASLt solution for (tb, N, K), or the skinny product
for tb <= 8), or torch.addmm for the heads' biased product, into a [tb, N] buffer, tb the engine's token bucket, with the rows packed in the
engine's order (longest first, ties in request order). Each output row is then bitwise the engine's for the same
input row, so an engine-vs-oracle comparison checks every other kernel (conv, recurrence, norms, RoPE, ring
attention, heads, bookkeeping) against the CPU restatement.
"""
import numpy as np
import torch


def bf16_ulp(x):
    """The spacing of bf16 values at |x| (8 significant bits)."""
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def close_bf16(got, ref, what, frac=5e-3, atol=1e-30, ulps=None):
    """bf16 outputs against the oracle. Default bar: 2^-8 relative. With ``ulps``: that many bf16 ulps of the
    reference value (one ulp is 2^-8 to 2^-7 relative, so a single rounding flip at the bottom of a binade passes
    only this form). At most ``frac`` of the values may differ at all."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = np.abs(got - ref)
    tol = 2.0 ** -8 * np.abs(ref) if ulps is None else ulps * bf16_ulp(ref)
    bad = diff > tol + atol
    assert not bad.any(), f"{what}: {int(bad.sum())} values beyond the bar (max {diff.max():.3e})"
    assert np.mean(diff > 0) <= frac, f"{what}: {np.mean(diff > 0):.3%} of values differ"


def matched_gemm(eng):
    from hs_guard.engine.slot_engine import bucket, gdn_proj_width
    cache = {}
    cfg = eng.cfg
    gdn_n = cfg.conv_dim + cfg.value_dim + 2 * cfg.linear_num_value_heads

    def gemm(x, w, bias, lens):
        n, lb, K = x.shape
        lens = np.asarray(lens)
        total = int(lens.sum())
        tb = bucket(total, eng.token_buckets)
        order = np.argsort(-lens, kind="stable")
        xp = np.zeros((tb, K), dtype=np.float32)
        xp[:total] = np.concatenate([x[r, :lens[r]] for r in order])
        key = (id(w), w.shape)
        if key not in cache:
            wp = w
            if w.shape == (gdn_n, cfg.hidden_size):   # the engine's GDN projection carries zero padding rows
                wp = np.concatenate([w, np.zeros((gdn_proj_width(cfg) - gdn_n, w.shape[1]), w.dtype)])
            cache[key] = (w, torch.from_numpy(np.ascontiguousarray(wp)).to(torch.bfloat16).cuda().contiguous())
        W = cache[key][1]
        xd = torch.from_numpy(xp).to(torch.bfloat16).cuda()
        out = torch.empty(tb, W.shape[0], dtype=torch.bfloat16, device="cuda")
        if bias is None:
            eng.mm(xd, W, out)       # the engine's own product: same hipBLASLt solution for (tb, N, K)
        else:
            torch.addmm(torch.from_numpy(bias).to(torch.bfloat16).cuda(), xd, W.t(), out=out)
        y = out.float().cpu().numpy()[:, :w.shape[0]]
        res = np.zeros((n, lb, w.shape[0]), dtype=np.float32)
        at = 0
        for r in order:
            res[r, :lens[r]] = y[at:at + lens[r]]
            at += lens[r]
        return res
    return gemm


def max_diff(got, ref):
    """Largest per-token difference of the cut score 1 - p(safe) over both roles (the north-star quantity)."""
    return max(np.abs(g.numpy()[:, 0] - e[:, 0]).max() for role in ("user", "assistant")
               for g, e in zip(got[role], ref[role]))


def whole_matched_gemm(cfg):
    """The complete-message scorer's product for the oracle run over a whole sequence in one tick: torch.mm of
    the [T, K] activations at M = T, as hs_guard.engine.whole runs every projection."""
    from hs_guard.engine.slot_engine import gdn_proj_width
    cache = {}
    gdn_n = cfg.conv_dim + cfg.value_dim + 2 * cfg.linear_num_value_heads

    def gemm(x, w, bias, lens):
        n, T, K = x.shape
        assert n == 1 and int(lens[0]) == T
        key = (id(w), w.shape)
        if key not in cache:
            wp = w
            if w.shape == (gdn_n, cfg.hidden_size):
                wp = np.concatenate([w, np.zeros((gdn_proj_width(cfg) - gdn_n, w.shape[1]), w.dtype)])
            cache[key] = (w, torch.from_numpy(np.ascontiguousarray(wp)).to(torch.bfloat16).cuda().contiguous())
        W = cache[key][1]
        xd = torch.from_numpy(np.ascontiguousarray(x[0])).to(torch.bfloat16).cuda()
        if bias is None:
            y = torch.mm(xd, W.t())
        else:
            y = torch.addmm(torch.from_numpy(bias).to(torch.bfloat16).cuda(), xd, W.t())
        return y.float().cpu().numpy()[None, :, :w.shape[0]]
    return gemm


def oracle_whole(weights, cfg, ids, gemm=None, roles=("user", "assistant")):
    """The oracle over a whole sequence in one tick (tick size does not change its results,
    tests/test_oracle_backbone.py), read out like the complete-message scorer: the float32 risk heads on the
    final hidden state. Returns probabilities [roles, T, 3]."""
    from oracle import glue as oglue
    from oracle.backbone import StreamOracle
    _, normed = StreamOracle(weights, cfg, 1).tick([(0, list(ids))], gemm=gemm)
    w = weights
    return np.stack([oglue.risk_probs_f32(normed[0], w[f"heads.{r}.projection.0.weight"],
                                          w[f"heads.{r}.projection.0.bias"], w[f"heads.{r}.projection.1.weight"],
                                          w[f"heads.{r}.projection.1.bias"], w[f"heads.{r}.risk.weight"],
                                          w[f"heads.{r}.risk.bias"], cfg.layer_norm_eps) for r in roles])
