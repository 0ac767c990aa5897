"""Per-token glue of the streaming step (test infrastructure only).

Rounding points follow the reference's fused kernels (bf16 where they store bf16, fp32/float64 inside):

* ``conv_silu_update``  -- fused_kernels.py:94-136: causal depthwise conv (4 taps) over [pool(3 rows); new
  tokens], fp32 accumulate, round to bf16, SiLU, round to bf16; pool row i <- ext[len + i] when len > 0.
  Pinned against transformers' ``causal_conv1d_update`` (qwen3_5/modeling_qwen3_5.py:200-216).
* ``rms_finish``, ``gated_finish``, ``norm_rope_given`` -- the same formulas with the row variance as an
  input, as the reference's kernels take it; ``rmsnorm``, ``gated_rmsnorm`` and ``norm_rope`` are these with
  the variance computed, so the pins below hold for both forms.
* ``add_rmsnorm``       -- add_square + rms_finish (fused_kernels.py:30-72, slot_engine_v8.py:42-55):
  h = bf16(res + mix); out = bf16(h * rsqrt(mean(h^2) + eps) * (1 + w)). Pinned against transformers'
  ``Qwen3_5RMSNorm`` (modeling_qwen3_5.py:720-737 of that file's class).
* ``gated_rmsnorm``     -- gated_finish (fused_kernels.py:215-233): bf16(bf16(w * bf16(x * r)) * silu(z)),
  r = rsqrt(mean(x^2) + eps). Pinned against ``Qwen3_5RMSNormGated`` (modeling_qwen3_5.py:168-184).
* ``silu_mul``          -- fused_kernels.py:76-90: bf16(bf16(silu(g)) * u).
* ``rope_cos_sin``      -- rotary cos/sin in fp32 then bf16 (qwen3_5 rotary embedding; with three equal
  position ids the interleaved mrope reduces to plain RoPE).
* ``norm_rope``         -- square_rows + norm_rope (fused_kernels.py:237-284): per-head RMSNorm(1+w) to
  bf16, then rotate-half RoPE on the first ``rot`` dims with bf16 products and a bf16 sum. Pinned against
  transformers' ``apply_rotary_pos_emb`` (modeling_qwen3_5.py, rotate_half / apply_rotary_pos_emb).
* ``risk_probs``        -- Classifier.readout risk path (runtime.py:61-74, slot_engine_v7.py:58-61):
  Linear(bf16) -> LayerNorm (fp32) -> SiLU -> Linear (bf16 in/out) -> softmax fp32. Pinned against
  torch.nn.functional on CPU.
* ``risk_probs_f32``    -- the complete-message readout (runtime.py:70-73,141): the same layers on
  ``hidden.float()`` outside autocast, nothing rounded to bf16. Pinned against torch.nn.functional in float64.
"""
import numpy as np

from .bf16 import bf16, silu


def linear_bf16(x, w, bias=None):
    """bf16 GEMM under autocast: fp32 accumulate of bf16 operands, bias added, output rounded to bf16
    (float64 throughout inside ``oracle.bf16.exact()``)."""
    dt = np.float32 if bf16(np.float32(1.5)).dtype == np.float32 else np.float64
    y = np.asarray(x, dtype=dt) @ np.asarray(w, dtype=dt).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=dt)
    return bf16(y)


def conv_silu_update(qkv, pool, weight, slots, lens):
    """qkv [N, L, C]; pool [S, KS-1, C] (a copy is updated); weight [C, 1, KS] or [C, KS].
    Returns (out [N, L, C] bf16 values, pool')."""
    qkv = np.asarray(qkv, dtype=np.float64)
    N, L, C = qkv.shape
    w = np.asarray(weight, dtype=np.float64).reshape(C, -1)
    ks = w.shape[1]
    keep = ks - 1
    pool2 = np.array(pool, copy=True)
    out = np.zeros((N, L, C), dtype=np.float32)
    for n in range(N):
        s = int(slots[n])
        ext = np.concatenate([np.asarray(pool, dtype=np.float64)[s], qkv[n]], 0)   # [keep + L, C]
        # out[t] = sum_i ext[t + i] * w[:, i], taps summed in order, for every t at once
        acc = ext[0:L] * w[:, 0]
        for i in range(1, ks):
            acc = acc + ext[i:i + L] * w[:, i]
        out[n] = bf16(silu(bf16(acc.astype(np.float32))))
        if lens[n] > 0:
            pool2[s] = ext[int(lens[n]):int(lens[n]) + keep]
    return out, pool2


def rms_finish(x, var, w1, eps):
    """rms_finish (fused_kernels.py:56-72): bf16((x * rsqrt(var + eps)) * w1) with the row variance given
    (var [..., 1], the caller's mean of x^2), w1 = 1 + weight (fp32)."""
    x = np.asarray(x, dtype=np.float64)
    return bf16((x / np.sqrt(np.asarray(var, dtype=np.float64) + eps)) * np.asarray(w1, dtype=np.float64))


def rmsnorm(h, w1, eps):
    """bf16((h * rsqrt(mean(h^2) + eps)) * w1) with h already bf16 values, w1 = 1 + weight (fp32)."""
    h = np.asarray(h, dtype=np.float64)
    return rms_finish(h, (h * h).mean(-1, keepdims=True), w1, eps)


def add_rmsnorm(res, mix, w1, eps):
    """Returns (h = bf16(res + mix), rmsnorm(h)). mix None: h = res."""
    h = np.asarray(res, dtype=np.float32) if mix is None else bf16(np.asarray(res, np.float32) + np.asarray(mix, np.float32))
    return h, rmsnorm(h, w1, eps)


def gated_finish(x, var, w, z, eps):
    """gated_finish (fused_kernels.py:215-233) with the row variance given (var [..., 1]):
    bf16(bf16(w * bf16(x * rsqrt(var + eps))) * silu(z))."""
    x = np.asarray(x, dtype=np.float64)
    hb = bf16(x / np.sqrt(np.asarray(var, dtype=np.float64) + eps))
    t = bf16(np.asarray(w, dtype=np.float64) * hb)
    return bf16(t * silu(z))


def gated_rmsnorm(x, z, w, eps):
    """x, z [..., V] (x bf16 values), w [V] -> bf16 values."""
    x = np.asarray(x, dtype=np.float64)
    return gated_finish(x, (x * x).mean(-1, keepdims=True), w, z, eps)


def silu_mul(g, u):
    return bf16(bf16(silu(g)) * np.asarray(u, dtype=np.float64))


def inv_freq(rot_dim, theta):
    """1 / theta^(arange(0, rot, 2) / rot) in fp32, as the rotary embedding computes it."""
    return (1.0 / (np.float32(theta) ** (np.arange(0, rot_dim, 2, dtype=np.float32) / np.float32(rot_dim)))).astype(np.float32)


def rope_cos_sin(pos, inv):
    """pos [...] int -> (cos, sin) [..., rot] bf16 values (emb = cat(freqs, freqs))."""
    freqs = (np.asarray(pos, dtype=np.float32)[..., None] * inv).astype(np.float32)
    emb = np.concatenate([freqs, freqs], -1).astype(np.float64)
    return bf16(np.cos(emb)), bf16(np.sin(emb))


def norm_rope(x, w1, eps, cos, sin):
    """x [..., heads, D] bf16 values; cos, sin [..., rot] (broadcast over heads) -> bf16 values."""
    x = np.asarray(x, dtype=np.float64)
    return norm_rope_given(x, (x * x).mean(-1, keepdims=True), w1, eps, cos, sin)


def norm_rope_given(x, var, w1, eps, cos, sin):
    """norm_rope (fused_kernels.py:252-284) with the per-head variance given (var [..., heads, 1])."""
    x = np.asarray(x, dtype=np.float64)
    y = bf16((x / np.sqrt(np.asarray(var, dtype=np.float64) + eps)) * np.asarray(w1, dtype=np.float64)).astype(np.float64)
    rot = cos.shape[-1]
    half = rot // 2
    c = np.asarray(cos, dtype=np.float64)[..., None, :]
    s = np.asarray(sin, dtype=np.float64)[..., None, :]
    xr = y[..., :rot]
    rh = np.concatenate([-xr[..., half:], xr[..., :half]], -1)
    first = bf16(xr * c).astype(np.float64)
    second = bf16(rh * s).astype(np.float64)
    out = y.copy()
    out[..., :rot] = bf16(first + second)
    return out.astype(np.float32)


def layer_norm(x, w, b, eps=1e-5):
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def risk_probs(hidden, w1, b1, ln_w, ln_b, w2, b2, eps=1e-5):
    """hidden [T, hidden] bf16 values -> softmax(risk logits) [T, 3] float64."""
    return risk_probs_from_projection(linear_bf16(hidden, w1, b1), ln_w, ln_b, w2, b2, eps)


def risk_probs_from_projection(y, ln_w, ln_b, w2, b2, eps=1e-5):
    """The head after its first Linear: y [T, 512] bf16 values -> softmax(risk logits) [T, 3] float64."""
    y = silu(layer_norm(y, ln_w, ln_b, eps))
    logits = linear_bf16(bf16(y), w2, b2).astype(np.float64)
    logits = logits - logits.max(-1, keepdims=True)
    e = np.exp(logits)
    return e / e.sum(-1, keepdims=True)


def risk_probs_f32(hidden, w1, b1, ln_w, ln_b, w2, b2, eps=1e-5):
    """hidden [T, hidden] -> softmax(risk logits) [T, 3] float64, with no bf16 rounding anywhere."""
    y = np.asarray(hidden, np.float64) @ np.asarray(w1, np.float64).T + np.asarray(b1, np.float64)
    y = silu(layer_norm(y, ln_w, ln_b, eps))
    logits = y @ np.asarray(w2, np.float64).T + np.asarray(b2, np.float64)
    logits = logits - logits.max(-1, keepdims=True)
    e = np.exp(logits)
    return e / e.sum(-1, keepdims=True)
