"""Ring-window GQA attention oracle (test infrastructure only; float64).

``ring_attention_reference`` restates the reference's own torch contract
``src/hs_guard/engine/ring_attention_kernel.py:7-26``: each query row ``r = g*Lb + l`` of kv-head h sits at
``qpos = start + l`` and is valid when ``l < len``; it attends to the slot's W ring columns (key position
``ring_pos[slot, c]``) and to this tick's Lb new keys (position ``start + j`` when ``j < len``, else -1),
keeping exactly the keys with ``kpos >= 0 and kpos <= qpos and kpos > qpos - W``. A row with no key gives 0.

``ring_attention_v8`` adds the v8 epilogue of ``fused_kernels.py:341-355``: output rounded to bf16, times
``bf16(sigmoid(gate))`` (gate = second half of each q head's ``q_proj`` slice) rounded to bf16, written as
``[N, Lb, Hq*D]`` with q head ``h*G + g``; when ``write_ring`` (Lb == 1) and ``len > 0`` the new key/value go
to ring column ``start % W``. ``ring_scatter`` is the Lb > 1 write of ``slot_engine_v8.py:86-88``
(column ``pos % W`` for valid steps, scratch column W otherwise).

``attend_blockwise`` restates the numerics of the reference's Triton kernels (fused_kernels.py:309-341,
ring_attention_kernel.py:56-87): keys in blocks of 32 (the W ring columns in order, then the tick's new
keys), a running max per query row, ``acc = acc * alpha + bf16(p) @ v`` and ``l = l * alpha + sum(p)`` with
p in full precision in the sum; ``ring_attention_v8`` uses it. Without bf16 rounding (``oracle.bf16.exact``)
it equals ``ring_attention_reference``.

Pinning (``tests/test_oracle_ring.py``): torch ``scaled_dot_product_attention`` with an explicit boolean
mask; fill 0 with only the new key gives ``v_new * sigmoid(gate)``; all-equal keys give the mean of the
valid values; a brute-force enumeration of the window predicate; blockwise == exact without rounding and
within the bf16 bound of p with it.
"""
import numpy as np

from .bf16 import bf16, sigmoid


def key_positions(ring_pos, slots, starts, lens, lb, window):
    slots = np.asarray(slots, dtype=np.int64)
    starts = np.asarray(starts, dtype=np.int64)
    lens = np.asarray(lens, dtype=np.int64)
    j = np.arange(lb)[None, :]
    new_pos = np.where(j < lens[:, None], starts[:, None] + j, -1)
    return np.concatenate([np.asarray(ring_pos)[slots, :window], new_pos], 1)     # [N, W + Lb]


def allowed_mask(ring_pos, slots, starts, lens, lb, groups, window):
    """[N, G*Lb, W + Lb] boolean predicate of ring_attention_kernel.py:17-23."""
    starts = np.asarray(starts, dtype=np.int64)
    lens = np.asarray(lens, dtype=np.int64)
    rows = np.arange(groups * lb)
    l_idx = rows % lb
    qpos = starts[:, None] + l_idx[None]
    q_valid = l_idx[None] < lens[:, None]
    kpos = key_positions(ring_pos, slots, starts, lens, lb, window)
    ok = (kpos[:, None] >= 0) & (kpos[:, None] <= qpos[..., None]) & (kpos[:, None] > qpos[..., None] - window)
    return ok & q_valid[..., None]


def ring_attention_reference(q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, scale, window):
    """q [N, Hkv, G*Lb, D]; ring_k/v [S, Hkv, W+1, D]; new_k/v [N, Hkv, Lb, D] -> [N, Hkv, G*Lb, D] float64."""
    q = np.asarray(q, dtype=np.float64)
    N, Hkv, M, D = q.shape
    lb = new_k.shape[2]
    ok = allowed_mask(ring_pos, slots, starts, lens, lb, M // lb, window)
    slots = np.asarray(slots, dtype=np.int64)
    keys = np.concatenate([np.asarray(ring_k, dtype=np.float64)[slots, :, :window],
                           np.asarray(new_k, dtype=np.float64)], 2)
    values = np.concatenate([np.asarray(ring_v, dtype=np.float64)[slots, :, :window],
                             np.asarray(new_v, dtype=np.float64)], 2)
    scores = np.einsum('nhmd,nhjd->nhmj', q, keys) * scale
    scores = np.where(ok[:, None], scores, -np.inf)
    mx = scores.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    p = np.where(ok[:, None], np.exp(scores - mx), 0.0)
    den = p.sum(-1, keepdims=True)
    p = np.where(den > 0, p / np.where(den > 0, den, 1.0), 0.0)
    return np.einsum('nhmj,nhjd->nhmd', p, values)


def _blocks(window, lb, block):
    """(start, end) of the key blocks: the W ring columns in blocks of ``block``, then the tick's new keys."""
    edges = list(range(0, window, block)) + [window + j for j in range(0, lb, block)]
    ends = edges[1:] + [window + lb]
    return [(b0, min(b1, window) if b0 < window else b1) for b0, b1 in zip(edges, ends)]


def attend_blockwise(q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, scale, window, block=32):
    """Same contract as ring_attention_reference, with the Triton kernels' blockwise online softmax and bf16
    probabilities in the P.V product. Returns [N, Hkv, G*Lb, D] float64.

    Evaluated in closed form: with m_b the running max after block b (the prefix maximum of the block maxima),
    the online recurrence ``acc = acc * exp(m_{b-1} - m_b) + bf16(exp(s - m_b)) @ v`` multiplies out to
    ``acc = sum_b exp(m_b - m_last) * bf16(exp(s_b - m_b)) @ v_b`` (and the same for l with unrounded p), so
    every bf16 rounding sits where the reference's loop puts it; ``attend_blockwise_online`` is the loop itself
    and ``tests/test_oracle_ring.py`` holds the two together."""
    q = np.asarray(q, dtype=np.float64)
    N, Hkv, M, D = q.shape
    lb = new_k.shape[2]
    ok = allowed_mask(ring_pos, slots, starts, lens, lb, M // lb, window)
    slots = np.asarray(slots, dtype=np.int64)
    keys = np.concatenate([np.asarray(ring_k, dtype=np.float64)[slots, :, :window],
                           np.asarray(new_k, dtype=np.float64)], 2)
    values = np.concatenate([np.asarray(ring_v, dtype=np.float64)[slots, :, :window],
                             np.asarray(new_v, dtype=np.float64)], 2)
    scores = np.where(ok[:, None], np.matmul(q, keys.transpose(0, 1, 3, 2)) * scale, -np.inf)
    blocks = _blocks(window, lb, block)
    bmax = np.stack([scores[..., b0:b1].max(-1) for b0, b1 in blocks], -1)       # [N, Hkv, M, nblocks]
    run = np.maximum.accumulate(bmax, -1)                                       # m_b
    last = run[..., -1:]
    width = np.array([b1 - b0 for b0, b1 in blocks])
    m_key = np.repeat(run, width, axis=-1)                                      # m_b of each key's block
    m_safe = np.where(np.isfinite(m_key), m_key, 0.0)
    p = np.where(np.isfinite(scores), np.exp(scores - m_safe), 0.0)
    wgt = np.where(np.isfinite(run), np.exp(run - np.where(np.isfinite(last), last, 0.0)), 0.0)
    w_key = np.repeat(wgt, width, axis=-1)
    acc = np.matmul(np.asarray(bf16(p), np.float64) * w_key, values)
    l = (p * w_key).sum(-1)
    return np.where(l[..., None] > 0, acc / np.where(l > 0, l, 1.0)[..., None], 0.0)


def attend_blockwise_online(q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, scale, window,
                            block=32):
    """attend_blockwise as the reference kernels' loop (fused_kernels.py:309-341): one block at a time, the running
    max updated and the accumulator and row sum rescaled after each block."""
    q = np.asarray(q, dtype=np.float64)
    N, Hkv, M, D = q.shape
    lb = new_k.shape[2]
    ok = allowed_mask(ring_pos, slots, starts, lens, lb, M // lb, window)
    slots = np.asarray(slots, dtype=np.int64)
    keys = np.concatenate([np.asarray(ring_k, dtype=np.float64)[slots, :, :window],
                           np.asarray(new_k, dtype=np.float64)], 2)
    values = np.concatenate([np.asarray(ring_v, dtype=np.float64)[slots, :, :window],
                             np.asarray(new_v, dtype=np.float64)], 2)
    scores = np.where(ok[:, None], np.matmul(q, keys.transpose(0, 1, 3, 2)) * scale, -np.inf)
    m = np.full((N, Hkv, M), -np.inf)
    l = np.zeros((N, Hkv, M))
    acc = np.zeros((N, Hkv, M, D))
    for b0, b1 in _blocks(window, lb, block):
        sb = scores[..., b0:b1]
        m_new = np.maximum(m, sb.max(-1))
        m_safe = np.where(np.isfinite(m_new), m_new, 0.0)
        pb = np.where(np.isfinite(sb), np.exp(sb - m_safe[..., None]), 0.0)
        alpha = np.where(np.isfinite(m), np.exp(m - m_safe), 0.0)
        acc = acc * alpha[..., None] + np.matmul(np.asarray(bf16(pb), np.float64), values[:, :, b0:b1])
        l = l * alpha + pb.sum(-1)
        m = m_new
    return np.where(l[..., None] > 0, acc / np.where(l > 0, l, 1.0)[..., None], 0.0)


def ring_attention_v8(q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, lens, scale, window,
                      write_ring):
    """Returns (out [N, Lb, Hq*D] float32 of bf16 values, attn [N, Hkv, G*Lb, D] float64, ring_k', ring_v')."""
    N, Hkv, M, D = q.shape
    lb = new_k.shape[2]
    G = M // lb
    Hq = Hkv * G
    value = np.asarray(value, dtype=np.float64).reshape(N, lb, Hkv, D)
    new_v = value.transpose(0, 2, 1, 3)
    attn = attend_blockwise(q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, scale, window)
    o = attn.reshape(N, Hkv, G, lb, D).transpose(0, 3, 1, 2, 4).reshape(N, lb, Hq, D)
    gt = np.asarray(gate, dtype=np.float64).reshape(N, lb, Hq, 2 * D)[..., D:]
    sig = bf16(sigmoid(gt))
    out = bf16(bf16(o).astype(np.float64) * sig).reshape(N, lb, Hq * D)
    rk = np.array(ring_k, copy=True)
    rv = np.array(ring_v, copy=True)
    if write_ring:
        assert lb == 1
        for n, s in enumerate(np.asarray(slots, dtype=np.int64)):
            if lens[n] > 0:
                col = int(starts[n]) % window
                rk[s, :, col] = np.asarray(new_k)[n, :, 0]
                rv[s, :, col] = new_v[n, :, 0]
    return out, attn, rk, rv


def ring_scatter(ring_k, ring_v, new_k, new_v, slots, starts, lens, window):
    """In-place scatter of slot_engine_v8.py:86-88 (new_k/new_v [N, Hkv, Lb, D])."""
    lb = new_k.shape[2]
    for n, s in enumerate(np.asarray(slots, dtype=np.int64)):
        for t in range(lb):
            col = (int(starts[n]) + t) % window if t < lens[n] else window
            ring_k[s, :, col] = new_k[n, :, t]
            ring_v[s, :, col] = new_v[n, :, t]
    return ring_k, ring_v
