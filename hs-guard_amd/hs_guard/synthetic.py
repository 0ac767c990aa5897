"""Seeded synthetic inputs of the BASELINE configurations (generated on the CPU, then moved).

Every generator draws from one ``torch.Generator`` seeded as given (0 by default) in the documented order,
so the GPU path and the CPU checker consume identical bytes.
"""
from __future__ import annotations

import torch

BF16 = torch.bfloat16


def _bf16_randn(gen, *shape):
    return torch.randn(*shape, generator=gen).to(BF16)


def _l2_bf16(x):
    xf = x.float()
    return (xf / xf.norm(dim=-1, keepdim=True)).to(BF16)


def gdn_step_inputs(slots=16, heads=16, head_dim=128, steps=64, seed=0, state_dtype=torch.float32):
    """Config 1: ``slots`` rows x 1 token for ``steps`` sequential steps, H = HV = heads, K = V = head_dim.

    Draw order: state0 [slots+1, H, K, V] ~ N(0, 0.02) (the extra row is the scratch slot, zeroed), then per
    step q [slots, H, K], k [slots, H, K] (bf16 N(0,1), then L2-normalised per head and rounded to bf16),
    v [slots, H, V] bf16 N(0,1), a [slots, H] bf16 N(0,1), b [slots, H] bf16 N(0,1). A_log = dt_bias = 0,
    so the kernel's g = -softplus(a) and beta = sigmoid(b).
    Returns dict with state0, packed [steps, slots, 1, 3*H*K], a/b [steps, slots, 1, H], A_log, dt_bias.
    """
    gen = torch.Generator().manual_seed(seed)
    H, K = heads, head_dim
    state0 = torch.randn(slots + 1, H, K, K, generator=gen) * 0.02
    state0[slots] = 0
    packed, a_all, b_all = [], [], []
    for _ in range(steps):
        q = _l2_bf16(_bf16_randn(gen, slots, H, K))
        k = _l2_bf16(_bf16_randn(gen, slots, H, K))
        v = _bf16_randn(gen, slots, H, K)
        a = _bf16_randn(gen, slots, H)
        b = _bf16_randn(gen, slots, H)
        packed.append(torch.cat([q.reshape(slots, -1), k.reshape(slots, -1), v.reshape(slots, -1)], -1)[:, None])
        a_all.append(a[:, None])
        b_all.append(b[:, None])
    return {
        "state0": state0.to(state_dtype),
        "packed": torch.stack(packed),
        "a": torch.stack(a_all),
        "b": torch.stack(b_all),
        "A_log": torch.zeros(H, dtype=BF16),
        "dt_bias": torch.zeros(H, dtype=BF16),
        "heads": H,
        "head_dim": K,
    }


def chunk_prefill_inputs(rows=16, lengths=(512, 2048, 8000), heads=16, head_dim=128, seed=0, random_state=False):
    """Config 4: ``rows`` rows whose lengths cycle through ``lengths`` (16 rows: 6 x 512, 5 x 2048, 5 x 8000 =
    53,312 tokens), packed back to back; H = HV = heads, K = V = head_dim.

    Draw order: state0 [rows+1, H, K, V] (zeros, or N(0, 0.02) with ``random_state``; the extra row is the
    scratch slot, zeroed), then over all T tokens q [T, H, K], k [T, H, K] (bf16 N(0,1), L2-normalised per
    head, rounded to bf16), v [T, H, V] bf16 N(0,1), a [T, H], b [T, H] bf16 N(0,1). A_log = dt_bias = 0.
    Returns dict with state0, packed [T, 3*H*K], a/b [T, H], lens, offsets, A_log, dt_bias.
    """
    gen = torch.Generator().manual_seed(seed)
    H, K = heads, head_dim
    lens = torch.tensor([lengths[i % len(lengths)] for i in range(rows)], dtype=torch.long)
    offsets = torch.cumsum(lens, 0) - lens
    T = int(lens.sum())
    if random_state:
        state0 = torch.randn(rows + 1, H, K, K, generator=gen) * 0.02
    else:
        state0 = torch.zeros(rows + 1, H, K, K)
    state0[rows] = 0
    q = _l2_bf16(_bf16_randn(gen, T, H, K))
    k = _l2_bf16(_bf16_randn(gen, T, H, K))
    v = _bf16_randn(gen, T, H, K)
    a = _bf16_randn(gen, T, H)
    b = _bf16_randn(gen, T, H)
    return {
        "state0": state0,
        "packed": torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], -1).contiguous(),
        "a": a, "b": b, "lens": lens, "offsets": offsets,
        "A_log": torch.zeros(H, dtype=BF16), "dt_bias": torch.zeros(H, dtype=BF16),
        "heads": H, "head_dim": K,
    }


def ring_decode_inputs(rows=64, hq=16, hkv=4, head_dim=256, window=512, seed=0, pool_rows=None):
    """Config 2: ``rows`` slots x 1 new token, GQA hq/hkv, ring [pool_rows, hkv, window+1, D].

    Draw order: per row ptr ~ U{0..W-1} and fill ~ U{1..W} (both via torch.randint), then q [rows, hkv,
    G, D], ring_k, ring_v [pool_rows, hkv, W+1, D], new_k [rows, hkv, 1, D], new_v [rows, hkv, 1, D],
    gate [rows, hq, D], all bf16 N(0,1). start = 16 W + ptr; ring_pos[c] = p for p in [start-fill, start-1]
    with c = p mod W, else -1 (column W is -1). Slot of row r is r (pool_rows defaults to rows + 1, the
    last row being the scratch slot).
    """
    gen = torch.Generator().manual_seed(seed)
    W, D, G = window, head_dim, hq // hkv
    S = rows + 1 if pool_rows is None else pool_rows
    ptr = torch.randint(0, W, (rows,), generator=gen)
    fill = torch.randint(1, W + 1, (rows,), generator=gen)
    q = _bf16_randn(gen, rows, hkv, G, D)
    ring_k = _bf16_randn(gen, S, hkv, W + 1, D)
    ring_v = _bf16_randn(gen, S, hkv, W + 1, D)
    new_k = _bf16_randn(gen, rows, hkv, 1, D)
    new_v = _bf16_randn(gen, rows, hkv, 1, D)
    gate_half = _bf16_randn(gen, rows, hq, D)
    starts = 16 * W + ptr
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for r in range(rows):
        for p in range(int(starts[r] - fill[r]), int(starts[r])):
            ring_pos[r, p % W] = p
    # q_proj output layout [N, 1, Hq*2D]: query half (unused here) then gate half per head
    gate = torch.cat([torch.zeros(rows, hq, D, dtype=BF16), gate_half], -1).reshape(rows, 1, hq * 2 * D)
    value = new_v.permute(0, 2, 1, 3).reshape(rows, 1, hkv * D).contiguous()
    return {
        "q": q.reshape(rows, hkv, G, D).contiguous(),
        "ring_k": ring_k, "ring_v": ring_v, "new_k": new_k, "new_v": new_v, "value": value,
        "gate": gate, "ring_pos": ring_pos, "slots": torch.arange(rows, dtype=torch.long),
        "starts": starts.long(), "lens": torch.ones(rows, dtype=torch.long), "fill": fill, "ptr": ptr,
        "window": W, "hq": hq, "hkv": hkv, "head_dim": D,
    }


class MixedServingLoad:
    """Config 5: ``slots`` concurrent streams. Initial contexts uniform over ``contexts`` tokens; each step
    every slot appends c tokens with c = 1 (p 0.8), U{2..16} (p 0.15), U{17..64} (p 0.05); after a step
    each slot is reset with probability ``reset_p`` and gets a fresh context. Token ids uniform in
    [0, vocab). One numpy Generator seeded ``seed`` drives every draw, in call order."""

    def __init__(self, slots=352, vocab=151936, contexts=(512, 2048, 8000), reset_p=0.01, seed=0):
        import numpy as np
        self.np = np
        self.rng = np.random.default_rng(seed)
        self.slots, self.vocab, self.contexts, self.reset_p = slots, vocab, tuple(contexts), reset_p

    def context(self):
        n = int(self.rng.choice(self.contexts))
        return self.rng.integers(0, self.vocab, n).tolist()

    def chunk_sizes(self):
        u = self.rng.random(self.slots)
        small = self.rng.integers(2, 17, self.slots)
        large = self.rng.integers(17, 65, self.slots)
        return self.np.where(u < 0.8, 1, self.np.where(u < 0.95, small, large))

    def step_requests(self):
        sizes = self.chunk_sizes()
        ids = self.rng.integers(0, self.vocab, int(sizes.sum()))
        out, at = [], 0
        for s, c in enumerate(sizes.tolist()):
            out.append((s, ids[at:at + c].tolist()))
            at += c
        return out

    def resets(self):
        return self.np.nonzero(self.rng.random(self.slots) < self.reset_p)[0].tolist()
