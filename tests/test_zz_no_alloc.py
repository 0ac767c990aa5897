"""Allocation-free split-K decode: hsg_ring_decode_noalloc (scratch in the library's static device array)
against hsg_ring_decode with a caller-allocated workspace, through the C ABI.

Both entry points run the same kernels on the same inputs, so outputs and ring writes must be bitwise equal.
With 16 query heads per kv head the split-K kernels run and keep their scores, block maxima and partial sums in
the scratch; with 4 the one-launch fused kernel runs and reads nothing from it. Two calls in a row on one GPU, the
second with fewer rows, check that the second call reads nothing the first left in the shared scratch.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HKV, D, W = 4, 256, 512


def _case(seed, n, slots_total, G):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(n, HKV, G, D, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(slots_total, HKV, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(slots_total, HKV, W + 1, D, generator=gen).to(torch.bfloat16)
    new_k = torch.randn(n, HKV, 1, D, generator=gen).to(torch.bfloat16)
    value = torch.randn(n, 1, HKV * D, generator=gen).to(torch.bfloat16)
    gate = torch.randn(n, 1, HKV * G * 2 * D, generator=gen).to(torch.bfloat16)
    slots = torch.randperm(slots_total - 1, generator=gen)[:n]
    starts = torch.randint(0, 3 * W, (n,), generator=gen)
    fills = torch.randint(0, W + 1, (n,), generator=gen)
    lens = (torch.rand(n, generator=gen) > 0.1).long()          # about one row in ten has no step
    ring_pos = torch.full((slots_total, W + 1), -1, dtype=torch.long)
    for s, st, f in zip(slots.tolist(), starts.tolist(), fills.tolist()):
        for p in range(max(0, st - f), st):
            ring_pos[s, p % W] = p
    return dict(q=q, ring_k=ring_k, ring_v=ring_v, new_k=new_k, value=value, gate=gate, slots=slots,
                starts=starts, lens=lens, ring_pos=ring_pos)


def _call(inp, noalloc):
    from hs_guard._lib import lib
    L = lib()
    dev = torch.device("cuda:0")
    d = {k: v.to(dev) for k, v in inp.items()}
    n, G = d["q"].shape[0], d["q"].shape[2]
    out = torch.full((n, 1, HKV * G * D), 7.0, dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    args = (d["q"].data_ptr(), HKV * G * D, D, G * D, D,
            d["ring_k"].data_ptr(), d["ring_v"].data_ptr(), d["ring_k"].shape[0], W,
            d["new_k"].data_ptr(), HKV * D, D, D,
            d["value"].data_ptr(), HKV * D, HKV * D, D,
            d["gate"].data_ptr(), HKV * G * 2 * D, HKV * G * 2 * D, G * 2 * D, 2 * D, D,
            d["ring_pos"].data_ptr(), d["slots"].data_ptr(), d["starts"].data_ptr(), d["lens"].data_ptr(), None,
            n, HKV, G, D, D ** -0.5, 1,
            out.data_ptr(), HKV * G * D, HKV * G * D, G * D, D)
    if noalloc:
        rc = L.hsg_ring_decode_noalloc(*args, st)
    else:
        ws = torch.empty(L.hsg_ring_decode_workspace_bytes(n, HKV, G, W), dtype=torch.uint8, device=dev)
        rc = L.hsg_ring_decode(*args, ws.data_ptr(), ws.numel(), st)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out.cpu(), d["ring_k"].cpu(), d["ring_v"].cpu()


def _scratch_cap():
    """HSG_RING_DECODE_SCRATCH_BYTES as include/hsg.h defines it."""
    import os
    import re
    header = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "hsg.h")
    m = re.search(r"#define HSG_RING_DECODE_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(header).read())
    return int(m.group(1)) << int(m.group(2))


@pytest.mark.parametrize("groups", [16, 4])
def test_noalloc_equals_workspace_entry_point(groups):
    """G = 16: the largest first call that fits the scratch, then a much smaller one. G = 4 (the fused kernel, which
    uses no workspace): a first call with more rows than the scratch would hold as a split-K workspace, which the
    fused path takes, then a smaller one. Then a call of at most HSG_RING_DECODE_SPLIT_UNITS rows x kv heads, which
    both entry points give to the split-K kernels (through the scratch, and through the caller's workspace)."""
    from hs_guard._lib import lib
    unit = lib().hsg_ring_decode_workspace_bytes(1, HKV, groups, W)
    first = _scratch_cap() // unit if groups > 8 else _scratch_cap() // unit + 14
    for seed, n, slots_total in ((0, first, first + 8), (1, 24, 40), (2, 12, 20)):
        print(f"[noalloc] G {groups}, seed {seed}: {n} rows, then the workspace entry point", flush=True)
        inp = _case(seed, n, slots_total, groups)
        a = _call(inp, noalloc=True)
        b = _call(inp, noalloc=False)
        for x, y, what in zip(a, b, ("out", "ring_k", "ring_v")):
            assert torch.equal(x, y), f"{what} differs at {n} rows"
        assert not torch.equal(a[1], inp["ring_k"])      # the step's keys were written
        live = inp["lens"].numpy() == 1
        assert np.all(a[0][~live].float().numpy() == 0)  # rows without a step get zeros (padded layout)
