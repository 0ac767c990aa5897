"""GPU parity of the ring-window attention (hsg_ring_attention) against the CPU oracle.

Outputs are bf16: they must agree with the float64 oracle (rounded at the reference's rounding points)
within two bf16 rounding steps (2**-7 relative) plus 1e-3 of the output scale. Ring writes and untouched
ring columns are compared bit-exactly.
"""
import numpy as np
import pytest
import torch

from oracle import ring as oring

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _check(got, ref, rtol=2.0 ** -7, atol_frac=1e-3, what="out"):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    atol = atol_frac * max(np.abs(ref).max(), 1e-30)
    # steps counted in the binade of the larger magnitude: one step of the upper binade is two of the lower
    bad = np.abs(got - ref) > rtol * np.maximum(np.abs(ref), np.abs(got)) + atol
    assert not bad.any(), f"{what}: {int(bad.sum())} values off, max diff {np.abs(got - ref).max():.3e}"


def test_config2_decode_with_ring_write():
    """Config 2: 64 slots x 1 token, 16q/4kv, D=256, W=512, random write pointer and fill, seed 0."""
    from hs_guard.engine.kernels import ring_attention_v8
    from hs_guard.synthetic import ring_decode_inputs
    print("[ring] config2 decode + write", flush=True)
    inp = ring_decode_inputs()
    dev = torch.device("cuda:0")
    W, D = inp["window"], inp["head_dim"]
    d = {k: v.to(dev) for k, v in inp.items() if torch.is_tensor(v)}
    rk, rv = d["ring_k"].clone(), d["ring_v"].clone()
    out = ring_attention_v8(d["q"].reshape(64, 4, 4, D), rk, rv, d["new_k"], d["value"], d["gate"], d["ring_pos"],
                            d["slots"], d["starts"], d["lens"], D ** -0.5, W, True)
    ref, _, rk_ref, rv_ref = oring.ring_attention_v8(
        _np(inp["q"]), _np(inp["ring_k"]), _np(inp["ring_v"]), _np(inp["new_k"]), _np(inp["value"]),
        _np(inp["gate"]), inp["ring_pos"].numpy(), inp["slots"].numpy(), inp["starts"].numpy(),
        inp["lens"].numpy(), D ** -0.5, W, True)
    _check(_np(out), ref)
    np.testing.assert_array_equal(_np(rk), rk_ref)   # written column = start % W, others untouched
    np.testing.assert_array_equal(_np(rv), rv_ref)


def test_multi_token_tick_no_write():
    """Lb=4 tick with lens [4, 2, 0, 1] (v8 contract, write_ring False): masking of the new keys."""
    from hs_guard.engine.kernels import ring_attention_v8
    print("[ring] Lb=4 tick", flush=True)
    gen = torch.Generator().manual_seed(3)
    N, Hkv, G, D, W, Lb = 4, 4, 4, 256, 512, 4
    S = 6
    q = torch.randn(N, Hkv, G * Lb, D, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    new_k = torch.randn(N, Hkv, Lb, D, generator=gen).to(torch.bfloat16)
    value = torch.randn(N, Lb, Hkv * D, generator=gen).to(torch.bfloat16)
    gate = torch.randn(N, Lb, Hkv * G * 2 * D, generator=gen).to(torch.bfloat16)
    slots = torch.tensor([3, 0, 5, 1])
    starts = torch.tensor([700, 5, 0, 511])
    lens = torch.tensor([4, 2, 0, 1])
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s, st in zip(slots.tolist(), starts.tolist()):
        for p in range(max(0, st - 600), st):
            ring_pos[s, p % W] = p
    dev = torch.device("cuda:0")
    out = ring_attention_v8(q.to(dev), ring_k.to(dev), ring_v.to(dev), new_k.to(dev), value.to(dev), gate.to(dev),
                            ring_pos.to(dev), slots.to(dev), starts.to(dev), lens.to(dev), D ** -0.5, W, False)
    ref, _, _, _ = oring.ring_attention_v8(_np(q), _np(ring_k), _np(ring_v), _np(new_k), _np(value), _np(gate),
                                           ring_pos.numpy(), slots.numpy(), starts.numpy(), lens.numpy(),
                                           D ** -0.5, W, False)
    _check(_np(out), ref)
    assert torch.count_nonzero(out[2]).item() == 0  # lens 0 row


def test_reference_contract_ungated():
    """ring_attention (v4 contract, ungated [N, Hkv, G*Lb, D] output) vs ring_attention_reference."""
    from hs_guard.engine.kernels import ring_attention
    print("[ring] ungated contract", flush=True)
    gen = torch.Generator().manual_seed(4)
    N, Hkv, G, D, W, Lb = 3, 2, 4, 256, 512, 2
    S = 4
    q = torch.randn(N, Hkv, G * Lb, D, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    new_k = torch.randn(N, Hkv, Lb, D, generator=gen).to(torch.bfloat16)
    new_v = torch.randn(N, Hkv, Lb, D, generator=gen).to(torch.bfloat16)
    slots, starts, lens = torch.tensor([2, 0, 1]), torch.tensor([1000, 3, 40]), torch.tensor([2, 2, 1])
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s, st in zip(slots.tolist(), starts.tolist()):
        for p in range(0, st):
            ring_pos[s, p % W] = p
    dev = torch.device("cuda:0")
    out = ring_attention(q.to(dev), ring_k.to(dev), ring_v.to(dev), new_k.to(dev), new_v.to(dev), ring_pos.to(dev),
                         slots.to(dev), starts.to(dev), lens.to(dev), D ** -0.5, W)
    # the Triton contract's numerics (bf16 probabilities in P.V, blockwise running max)
    ref = oring.attend_blockwise(_np(q), _np(ring_k), _np(ring_v), _np(new_k), _np(new_v), ring_pos.numpy(),
                                 slots.numpy(), starts.numpy(), lens.numpy(), D ** -0.5, W)
    from oracle.bf16 import bf16
    _check(_np(out), bf16(ref), rtol=2.0 ** -8)


def _decode_case(seed, N, Hkv, G, W, S, fills, lens, D=256):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(N, Hkv, G, D, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    new_k = torch.randn(N, Hkv, 1, D, generator=gen).to(torch.bfloat16)
    value = torch.randn(N, 1, Hkv * D, generator=gen).to(torch.bfloat16)
    gate = torch.randn(N, 1, Hkv * G * 2 * D, generator=gen).to(torch.bfloat16)
    slots = torch.randperm(S - 1, generator=gen)[:N]
    starts = torch.randint(0, 3 * W, (N,), generator=gen)
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s, st, f in zip(slots.tolist(), starts.tolist(), fills):
        for p_ in range(max(0, st - f), st):
            ring_pos[s, p_ % W] = p_
    return q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, torch.tensor(lens, dtype=torch.long)


@pytest.mark.parametrize("G,W", [(4, 512), (1, 64), (2, 128), (8, 512), (16, 256)])
def test_split_k_decode_matches_oracle_and_tiled_kernel(G, W):
    """hsg_ring_decode against the blockwise oracle and against the tiled kernel on the same decode tick: full,
    partial and empty rings (only the step's own key visible), a row with lens 0 (zeros), ring write bit-exact.
    Groups <= 8 run the fused one-launch kernel, G = 16 the three split-K kernels."""
    from hs_guard.engine.kernels import ring_attention_v8
    print(f"[ring] split-K decode G={G} W={W}", flush=True)
    N, Hkv, S, D = 6, 2, 8, 256
    fills = [W, W // 2, 0, 5, W - 1, W]
    lens = [1, 1, 1, 1, 0, 1]
    q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, lens_t = _decode_case(7 + G, N, Hkv, G, W, S,
                                                                                         fills, lens)
    dev = torch.device("cuda:0")
    outs, rings = [], []
    for split in (True, False):
        rk, rv = ring_k.to(dev), ring_v.to(dev)
        out = ring_attention_v8(q.to(dev), rk, rv, new_k.to(dev), value.to(dev), gate.to(dev), ring_pos.to(dev),
                                slots.to(dev), starts.to(dev), lens_t.to(dev), D ** -0.5, W, True, split_k=split)
        outs.append(_np(out))
        rings.append((_np(rk), _np(rv)))
    ref, _, rk_ref, rv_ref = oring.ring_attention_v8(
        _np(q), _np(ring_k), _np(ring_v), _np(new_k), _np(value), _np(gate), ring_pos.numpy(), slots.numpy(),
        starts.numpy(), lens_t.numpy(), D ** -0.5, W, True)
    _check(outs[0], ref, what="split-K vs oracle")
    _check(outs[0], outs[1], rtol=2.0 ** -8, what="split-K vs tiled")
    assert np.count_nonzero(outs[0][4]) == 0            # lens 0 row
    for rk, rv in rings:
        np.testing.assert_array_equal(rk, rk_ref)
        np.testing.assert_array_equal(rv, rv_ref)


@pytest.mark.parametrize("G,W", [(4, 512), (8, 128), (2, 256)])
def test_few_row_decode_with_workspace_takes_split_k(G, W):
    """Up to 8 query heads per kv head, a call of at most HSG_RING_DECODE_SPLIT_UNITS rows x kv heads that passes a
    workspace runs the three split-K kernels: against the blockwise oracle, and against the fused kernel (the same
    call without a workspace) within one bf16 rounding; ring writes bit-exact both ways."""
    from hs_guard._lib import lib
    print(f"[ring] few-row split-K decode G={G} W={W}", flush=True)
    L = lib()
    N, Hkv, S, D = 6, 2, 8, 256
    assert N * Hkv <= 64
    fills = [W, W // 2, 0, 5, W - 1, W]
    lens = [1, 1, 1, 1, 0, 1]
    q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, lens_t = _decode_case(31 + G, N, Hkv, G, W, S,
                                                                                         fills, lens)
    dev = torch.device("cuda:0")
    d = {n: t.to(dev) for n, t in dict(q=q, new_k=new_k, value=value, gate=gate, ring_pos=ring_pos, slots=slots,
                                         starts=starts, lens=lens_t).items()}
    st = torch.cuda.current_stream().cuda_stream
    m = G
    outs, rings = [], []
    for with_ws in (True, False):
        rk, rv = ring_k.to(dev), ring_v.to(dev)
        out = torch.zeros(N, 1, Hkv * G * D, dtype=torch.bfloat16, device=dev)
        need = L.hsg_ring_decode_workspace_bytes(N, Hkv, G, W)
        ws = torch.empty(need, dtype=torch.uint8, device=dev) if with_ws else None
        rc = L.hsg_ring_decode(
            d["q"].data_ptr(), Hkv * m * D, D, m * D, D, rk.data_ptr(), rv.data_ptr(), S, W,
            d["new_k"].data_ptr(), Hkv * D, D, D, d["value"].data_ptr(), d["value"].stride(0), d["value"].stride(1), D,
            d["gate"].data_ptr(), d["gate"].stride(0), d["gate"].stride(1), G * 2 * D, 2 * D, D,
            d["ring_pos"].data_ptr(), d["slots"].data_ptr(), d["starts"].data_ptr(), d["lens"].data_ptr(), None,
            N, Hkv, G, D, D ** -0.5, 1, out.data_ptr(), Hkv * G * D, Hkv * G * D, G * D, D,
            ws.data_ptr() if with_ws else None, need if with_ws else 0, st)
        torch.cuda.synchronize()
        assert rc == 0, rc
        outs.append(_np(out))
        rings.append((_np(rk), _np(rv)))
    ref, _, rk_ref, rv_ref = oring.ring_attention_v8(
        _np(q), _np(ring_k), _np(ring_v), _np(new_k), _np(value), _np(gate), ring_pos.numpy(), slots.numpy(),
        starts.numpy(), lens_t.numpy(), D ** -0.5, W, True)
    _check(outs[0], ref, what="split-K (workspace) vs oracle")
    _check(outs[0], outs[1], rtol=2.0 ** -8, what="split-K vs fused")
    assert np.count_nonzero(outs[0][4]) == 0            # lens 0 row
    for rk, rv in rings:
        np.testing.assert_array_equal(rk, rk_ref)
        np.testing.assert_array_equal(rv, rv_ref)


def test_mixed_packed_tick_split_between_kernels():
    """A packed tick with single- and multi-step rows: hsg_ring_decode takes the single-step rows and
    hsg_ring_attention (min_len 2) the rest; the result equals hsg_ring_attention on every row (min_len 0)
    within one bf16 rounding, and the ring writes are identical."""
    from hs_guard._lib import lib
    print("[ring] mixed packed tick, split between kernels", flush=True)
    gen = torch.Generator().manual_seed(21)
    Hkv, G, D, W, S = 4, 4, 256, 512, 9
    lens = torch.tensor([1, 3, 1, 0, 2, 1, 7], dtype=torch.long)
    N = len(lens)
    offsets = torch.cumsum(lens, 0) - lens
    T = int(lens.sum())
    hq = Hkv * G
    att_in = hq * 2 * D + 2 * Hkv * D
    proj = torch.randn(T, att_in, generator=gen).to(torch.bfloat16)       # gate | k | v layout of the engine
    q = torch.randn(T, hq * D, generator=gen).to(torch.bfloat16)
    k = torch.randn(T, Hkv * D, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    slots = torch.randperm(S - 1, generator=gen)[:N]
    starts = torch.randint(0, 2000, (N,), generator=gen)
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s, st in zip(slots.tolist(), starts.tolist()):
        for p_ in range(max(0, st - 400), st):
            ring_pos[s, p_ % W] = p_
    dev = torch.device("cuda:0")
    d = {n: t.to(dev) for n, t in dict(proj=proj, q=q, k=k, slots=slots, starts=starts, lens=lens,
                                         offsets=offsets, ring_pos=ring_pos).items()}
    L = lib()
    st = torch.cuda.current_stream().cuda_stream
    base = d["proj"].data_ptr()
    ws = torch.empty(L.hsg_ring_decode_workspace_bytes(N, Hkv, G, W), dtype=torch.uint8, device=dev)

    def run(split):
        rk, rv = ring_k.to(dev), ring_v.to(dev)
        out = torch.zeros(T, hq * D, dtype=torch.bfloat16, device=dev)
        args_tail = (d["ring_pos"].data_ptr(), d["slots"].data_ptr(), d["starts"].data_ptr(), d["lens"].data_ptr(),
                     d["offsets"].data_ptr())
        common = (d["q"].data_ptr(), 0, hq * D, G * D, D, rk.data_ptr(), rv.data_ptr(), S, W,
                  d["k"].data_ptr(), 0, Hkv * D, D, base + 2 * (hq * 2 * D + Hkv * D), 0, att_in, D,
                  base, 0, att_in, G * 2 * D, 2 * D, D) + args_tail
        if split:
            rc = L.hsg_ring_decode(*common, N, Hkv, G, D, D ** -0.5, 1, out.data_ptr(), 0, hq * D, G * D, D,
                                   ws.data_ptr(), ws.numel(), st)
            assert rc == 0, rc
        rc = L.hsg_ring_attention(*common, N, 8, Hkv, G, D, D ** -0.5, 1, 2 if split else 0, out.data_ptr(), 0,
                                  hq * D, G * D, D, st)
        assert rc == 0, rc
        torch.cuda.synchronize()
        return _np(out), _np(rk), _np(rv)

    a, rka, rva = run(True)
    b, rkb, rvb = run(False)
    _check(a, b, rtol=2.0 ** -8, what="split vs single kernel")
    np.testing.assert_array_equal(rka, rkb)
    np.testing.assert_array_equal(rva, rvb)


def test_config4_window_fill_64_tokens():
    """Config 4's second leg: after contexts of 512 / 2048 / 8000 tokens (rings full and wrapped), one 64-token
    tick per slot at W = 512 through hsg_ring_attention with the ring write (packed rows, 16 q / 4 kv heads,
    D = 256), against the oracle's attention and its Lb > 1 scatter (slot_engine_v8.py:86-88). A row of 37 tokens
    and a row whose tick crosses column 0 cover ragged and wrapping writes. Outputs within two bf16 steps; every
    ring column bit-exact."""
    from hs_guard._lib import lib
    print("[ring] config-4 window fill, 64-token tick at W=512", flush=True)
    gen = torch.Generator().manual_seed(44)
    Hkv, G, D, W, Lb = 4, 4, 256, 512, 64
    N = 16
    S = N + 1
    hq = Hkv * G
    starts = torch.tensor([(512, 2048, 8000)[i % 3] for i in range(N)], dtype=torch.long)
    starts[5] = 500                     # the tick's columns run 500..511, then 0..51
    lens = torch.full((N,), Lb, dtype=torch.long)
    lens[9] = 37
    offsets = torch.cumsum(lens, 0) - lens
    T = int(lens.sum())
    slots = torch.randperm(S - 1, generator=gen)[:N]
    ring_k = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, Hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s, st in zip(slots.tolist(), starts.tolist()):
        for p_ in range(max(0, st - W), st):
            ring_pos[s, p_ % W] = p_
    att_in = hq * 2 * D + 2 * Hkv * D
    proj = torch.randn(T, att_in, generator=gen).to(torch.bfloat16)      # q|gate per head, k, v (engine layout)
    q = torch.randn(T, hq * D, generator=gen).to(torch.bfloat16)
    k = torch.randn(T, Hkv * D, generator=gen).to(torch.bfloat16)
    dev = torch.device("cuda:0")
    d = {n: t.to(dev) for n, t in dict(proj=proj, q=q, k=k, slots=slots, starts=starts, lens=lens,
                                         offsets=offsets, ring_pos=ring_pos, ring_k=ring_k, ring_v=ring_v).items()}
    out = torch.zeros(T, hq * D, dtype=torch.bfloat16, device=dev)
    base = d["proj"].data_ptr()
    rc = lib().hsg_ring_attention(
        d["q"].data_ptr(), 0, hq * D, G * D, D, d["ring_k"].data_ptr(), d["ring_v"].data_ptr(), S, W,
        d["k"].data_ptr(), 0, Hkv * D, D, base + 2 * (hq * 2 * D + Hkv * D), 0, att_in, D,
        base, 0, att_in, G * 2 * D, 2 * D, D,
        d["ring_pos"].data_ptr(), d["slots"].data_ptr(), d["starts"].data_ptr(), d["lens"].data_ptr(),
        d["offsets"].data_ptr(), N, Lb, Hkv, G, D, D ** -0.5, 1, 0, out.data_ptr(), 0, hq * D, G * D, D,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    # oracle in the padded [N, Lb] layout
    qn, kn, pn = _np(q), _np(k), _np(proj)
    qp = np.zeros((N, Lb, hq * D), np.float32)
    kp = np.zeros((N, Lb, Hkv * D), np.float32)
    vp = np.zeros((N, Lb, Hkv * D), np.float32)
    gp = np.zeros((N, Lb, hq * 2 * D), np.float32)
    for n in range(N):
        o0, ln = int(offsets[n]), int(lens[n])
        qp[n, :ln], kp[n, :ln] = qn[o0:o0 + ln], kn[o0:o0 + ln]
        gp[n, :ln] = pn[o0:o0 + ln, :hq * 2 * D]
        vp[n, :ln] = pn[o0:o0 + ln, hq * 2 * D + Hkv * D:]
    qg = qp.reshape(N, Lb, Hkv, G, D).transpose(0, 2, 3, 1, 4).reshape(N, Hkv, G * Lb, D)
    new_k = kp.reshape(N, Lb, Hkv, D).transpose(0, 2, 1, 3)
    rk, rv = _np(ring_k), _np(ring_v)
    ref, _, _, _ = oring.ring_attention_v8(qg, rk, rv, new_k, vp, gp, ring_pos.numpy(), slots.numpy(),
                                           starts.numpy(), lens.numpy(), D ** -0.5, W, False)
    oring.ring_scatter(rk, rv, new_k, vp.reshape(N, Lb, Hkv, D).transpose(0, 2, 1, 3), slots.numpy(),
                       starts.numpy(), lens.numpy(), W)
    got = _np(out)
    far = 0
    for n in range(N):
        o0, ln = int(offsets[n]), int(lens[n])
        # output = bf16(bf16(o) * bf16(sigmoid(gate))): a one-step flip of bf16(o) near the top of its binade
        # becomes two steps of the product's lower binade, so the bound is 2**-6 with almost all within 2**-7
        _check(got[o0:o0 + ln], ref[n, :ln], rtol=2.0 ** -6, what=f"row {n}")
        g, r = got[o0:o0 + ln].astype(np.float64), ref[n, :ln].astype(np.float64)
        far += int((np.abs(g - r) > 2.0 ** -7 * np.maximum(np.abs(g), np.abs(r)) + 1e-3 * np.abs(r).max()).sum())
    assert far <= 1e-5 * got.size, f"{far} values beyond two bf16 steps"
    # the scratch column W takes the padded steps in the reference's scatter; this build never writes it
    np.testing.assert_array_equal(_np(d["ring_k"])[:, :, :W], rk[:, :, :W])
    np.testing.assert_array_equal(_np(d["ring_v"])[:, :, :W], rv[:, :, :W])


@pytest.mark.parametrize("hq", [16, 8])
def test_decode_rope_equals_norm_rope_then_decode(hq):
    """hsg_ring_decode_rope (q / k norm + RoPE inside the split-K scores kernel) is bitwise hsg_norm_rope followed by
    hsg_ring_decode on the same packed single-step rows: outputs, the new keys it writes out and both rings; a row
    with no step is left alone."""
    from hs_guard._lib import lib
    L = lib()
    print(f"[ring] decode with on-the-fly norm + RoPE, hq={hq}", flush=True)
    gen = torch.Generator().manual_seed(40 + hq)
    hkv, D, W, S = 4, 256, 512, 9
    G = hq // hkv
    lens = torch.tensor([1, 1, 0, 1, 1], dtype=torch.long)
    N = T = len(lens)
    att_in = hq * 2 * D + 2 * hkv * D
    proj = torch.randn(T, att_in, generator=gen).to(torch.bfloat16)
    ring_k = torch.randn(S, hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    ring_v = torch.randn(S, hkv, W + 1, D, generator=gen).to(torch.bfloat16)
    slots = torch.randperm(S - 1, generator=gen)[:N]
    starts = torch.randint(0, 3000, (N,), generator=gen)
    ring_pos = torch.full((S, W + 1), -1, dtype=torch.long)
    for s_, st_ in zip(slots.tolist(), starts.tolist()):
        for p_ in range(max(0, st_ - 450), st_):
            ring_pos[s_, p_ % W] = p_
    offsets = torch.arange(N, dtype=torch.long)
    pos = starts.clone()                      # one step per row: its position is its start
    qw = 1 + 0.1 * torch.randn(D, generator=gen)
    kw = 1 + 0.1 * torch.randn(D, generator=gen)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2).float() / 64))
    dev = torch.device("cuda:0")
    d = {k: v.to(dev) for k, v in dict(proj=proj, slots=slots, starts=starts, lens=lens, offsets=offsets, pos=pos,
                                        ring_pos=ring_pos, qw=qw, kw=kw, inv=inv).items()}
    st = torch.cuda.current_stream().cuda_stream
    base = d["proj"].data_ptr()
    kbase, vbase = base + 2 * hq * 2 * D, base + 2 * (hq * 2 * D + hkv * D)
    need = L.hsg_ring_decode_workspace_bytes(N, hkv, G, W)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    results = []
    for fused in (False, True):
        rk, rv = ring_k.to(dev), ring_v.to(dev)
        out = torch.zeros(T, hq * D, dtype=torch.bfloat16, device=dev)
        kbuf = torch.zeros(T, hkv * D, dtype=torch.bfloat16, device=dev)
        common_tail = (rk.data_ptr(), rv.data_ptr(), S, W)
        if fused:
            rc = L.hsg_ring_decode_rope(base, att_in, 2 * D, d["qw"].data_ptr(), 1e-6, kbase, att_in, D,
                                        d["kw"].data_ptr(), 1e-6, d["pos"].data_ptr(), d["inv"].data_ptr(), 64,
                                        kbuf.data_ptr(), hkv * D, *common_tail, vbase, att_in, D,
                                        base, att_in, G * 2 * D, 2 * D, D, d["ring_pos"].data_ptr(),
                                        d["slots"].data_ptr(), d["starts"].data_ptr(), d["lens"].data_ptr(),
                                        d["offsets"].data_ptr(), N, hkv, G, D, D ** -0.5, 1, out.data_ptr(),
                                        hq * D, G * D, D, ws.data_ptr(), need, st)
            assert rc == 0, rc
        else:
            q = torch.zeros(T, hq * D, dtype=torch.bfloat16, device=dev)
            rc = L.hsg_norm_rope(base, att_in, 2 * D, hq, d["qw"].data_ptr(), 1e-6, q.data_ptr(), hq * D, D,
                                 kbase, att_in, D, hkv, d["kw"].data_ptr(), 1e-6, kbuf.data_ptr(), hkv * D, D,
                                 d["pos"].data_ptr(), d["inv"].data_ptr(), 64, T, D, st)
            assert rc == 0, rc
            rc = L.hsg_ring_decode(q.data_ptr(), 0, hq * D, G * D, D, *common_tail, kbuf.data_ptr(), 0, hkv * D, D,
                                   vbase, 0, att_in, D, base, 0, att_in, G * 2 * D, 2 * D, D,
                                   d["ring_pos"].data_ptr(), d["slots"].data_ptr(), d["starts"].data_ptr(),
                                   d["lens"].data_ptr(), d["offsets"].data_ptr(), N, hkv, G, D, D ** -0.5, 1,
                                   out.data_ptr(), 0, hq * D, G * D, D, ws.data_ptr(), need, st)
            assert rc == 0, rc
        torch.cuda.synchronize()
        results.append((out.cpu(), kbuf.cpu(), rk.cpu(), rv.cpu()))
    (o0, k0, rk0, rv0), (o1, k1, rk1, rv1) = results
    live = lens.numpy() == 1
    assert torch.equal(o0[live], o1[live])
    assert torch.equal(k0[live], k1[live])
    assert torch.equal(rk0, rk1) and torch.equal(rv0, rv1)
    assert not torch.equal(rk1, ring_k)                 # the steps' keys were written
