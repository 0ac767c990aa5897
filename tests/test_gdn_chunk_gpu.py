"""GPU parity of the chunked GDN prefill (hsg_gdn_chunk_prefill) against the CPU oracle.

Reference: the float64 recurrence (``oracle.gdn.gdn_recurrent_seq``) for short rows and the float64 WY/UT
chunk form (``oracle.gdn.gdn_chunk``, pinned to the recurrence) at config 4's lengths. Tolerances as the
slot step: final fp32 state within 1e-3 relative (norm ratio and max ratio), bf16 outputs within one bf16
rounding (2**-8 relative) plus 1e-3 of the output scale; untouched pool rows bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn

pytestmark = pytest.mark.gpu

STATE_TOL = 1e-3


def _np(t):
    return t.detach().float().cpu().numpy()


def _state_err(got, ref):
    d = np.asarray(got, np.float64) - np.asarray(ref, np.float64)
    return float(np.linalg.norm(d) / np.linalg.norm(ref)), float(np.abs(d).max() / np.abs(ref).max())


def _out_close(got, ref, rtol=2.0 ** -8, atol_frac=1e-3):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    atol = atol_frac * max(np.abs(ref).max(), 1e-30)
    # steps counted in the binade of the larger magnitude: one step of the upper binade is two of the lower
    bad = np.abs(got - ref) > rtol * np.maximum(np.abs(ref), np.abs(got)) + atol
    return int(bad.sum()), float(np.abs(got - ref).max())


def _row_reference(packed, a, b, A_log, dt, S0, H, HV, K, chunk=False):
    """packed [T, 2*H*K + HV*K] of one row -> (o [T, HV, V], S [HV, K, V]) in float64."""
    T = packed.shape[0]
    rep = HV // H
    q = packed[:, :H * K].reshape(T, H, K).repeat(rep, axis=1)
    k = packed[:, H * K:2 * H * K].reshape(T, H, K).repeat(rep, axis=1)
    v = packed[:, 2 * H * K:].reshape(T, HV, K)
    g, beta = ogdn.gates(a, b, A_log, dt)
    if chunk:
        return ogdn.gdn_chunk(q, k, v, g, beta, S0)
    return ogdn.gdn_recurrent_seq(q, k, v, g, beta, S0)


def test_packed_rows_match_recurrence():
    """GQA (H=2, HV=4), packed rows of lengths [130, 64, 1, 0, 77] (partial and whole chunks, an empty row),
    permuted slots, nonzero A_log / dt_bias, random initial state."""
    from hs_guard.engine.kernels import gdn_chunk_prefill
    print("[chunk] packed rows vs recurrence", flush=True)
    gen = torch.Generator().manual_seed(11)
    H, HV, K = 2, 4, 128
    C = 2 * H * K + HV * K
    lens = torch.tensor([130, 64, 1, 0, 77], dtype=torch.long)
    offsets = torch.tensor([0, 130, 194, 195, 195], dtype=torch.long)
    T = int(lens.sum())
    packed = torch.randn(T, C, generator=gen).to(torch.bfloat16)
    a = torch.randn(T, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(T, HV, generator=gen).to(torch.bfloat16)
    A_log = (torch.rand(HV, generator=gen) * 2 - 1).to(torch.bfloat16)
    dt = torch.randn(HV, generator=gen).to(torch.bfloat16)
    S = 8
    state0 = torch.randn(S, HV, K, K, generator=gen) * 0.05
    slots = torch.tensor([5, 1, 7, 3, 0], dtype=torch.long)
    dev = torch.device("cuda:0")
    state = state0.to(dev)
    o, _ = gdn_chunk_prefill(packed.to(dev), H * K, H, K, HV, K, a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev),
                             state, slots.to(dev), lens.to(dev), offsets.to(dev))
    torch.cuda.synchronize()
    got_o, got_s = _np(o), _np(state)
    pk, an, bn = _np(packed), _np(a), _np(b)
    for n in range(5):
        ln, off, s = int(lens[n]), int(offsets[n]), int(slots[n])
        if ln == 0:
            continue
        o_ref, s_ref = _row_reference(pk[off:off + ln], an[off:off + ln], bn[off:off + ln], _np(A_log), _np(dt),
                                      _np(state0[s]), H, HV, K)
        bad, worst = _out_close(got_o[off:off + ln], o_ref)
        assert bad == 0, f"row {n}: {bad} outputs off (max diff {worst:.3e})"
        rel, mx = _state_err(got_s[s], s_ref)
        assert rel <= STATE_TOL and mx <= STATE_TOL, f"row {n}: state error norm {rel:.2e} max {mx:.2e}"
    for s in (2, 3, 4, 6):   # slot 3 belongs to the empty row; the others are unused
        np.testing.assert_array_equal(got_s[s], _np(state0[s]))


def test_padded_layout_fp16_state_and_sq():
    """Padded [N, L] layout (zeros past lens), fp16 state pool, sq = bf16(o)**2."""
    from hs_guard.engine.kernels import gdn_chunk_prefill
    print("[chunk] padded + fp16 state", flush=True)
    gen = torch.Generator().manual_seed(12)
    H = HV = 4
    K = 128
    N, L = 3, 100
    C = 2 * H * K + HV * K
    packed = torch.randn(N, L, C, generator=gen).to(torch.bfloat16)
    a = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    A_log = torch.zeros(HV, dtype=torch.bfloat16)
    dt = torch.zeros(HV, dtype=torch.bfloat16)
    state0 = (torch.randn(4, HV, K, K, generator=gen) * 0.02).half()
    slots = torch.tensor([2, 0, 1], dtype=torch.long)
    lens = torch.tensor([100, 37, 0], dtype=torch.long)
    dev = torch.device("cuda:0")
    state = state0.to(dev)
    o, sq = gdn_chunk_prefill(packed.to(dev), H * K, H, K, HV, K, a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev),
                              state, slots.to(dev), lens.to(dev), with_sq=True)
    torch.cuda.synchronize()
    got_o = _np(o)
    for n in range(N):
        ln, s = int(lens[n]), int(slots[n])
        assert np.count_nonzero(got_o[n, ln:]) == 0
        if ln == 0:
            continue
        o_ref, s_ref = _row_reference(_np(packed[n, :ln]), _np(a[n, :ln]), _np(b[n, :ln]), _np(A_log), _np(dt),
                                      _np(state0[s]), H, HV, K)
        bad, worst = _out_close(got_o[n, :ln], o_ref, rtol=2.0 ** -7)
        assert bad == 0, f"row {n}: {bad} outputs off (max diff {worst:.3e})"
        s_ref = s_ref.astype(np.float16).astype(np.float64)
        rel, mx = _state_err(_np(state[s]), s_ref)
        assert rel <= 4e-3 and mx <= 4e-3, f"row {n}: state error norm {rel:.2e} max {mx:.2e}"
    ob = got_o.astype(np.float64)
    np.testing.assert_array_equal(_np(sq), (ob * ob).astype(np.float32))
    np.testing.assert_array_equal(_np(state[1]), _np(state0[1]))   # the empty row's slot
    np.testing.assert_array_equal(_np(state[3]), _np(state0[3]))


def test_config4_lengths_match_chunk_oracle():
    """Config-4 geometry at its maximum lengths: rows of 512, 2048 and 8000 tokens, 16 heads x 128, q/k
    L2-normalised bf16, random initial state, against the float64 chunk form."""
    from hs_guard.engine.kernels import gdn_chunk_prefill
    from hs_guard.synthetic import chunk_prefill_inputs
    print("[chunk] config-4 lengths 512/2048/8000", flush=True)
    H = 16
    K = 128
    for random_state in (True,):
        inp = chunk_prefill_inputs(rows=3, random_state=random_state, seed=4)
        dev = torch.device("cuda:0")
        state = inp["state0"].to(dev)
        slots = torch.arange(3, dtype=torch.long)
        o, _ = gdn_chunk_prefill(inp["packed"].to(dev), H * K, H, K, H, K, inp["a"].to(dev), inp["b"].to(dev),
                                 inp["A_log"].to(dev), inp["dt_bias"].to(dev), state, slots.to(dev),
                                 inp["lens"].to(dev), inp["offsets"].to(dev))
        torch.cuda.synchronize()
        got_o, got_s = _np(o), _np(state)
        pk, an, bn = _np(inp["packed"]), _np(inp["a"]), _np(inp["b"])
        for n in range(3):
            ln, off = int(inp["lens"][n]), int(inp["offsets"][n])
            o_ref, s_ref = _row_reference(pk[off:off + ln], an[off:off + ln], bn[off:off + ln], _np(inp["A_log"]),
                                          _np(inp["dt_bias"]), _np(inp["state0"][n]), H, H, K, chunk=True)
            bad, worst = _out_close(got_o[off:off + ln], o_ref)
            assert bad == 0, f"len {ln}: {bad} outputs off (max diff {worst:.3e})"
            rel, mx = _state_err(got_s[n], s_ref)
            print(f"[chunk] len {ln} random_state={random_state}: state err norm {rel:.2e} max {mx:.2e}", flush=True)
            assert rel <= STATE_TOL and mx <= STATE_TOL, f"len {ln}: state error norm {rel:.2e} max {mx:.2e}"
        assert torch.count_nonzero(state[3]).item() == 0


def test_chunk_prefill_equals_streamed_slot_steps():
    """The same 300-token rows through the chunk kernel and through the slot-step kernel in 64-token ticks
    (the reference's streaming prefill) end in the same state."""
    from hs_guard.engine.kernels import gdn_chunk_prefill, gdn_slot_v8
    print("[chunk] chunk == streamed slot steps", flush=True)
    gen = torch.Generator().manual_seed(13)
    H = HV = 16
    K = 128
    N, L = 4, 300
    C = 2 * H * K + HV * K
    packed = torch.randn(N, L, C, generator=gen).to(torch.bfloat16)
    a = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    A_log = torch.zeros(HV, dtype=torch.bfloat16)
    dt = torch.zeros(HV, dtype=torch.bfloat16)
    state0 = torch.randn(N + 1, HV, K, K, generator=gen) * 0.02
    dev = torch.device("cuda:0")
    slots = torch.arange(N, device=dev)
    lens = torch.full((N,), L, dtype=torch.long, device=dev)
    pd, ad, bd, Ad, dd = packed.to(dev), a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev)
    s_chunk = state0.to(dev)
    o_chunk, _ = gdn_chunk_prefill(pd, H * K, H, K, HV, K, ad, bd, Ad, dd, s_chunk, slots, lens)
    s_step = state0.to(dev)
    outs = []
    for t0 in range(0, L, 64):
        t1 = min(L, t0 + 64)
        o, _ = gdn_slot_v8(pd[:, t0:t1].contiguous(), H * K, H, K, HV, K, ad[:, t0:t1].contiguous(),
                           bd[:, t0:t1].contiguous(), Ad, dd, s_step, slots,
                           torch.full((N,), t1 - t0, dtype=torch.long, device=dev))
        outs.append(o)
    torch.cuda.synchronize()
    rel, mx = _state_err(_np(s_chunk[:N]), _np(s_step[:N]))
    assert rel <= STATE_TOL and mx <= STATE_TOL, f"state error norm {rel:.2e} max {mx:.2e}"
    bad, worst = _out_close(_np(o_chunk), _np(torch.cat(outs, 1)), rtol=2.0 ** -7)
    assert bad == 0, f"{bad} outputs differ (max diff {worst:.3e})"


def test_tick_split_between_slot_step_and_chunk():
    """The engine's split of one packed tick: rows n < R with lens >= 9 through hsg_gdn_chunk_prefill_gated (raw
    outputs, then the gated RMSNorm), every other row through hsg_gdn_slot_step_gated with the matching skip
    filter. Against the whole tick through the slot step alone: states within 1e-3 relative, gated outputs
    within two bf16 steps; a row of >= 9 tokens at n >= R stays in the slot step."""
    from hs_guard._lib import lib
    print("[chunk] tick split slot step / chunk", flush=True)
    gen = torch.Generator().manual_seed(21)
    H, HV, K = 2, 4, 128
    C = 2 * H * K + HV * K
    stride = C + HV * K + 2 * HV               # qkv | z | b | a, the engine's fused projection
    lens = torch.tensor([40, 12, 1, 9, 11, 3, 0], dtype=torch.long)
    offsets = torch.cat([torch.zeros(1, dtype=torch.long), torch.cumsum(lens, 0)[:-1]])
    T, R, THR = int(lens.sum()), 4, 9
    proj = torch.randn(T, stride, generator=gen).to(torch.bfloat16)
    A_log = (torch.rand(HV, generator=gen) * 2 - 1).to(torch.bfloat16)
    dt = torch.randn(HV, generator=gen).to(torch.bfloat16)
    norm_w = (1 + 0.1 * torch.randn(K, generator=gen)).to(torch.bfloat16)
    state0 = torch.randn(8, HV, K, K, generator=gen) * 0.05
    slots = torch.tensor([6, 2, 0, 4, 1, 7, 3], dtype=torch.long)
    dev = torch.device("cuda:0")
    P, A_d, dt_d, w_d = proj.to(dev), A_log.to(dev), dt.to(dev), norm_w.to(dev)
    sl, ln, of = slots.to(dev), lens.to(dev), offsets.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    base = P.data_ptr()
    a_ptr, b_ptr, z_ptr = base + 2 * (C + HV * K + HV), base + 2 * (C + HV * K), base + 2 * C

    def slot_step(state, out, skip_rows):
        assert lib().hsg_gdn_slot_step_gated(base, stride, 0, H * K, 2 * H * K, a_ptr, b_ptr, stride, A_d.data_ptr(),
                                             dt_d.data_ptr(), state.data_ptr(), 0, 8, sl.data_ptr(), ln.data_ptr(),
                                             of.data_ptr(), 7, 0, H, HV, K, K, K ** -0.5, z_ptr, stride,
                                             w_d.data_ptr(), 1e-6, out.data_ptr(), skip_rows, THR, 8, st) == 0

    s_ref, o_ref = state0.to(dev), torch.zeros(T, HV * K, dtype=torch.bfloat16, device=dev)
    slot_step(s_ref, o_ref, 0)
    s_split, o_split = state0.to(dev), torch.zeros(T, HV * K, dtype=torch.bfloat16, device=dev)
    slot_step(s_split, o_split, R)
    raw = torch.zeros(T, HV * K, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(lib().hsg_gdn_chunk_workspace_bytes(R, 64, HV), dtype=torch.uint8, device=dev)
    assert lib().hsg_gdn_chunk_prefill_gated(base, stride, 0, H * K, 2 * H * K, a_ptr, b_ptr, stride, A_d.data_ptr(),
                                             dt_d.data_ptr(), s_split.data_ptr(), 0, 8, sl.data_ptr(), ln.data_ptr(),
                                             of.data_ptr(), R, 64, H, HV, K, K, K ** -0.5, raw.data_ptr(), z_ptr,
                                             stride, w_d.data_ptr(), 1e-6, o_split.data_ptr(), THR, ws.data_ptr(),
                                             ws.numel(), st) == 0
    torch.cuda.synchronize()
    chunk_rows = [n for n in range(R) if lens[n] >= THR]
    assert chunk_rows == [0, 1, 3]
    # the gated output is bf16(bf16(w * bf16(o * r)) * silu(z)): a one-step difference of bf16(o * r) between the
    # two paths can become two steps of the output, so all within 2**-6 and almost all within 2**-7
    far = 0
    for n in range(7):   # the skip filter left exactly the chunk rows to the chunk kernels
        ln_n, off = int(lens[n]), int(offsets[n])
        if ln_n == 0:
            continue
        bad, worst = _out_close(_np(o_split[off:off + ln_n]), _np(o_ref[off:off + ln_n]), rtol=2.0 ** -6)
        assert bad == 0, f"row {n}: {bad} outputs off (max diff {worst:.3e})"
        far += _out_close(_np(o_split[off:off + ln_n]), _np(o_ref[off:off + ln_n]), rtol=2.0 ** -7)[0]
    assert far <= 1e-4 * T * HV * K, f"{far} outputs beyond two bf16 steps"
    for s in range(8):
        rel, mx = _state_err(_np(s_split[s]), _np(s_ref[s]))
        assert rel <= STATE_TOL and mx <= STATE_TOL, f"slot {s}: state error norm {rel:.2e} max {mx:.2e}"
    np.testing.assert_array_equal(_np(s_split[5]), _np(state0[5]))   # unused slot


def test_chunk_output_rounding_rate_matches_slot_step():
    """Precision of the chunk path: over 4 rows of 512 tokens from a random state, the fraction of bf16 outputs
    whose rounding differs from the float64 recurrence's must stay within 1.5 times the slot-step kernel's (fp32
    FMA recurrence) on the same rows (measured: 1.2e-4 against 1.4e-4); the state within 1e-6 relative (1.2e-7).
    What this rate exposes: a bf16 hi + lo split of the state path's operands (~2^-17) flipped one output in 400,
    and an fp32 in-chunk cumulative decay, whose rounding every e^(G_i - G_j) inherits, one in 2,500."""
    from hs_guard.engine.kernels import gdn_chunk_prefill, gdn_slot_v8
    from oracle.bf16 import bf16
    print("[chunk] output rounding rate vs slot step", flush=True)
    gen = torch.Generator().manual_seed(17)
    H = HV = 16
    K = 128
    N, L = 4, 512
    C = 2 * H * K + HV * K
    packed = (torch.randn(N, L, C, generator=gen) * 0.5).to(torch.bfloat16)
    a = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    A_log = (torch.rand(HV, generator=gen) - 0.5).to(torch.bfloat16)
    dt = (torch.randn(HV, generator=gen) * 0.3).to(torch.bfloat16)
    state0 = torch.randn(N + 1, HV, K, K, generator=gen) * 0.02
    dev = torch.device("cuda:0")
    slots = torch.arange(N, device=dev)
    lens = torch.full((N,), L, dtype=torch.long, device=dev)
    pd, ad, bd, Ad, dd = packed.to(dev), a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev)
    s_chunk = state0.to(dev)
    o_chunk, _ = gdn_chunk_prefill(pd, H * K, H, K, HV, K, ad, bd, Ad, dd, s_chunk, slots, lens)
    s_step = state0.to(dev)
    outs = []
    for t0 in range(0, L, 64):
        o, _ = gdn_slot_v8(pd[:, t0:t0 + 64].contiguous(), H * K, H, K, HV, K, ad[:, t0:t0 + 64].contiguous(),
                           bd[:, t0:t0 + 64].contiguous(), Ad, dd, s_step, slots,
                           torch.full((N,), 64, dtype=torch.long, device=dev))
        outs.append(o)
    o_step = torch.cat(outs, 1)
    torch.cuda.synchronize()
    flips = {"chunk": 0, "step": 0}
    worst = 0.0
    for n in range(N):
        o_ref, s_ref = _row_reference(_np(packed[n]), _np(a[n]), _np(b[n]), _np(A_log), _np(dt), _np(state0[n]),
                                      H, HV, K, chunk=True)
        ref = bf16(o_ref)
        flips["chunk"] += int((_np(o_chunk[n]) != ref).sum())
        flips["step"] += int((_np(o_step[n]) != ref).sum())
        worst = max(worst, _state_err(_np(s_chunk[n]), s_ref)[0])
    total = N * L * HV * K
    rate = {k: v / total for k, v in flips.items()}
    print(f"[chunk] bf16 flips vs float64: chunk {rate['chunk']:.2e}, slot step {rate['step']:.2e}; "
          f"chunk state rel {worst:.2e}", flush=True)
    assert rate["chunk"] <= 1.5 * rate["step"]
    assert worst <= 1e-6
