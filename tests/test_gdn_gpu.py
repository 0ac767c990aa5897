"""GPU parity of the GDN slot step (hsg_gdn_slot_step / _gated) against the CPU oracle.

Tolerances (north star): fp32 recurrent state within 1e-3 relative error, both as the norm ratio
||S_gpu - S_ref|| / ||S_ref|| and as max |S_gpu - S_ref| / max |S_ref|. bf16 outputs within one bf16
rounding (2**-8 relative) plus 1e-3 of the output scale. Untouched pool rows are compared bit-exactly.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from oracle import glue as oglue

pytestmark = pytest.mark.gpu

STATE_TOL = 1e-3


def _state_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = got - ref
    return float(np.linalg.norm(d) / np.linalg.norm(ref)), float(np.abs(d).max() / np.abs(ref).max())


def _out_close(got, ref, rtol=2.0 ** -8, atol_frac=1e-3):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    atol = atol_frac * max(np.abs(ref).max(), 1e-30)
    bad = np.abs(got - ref) > rtol * np.abs(ref) + atol
    return int(bad.sum()), float(np.abs(got - ref).max())


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("state_dtype", [torch.float32, torch.float16])
def test_config1_64_steps(state_dtype):
    """Config 1: 16 slots x 1 token, 16 heads x 128, 64 sequential steps, seed 0."""
    from hs_guard.engine.kernels import gdn_slot_v8
    from hs_guard.synthetic import gdn_step_inputs
    print(f"[gdn] config1 state={state_dtype}", flush=True)
    inp = gdn_step_inputs(state_dtype=state_dtype)
    H, K = inp["heads"], inp["head_dim"]
    dev = torch.device("cuda:0")
    state = inp["state0"].to(dev)
    slots = torch.arange(16, dtype=torch.long, device=dev)
    lens = torch.ones(16, dtype=torch.long, device=dev)
    A_log, dt = inp["A_log"].to(dev), inp["dt_bias"].to(dev)
    ref_state = _np(inp["state0"]).astype(np.float64)
    for t in range(inp["packed"].shape[0]):
        packed = inp["packed"][t]
        o, sq = gdn_slot_v8(packed.to(dev), H * K, H, K, H, K, inp["a"][t].to(dev), inp["b"][t].to(dev),
                            A_log, dt, state, slots, lens)
        o_ref, sq_ref, ref_state = ogdn.gdn_slot_step(_np(packed), H * K, H, K, H, K, _np(inp["a"][t]),
                                                      _np(inp["b"][t]), _np(inp["A_log"]), _np(inp["dt_bias"]),
                                                      ref_state, np.arange(16), np.ones(16, np.int64))
        if state_dtype == torch.float16:
            ref_state = ref_state.astype(np.float16).astype(np.float64)  # storage rounding of the pool
        bad, worst = _out_close(_np(o), o_ref, rtol=2.0 ** -7 if state_dtype == torch.float16 else 2.0 ** -8)
        assert bad == 0, f"step {t}: {bad} outputs off (max diff {worst})"
        ob = _np(o).astype(np.float64)
        np.testing.assert_array_equal(_np(sq), (ob * ob).astype(np.float32))
    torch.cuda.synchronize()
    rel, mx = _state_err(_np(state[:16]), ref_state[:16])
    tol = STATE_TOL if state_dtype == torch.float32 else 4e-3
    assert rel <= tol and mx <= tol, f"state error norm {rel:.2e} max {mx:.2e}"
    assert torch.count_nonzero(state[16]).item() == 0  # scratch slot untouched


@pytest.mark.parametrize("burst_min", [8, 1])
def test_multi_token_and_padding(burst_min):
    """L=7 tick with lens [7, 3, 0, 1, 5]; slots permuted; a row with lens 0 leaves its slot bit-exact. burst_min 1:
    every row through the 8-token MFMA burst path (padded layout, zeros past lens, two value heads per key head)."""
    from hs_guard.engine.kernels import gdn_slot_v8
    print("[gdn] multi-token padded tick", flush=True)
    gen = torch.Generator().manual_seed(1)
    N, L, H, K = 5, 7, 4, 128
    HV = 8  # two value heads per key head
    S = 9
    packed = torch.randn(N, L, 2 * H * K + HV * K, generator=gen).to(torch.bfloat16)
    a = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(N, L, HV, generator=gen).to(torch.bfloat16)
    A_log = (torch.rand(HV, generator=gen) * 2 - 1).to(torch.bfloat16)
    dt = torch.randn(HV, generator=gen).to(torch.bfloat16)
    state0 = torch.randn(S, HV, K, K, generator=gen) * 0.05
    slots = torch.tensor([6, 2, 4, 0, 8], dtype=torch.long)
    lens = torch.tensor([7, 3, 0, 1, 5], dtype=torch.long)
    dev = torch.device("cuda:0")
    state = state0.to(dev)
    o, sq = gdn_slot_v8(packed.to(dev), H * K, H, K, HV, K, a.to(dev), b.to(dev), A_log.to(dev), dt.to(dev),
                        state, slots.to(dev), lens.to(dev), burst_min=burst_min)
    o_ref, _, st_ref = ogdn.gdn_slot_step(_np(packed), H * K, H, K, HV, K, _np(a), _np(b), _np(A_log), _np(dt),
                                          _np(state0), slots.numpy(), lens.numpy())
    ob = _np(o).astype(np.float64)
    np.testing.assert_array_equal(_np(sq), (ob * ob).astype(np.float32))
    bad, worst = _out_close(_np(o), o_ref)
    assert bad == 0, f"{bad} outputs off (max diff {worst})"
    for n in range(N):
        assert torch.count_nonzero(o[n, int(lens[n]):]).item() == 0
    got = _np(state)
    for s in range(S):
        if s in (6, 2, 0, 8):
            rel, mx = _state_err(got[s], st_ref[s])
            assert rel <= STATE_TOL and mx <= STATE_TOL, f"slot {s}: {rel:.2e} {mx:.2e}"
        else:  # slot 4 (lens 0) and unused slots are not touched
            np.testing.assert_array_equal(got[s], _np(state0[s]))


def _check_packed_gated(lens_list, A_log_vals, dt_scale, seed, state_scale=0.02, burst_min=8, fp16_state=False):
    """Packed rows (offsets) with the fused gated RMSNorm epilogue, z read from a strided projection; gated
    outputs and states against the oracle, rows of zero length bit-exact. fp16_state: the pool stored in fp16 (the
    oracle starts from the same fp16 values and its final state is rounded to fp16 as the kernel stores it), held
    to the fp16 bar of test_config1_64_steps."""
    from hs_guard._lib import lib
    gen = torch.Generator().manual_seed(seed)
    H = HV = 16
    K = 128
    N = len(lens_list)
    lens = torch.tensor(lens_list, dtype=torch.long)
    offsets = torch.cumsum(lens, 0) - lens
    T = int(lens.sum())
    C = 2 * H * K + HV * K
    stride = C + HV * K + 2 * HV + 8   # fused projection row: qkv | z | b | a | pad
    proj = torch.randn(T, stride, generator=gen).to(torch.bfloat16)
    qkv, z = proj[:, :C], proj[:, C:C + HV * K]
    ab = torch.randn(T, 2 * HV, generator=gen).to(torch.bfloat16)
    A_log = torch.tensor(A_log_vals, dtype=torch.float32).repeat(HV // len(A_log_vals)).to(torch.bfloat16)
    dt = (torch.randn(HV, generator=gen) * dt_scale).to(torch.bfloat16)
    norm_w = (1 + 0.1 * torch.randn(K, generator=gen)).to(torch.bfloat16)
    S = N + 2
    state0 = torch.randn(S, HV, K, K, generator=gen) * state_scale
    if fp16_state:
        state0 = state0.half()
    slots = torch.randperm(S, generator=gen)[:N]
    dev = torch.device("cuda:0")
    proj_d, ab_d, state = proj.to(dev), ab.to(dev), state0.to(dev)
    out = torch.empty(T, HV * K, dtype=torch.bfloat16, device=dev)
    slots_d, lens_d, off_d = slots.to(dev), lens.to(dev), offsets.to(dev)
    A_d, dt_d, w_d = A_log.to(dev), dt.to(dev), norm_w.to(dev)
    rc = lib().hsg_gdn_slot_step_gated(
        proj_d.data_ptr(), stride, 0, H * K, 2 * H * K, ab_d[:, HV:].data_ptr(), ab_d.data_ptr(), 2 * HV,
        A_d.data_ptr(), dt_d.data_ptr(), state.data_ptr(), 1 if fp16_state else 0, S, slots_d.data_ptr(),
        lens_d.data_ptr(), off_d.data_ptr(), N, 0, H, HV, K, K, K ** -0.5, proj_d[:, C:].data_ptr(), stride,
        w_d.data_ptr(), 1e-6, out.data_ptr(), 0, 0, burst_min, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    # oracle in padded form
    L = int(lens.max())
    packed_pad = np.zeros((N, L, C))
    a_pad = np.zeros((N, L, HV))
    b_pad = np.zeros((N, L, HV))
    z_pad = np.zeros((N, L, HV, K))
    for n in range(N):
        o0, ln = int(offsets[n]), int(lens[n])
        packed_pad[n, :ln] = _np(qkv[o0:o0 + ln])
        a_pad[n, :ln] = _np(ab[o0:o0 + ln, HV:])
        b_pad[n, :ln] = _np(ab[o0:o0 + ln, :HV])
        z_pad[n, :ln] = _np(z[o0:o0 + ln]).reshape(ln, HV, K)
    o_ref, _, st_ref = ogdn.gdn_slot_step(packed_pad, H * K, H, K, HV, K, a_pad, b_pad, _np(A_log), _np(dt),
                                          _np(state0), slots.numpy(), lens.numpy())
    if fp16_state:
        st_ref = st_ref.astype(np.float16).astype(np.float64)   # the pool's storage rounding
    from oracle.bf16 import bf16
    gated_ref = oglue.gated_rmsnorm(bf16(o_ref), z_pad, _np(norm_w), 1e-6)
    got = _np(out)
    for n in range(N):
        o0, ln = int(offsets[n]), int(lens[n])
        if ln == 0:
            continue
        bad, worst = _out_close(got[o0:o0 + ln], gated_ref[n, :ln].reshape(ln, HV * K), rtol=2.0 ** -6,
                                atol_frac=4e-3)
        assert bad == 0, f"row {n}: {bad} gated outputs off (max {worst})"
    torch.cuda.synchronize()
    gs = _np(state)
    for n in range(N):
        s = int(slots[n])
        if int(lens[n]) > 0:
            rel, mx = _state_err(gs[s], st_ref[s])
            tol = 4e-3 if fp16_state else STATE_TOL
            assert rel <= tol and mx <= tol, f"row {n} slot {s}: {rel:.2e} {mx:.2e}"
        else:
            np.testing.assert_array_equal(gs[s], _np(state0[s]))
    for s in set(range(S)) - set(slots.tolist()):
        np.testing.assert_array_equal(gs[s], _np(state0[s]))


@pytest.mark.parametrize("burst_min", [0, 1], ids=["tokens", "bursts_all"])
def test_packed_gated_fp16_state(burst_min):
    """fp16 state storage (the reference StreamingGuard's) on rows of 1-64 tokens, token by token and with every row
    in MFMA bursts (full and partial), against the oracle."""
    print(f"[gdn] packed + gated, fp16 state, burst_min {burst_min}", flush=True)
    _check_packed_gated([64, 17, 1, 9, 0, 33, 8, 2], [0.0, -1.0], 1.0, seed=13, state_scale=0.05, burst_min=burst_min,
                        fp16_state=True)


def test_packed_gated_matches_oracle():
    """Packed rows with the fused gated RMSNorm epilogue: short rows, one of zero length."""
    print("[gdn] packed + gated", flush=True)
    _check_packed_gated([3, 1, 0, 4], [0.0], 0.5, seed=2)


@pytest.mark.parametrize("burst_min", [0, 8, 1], ids=["tokens", "bursts8", "bursts_all"])
@pytest.mark.parametrize("case", ["bursts", "fast_decay", "zero_decay"])
def test_packed_gated_long_rows_and_decay(case, burst_min):
    """Rows spanning several 8-token bursts (full and partial), and heads whose decay is fast enough that the
    kernel's deferred decay factor is folded back into the state mid-row (exp(A_log) = 20: exp(g) ~ 1e-6 per
    token, below 2^-40 after two tokens) or underflows to exactly zero in fp32 (exp(A_log) = 403). burst_min: the
    token path for every row (0), the MFMA burst path for the rows of 8 or more tokens (8), or for every row with
    partial bursts padded (1)."""
    print(f"[gdn] packed + gated, {case}, burst_min {burst_min}", flush=True)
    lens = [64, 17, 1, 9, 0, 33, 8, 2]
    A_log = {"bursts": [0.0, -1.0], "fast_decay": [0.0, 3.0, -2.0, 3.0], "zero_decay": [6.0, 0.0, 3.0, 6.0]}[case]
    _check_packed_gated(lens, A_log, 1.0, seed=11, state_scale=0.05, burst_min=burst_min)


@pytest.mark.parametrize("burst_min", [0, 8])
@pytest.mark.parametrize("state_code", [0, 1])
def test_conv_fused_step_equals_conv_then_step(state_code, burst_min):
    """hsg_gdn_conv_slot_step_gated (conv + SiLU inside the slot step) == hsg_conv_silu_update followed by
    hsg_gdn_slot_step_gated, bit for bit on the gated outputs, the state and the conv history pool: rows of 0 to 64
    tokens (one to eight 8-token bursts, rows shorter than the 3-token history), HV == H; on the token path and with
    the rows of 8 or more tokens on the MFMA burst path."""
    from hs_guard._lib import lib
    L = lib()
    print(f"[gdn] conv fused, state code {state_code}", flush=True)
    gen = torch.Generator().manual_seed(21)
    H = HV = 4
    K = 128
    C = 3 * H * K
    lens = torch.tensor([64, 17, 9, 8, 3, 2, 1, 0, 1, 33], dtype=torch.long)
    N = len(lens)
    offsets = torch.cumsum(lens, 0) - lens
    T = int(lens.sum())
    stride = C + HV * K + 2 * HV + 24          # raw projection row: qkv | z | b | a | pad
    proj = torch.randn(T, stride, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, 4, generator=gen) * 0.5).to(torch.bfloat16)
    S = N + 3
    pool0 = torch.randn(S, 3, C, generator=gen).to(torch.bfloat16)
    state0 = torch.randn(S, HV, K, K, generator=gen) * 0.05
    if state_code == 1:
        state0 = state0.half()
    A_log = (torch.rand(HV, generator=gen) * 2 - 1).to(torch.bfloat16)
    dt = torch.randn(HV, generator=gen).to(torch.bfloat16)
    norm_w = (1 + 0.1 * torch.randn(K, generator=gen)).to(torch.bfloat16)
    slots = torch.randperm(S, generator=gen)[:N]
    dev = torch.device("cuda:0")
    pd, wd, nwd = proj.to(dev), w.to(dev), norm_w.to(dev)
    Ad, dtd = A_log.to(dev), dt.to(dev)
    sl, ln, of = slots.to(dev), lens.to(dev), offsets.to(dev)
    st = torch.cuda.current_stream().cuda_stream
    base = pd.data_ptr()
    a_ptr, b_ptr, z_ptr = base + 2 * (C + HV * K + HV), base + 2 * (C + HV * K), base + 2 * C
    # separate kernels
    pool_a, state_a = pool0.to(dev), state0.to(dev)
    conv = torch.empty(T, C, dtype=torch.bfloat16, device=dev)
    out_a = torch.zeros(T, HV * K, dtype=torch.bfloat16, device=dev)
    assert L.hsg_conv_silu_update(base, stride, pool_a.data_ptr(), S, wd.data_ptr(), 4, sl.data_ptr(), ln.data_ptr(),
                                  of.data_ptr(), N, 0, C, conv.data_ptr(), C, st) == 0
    assert L.hsg_gdn_slot_step_gated(conv.data_ptr(), C, 0, H * K, 2 * H * K, a_ptr, b_ptr, stride, Ad.data_ptr(),
                                     dtd.data_ptr(), state_a.data_ptr(), state_code, S, sl.data_ptr(), ln.data_ptr(),
                                     of.data_ptr(), N, 0, H, HV, K, K, K ** -0.5, z_ptr, stride, nwd.data_ptr(), 1e-6,
                                     out_a.data_ptr(), 0, 0, burst_min, st) == 0
    # fused
    pool_b, state_b = pool0.to(dev), state0.to(dev)
    out_b = torch.zeros(T, HV * K, dtype=torch.bfloat16, device=dev)
    assert L.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, wd.data_ptr(), pool_b.data_ptr(), C,
                                          a_ptr, b_ptr, stride, Ad.data_ptr(), dtd.data_ptr(), state_b.data_ptr(),
                                          state_code, S, sl.data_ptr(), ln.data_ptr(), of.data_ptr(), N, H, HV, K, K,
                                          K ** -0.5, z_ptr, stride, nwd.data_ptr(), 1e-6, out_b.data_ptr(), burst_min,
                                          st) == 0
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(state_a, state_b)
    assert torch.equal(pool_a, pool_b)
    assert torch.equal(pool_b[slots[lens == 0]], pool0[slots[lens == 0]].to(dev))   # untouched
    # only packed rows and one value head per key head are accepted
    assert L.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, wd.data_ptr(), pool_b.data_ptr(), C,
                                          a_ptr, b_ptr, stride, Ad.data_ptr(), dtd.data_ptr(), state_b.data_ptr(),
                                          state_code, S, sl.data_ptr(), ln.data_ptr(), None, N, H, HV, K, K,
                                          K ** -0.5, z_ptr, stride, nwd.data_ptr(), 1e-6, out_b.data_ptr(), burst_min,
                                          st) == -1
    assert L.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, wd.data_ptr(), pool_b.data_ptr(), C,
                                          a_ptr, b_ptr, stride, Ad.data_ptr(), dtd.data_ptr(), state_b.data_ptr(),
                                          state_code, S, sl.data_ptr(), ln.data_ptr(), of.data_ptr(), N, H // 2, HV, K,
                                          K, K ** -0.5, z_ptr, stride, nwd.data_ptr(), 1e-6, out_b.data_ptr(),
                                          burst_min, st) == -3
