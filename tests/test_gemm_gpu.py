"""hsg_gemm_bf16, the projections' GEMM with a fixed hipBLASLt solution, and the committed plan table.

D[M, N] = A[M, K] . W[N, K]^T in bf16 with fp32 accumulation (the reference's nn.Linear products,
src/hs_guard/engine/slot_engine_v8.py:52-53,63-65,72,78,89). Checked against the fp32 product of the same bf16
inputs: relative Frobenius error within 2^-7 (bf16 output rounding plus accumulation order), repeated calls equal
bit for bit, every plan-table solution runnable on its problem, and the engine's mm equal to a direct call with
the table's solution.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(8448, 1024), (1024, 2048), (10240, 1024), (1024, 4096), (7168, 1024), (1024, 3584)]


def _run(A, W, index, ws):
    from hs_guard._lib import lib
    M, K = A.shape
    N = W.shape[0]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    rc = lib().hsg_gemm_bf16(A.data_ptr(), K, W.data_ptr(), K, out.data_ptr(), N, M, N, K, index, ws.data_ptr(),
                             ws.numel(), torch.cuda.current_stream().cuda_stream)
    return rc, out


def _inputs(M, N, K, seed=0):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn(M, K, generator=gen, device="cuda").bfloat16()
    W = (torch.randn(N, K, generator=gen, device="cuda") * 0.02).bfloat16()
    return A, W


def _rel(out, A, W):
    ref = A.float() @ W.float().t()
    return ((out.float() - ref).norm() / ref.norm()).item()


@pytest.mark.parametrize("M", [1, 17, 352, 1536])
def test_heuristic_solution_matches_fp32_and_repeats(M):
    from hs_guard.engine.gemm_plan import WORKSPACE_BYTES
    print(f"[gemm] heuristic solution M={M}", flush=True)
    ws = torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device="cuda")
    for N, K in SHAPES:
        A, W = _inputs(M, N, K)
        rc, out = _run(A, W, -1, ws)
        assert rc == 0, (M, N, K, rc)
        rc2, out2 = _run(A, W, -1, ws)
        torch.cuda.synchronize()
        assert rc2 == 0 and torch.equal(out, out2)
        assert _rel(out, A, W) <= 2.0 ** -7, (M, N, K)


@pytest.mark.parametrize("ws_bytes", [32 << 20, 0], ids=["32MiB", "none"])
def test_heuristic_solution_fits_the_workspace(ws_bytes):
    """Solution -1 at a shape whose first heuristic candidate needs more workspace than the caller has (the running
    hipBLASLt returns a 61 MiB candidate first at M = 11264, N = 7168, K = 1024 whatever the preference's limit):
    the first candidate that fits runs, as a 176-slot engine's 64-token prefill tick needs. The candidates the
    plan table is built from respect the limit too."""
    from hs_guard._lib import lib
    print(f"[gemm] heuristic within {ws_bytes} bytes of workspace at M=11264", flush=True)
    M, N, K = 11264, 7168, 1024
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    A, W = _inputs(M, N, K)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    rc = lib().hsg_gemm_bf16(A.data_ptr(), K, W.data_ptr(), K, out.data_ptr(), N, M, N, K, -1, ws.data_ptr(), ws_bytes,
                             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, rc
    assert _rel(out, A, W) <= 2.0 ** -7
    idx = (ctypes.c_int32 * 16)()
    wsz = (ctypes.c_size_t * 16)()
    n = lib().hsg_gemm_candidates(M, N, K, idx, wsz, 16, ws_bytes)
    assert n > 0 and all(wsz[i] <= ws_bytes for i in range(n))


def test_candidates_and_rejections():
    from hs_guard._lib import lib
    from hs_guard.engine.gemm_plan import WORKSPACE_BYTES
    L = lib()
    ws = torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device="cuda")
    idx = (ctypes.c_int32 * 16)()
    wsz = (ctypes.c_size_t * 16)()
    n = L.hsg_gemm_candidates(1536, 8448, 1024, idx, wsz, 16, WORKSPACE_BYTES)
    assert 0 < n <= 16 and all(wsz[i] <= WORKSPACE_BYTES for i in range(n))
    A, W = _inputs(1536, 8448, 1024)
    for i in range(min(n, 4)):
        rc, out = _run(A, W, idx[i], ws)
        assert rc == 0 and _rel(out, A, W) <= 2.0 ** -7
    assert _run(A, W, 1 << 30, ws)[0] == -3          # no such solution: HSG_ERR_SHAPE, nothing launched
    out = torch.empty(4, 4, dtype=torch.bfloat16, device="cuda")
    assert L.hsg_gemm_bf16(A.data_ptr(), 1024, W.data_ptr(), 1024, out.data_ptr(), 8448, 0, 8448, 1024, -1,
                           ws.data_ptr(), ws.numel(), None) == -1       # M = 0
    assert L.hsg_gemm_bf16(A.data_ptr(), 512, W.data_ptr(), 1024, out.data_ptr(), 8448, 4, 8448, 1024, -1,
                           ws.data_ptr(), ws.numel(), None) == -1       # lda < K
    assert L.hsg_gemm_blas_version() > 0


def test_plan_table_solutions_run_on_their_problems():
    """Every committed solution of a sample of table entries (all shapes, the smallest, a middle and the largest
    bucket) runs on its problem within the fp32 bar; the table loads for this hipBLASLt."""
    from hs_guard.engine.gemm_plan import PLAN_PATH, WORKSPACE_BYTES, GemmPlans
    import json
    import os
    if not os.path.exists(PLAN_PATH):
        pytest.skip("no committed plan table")
    plans = GemmPlans.load()
    data = json.load(open(PLAN_PATH))
    assert plans.table, f"plan table generated for hipBLASLt {data['blas_version']}, not this one"
    ws = torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device="cuda")
    Ms = sorted({k[0] for k in plans.table})
    sample = {Ms[0], Ms[len(Ms) // 2], Ms[-1]}
    checked = 0
    for (M, N, K), index in plans.table.items():
        if M not in sample:
            continue
        A, W = _inputs(M, N, K, seed=M)
        rc, out = _run(A, W, index, ws)
        assert rc == 0, (M, N, K, index, rc)
        assert _rel(out, A, W) <= 2.0 ** -7, (M, N, K, index)
        checked += 1
    print(f"[gemm] {checked} committed solutions checked", flush=True)
    assert checked > 0


def test_engine_mm_uses_the_table():
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    model = GuardModel.random(cfg, seed=0, device="cuda")
    eng = SlotStreamEngine(model, 4, use_graphs=False)
    w = eng.layers[0]["w_in"]
    M = 16
    x = torch.randn(M, w.shape[1], device="cuda").bfloat16()
    got = eng.mm(x, w, torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda"))
    rc, ref = _run(x, w, eng.gemm_plans.index(M, w.shape[0], w.shape[1]), eng.gemm_ws)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(got, ref)


def test_engine_mm_falls_back_when_a_solution_is_rejected():
    """A table entry the running hipBLASLt does not have (an index out of its solution map: HSG_ERR_SHAPE, nothing
    launched) is dropped with a warning and the product runs on the heuristic's first candidate."""
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    eng = SlotStreamEngine(GuardModel.random(cfg, seed=0, device="cuda"), 4, use_graphs=False)
    w = eng.layers[0]["w_in"]
    M, N, K = 24, w.shape[0], w.shape[1]
    eng.gemm_plans.table[(M, N, K)] = 1 << 30
    x = torch.randn(M, K, device="cuda").bfloat16()
    with pytest.warns(UserWarning, match="rejected solution"):
        got = eng.mm(x, w, torch.empty(M, N, dtype=torch.bfloat16, device="cuda"))
    assert (M, N, K) not in eng.gemm_plans.table
    rc, ref = _run(x, w, -1, eng.gemm_ws)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(got, ref)


def test_process_runs_torchs_hipblaslt():
    """Loading the library binds the hipBLASLt torch bundles (the one the plan table was made with), whatever the
    import order of the caller."""
    import os
    import torch as _torch
    from hs_guard._lib import lib
    lib().hsg_gemm_blas_version()
    maps = open("/proc/self/maps").read()
    paths = {line.split()[-1] for line in maps.splitlines() if "libhipblaslt.so" in line}
    torch_lib = os.path.realpath(os.path.join(os.path.dirname(_torch.__file__), "lib"))
    assert paths and all(os.path.realpath(p).startswith(torch_lib) for p in paths), paths


def _skinny(A, W, out=None):
    from hs_guard._lib import lib
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    rc = lib().hsg_gemm_bf16_skinny(A.data_ptr(), A.stride(0), W.data_ptr(), W.stride(0), out.data_ptr(),
                                    out.stride(0), M, N, K, torch.cuda.current_stream().cuda_stream)
    return rc, out


def _within_rounding(out, A, W):
    """Every element within bf16 output rounding (2^-8 relative, twice the half-ulp) of the float64 product, plus
    2^-16 of sum_k |a_k w_k| for fp32 accumulation: a dropped, doubled or misplaced 8-element piece fails it."""
    a, w = A.double().cpu(), W.double().cpu()
    ref = a @ w.t()
    mag = a.abs() @ w.abs().t()
    err = (out.double().cpu() - ref).abs()
    bad = err > 2.0 ** -8 * ref.abs() + 2.0 ** -16 * mag
    return int(bad.sum())


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
def test_skinny_matches_float64_per_element(M):
    """hsg_gemm_bf16_skinny at the engine's projection shapes and at ragged ones (N not a multiple of 4, K not a
    multiple of 512, K = 8), every element against the float64 product; repeated calls equal bit for bit."""
    print(f"[gemm] skinny M={M}", flush=True)
    for N, K in SHAPES + [(1027, 1016), (5, 8), (13, 4104), (3, 520)]:
        A, W = _inputs(M, N, K, seed=M)
        rc, out = _skinny(A, W)
        rc2, out2 = _skinny(A, W)
        torch.cuda.synchronize()
        assert rc == 0 and rc2 == 0, (M, N, K, rc, rc2)
        assert torch.equal(out, out2), (M, N, K)
        assert _within_rounding(out, A, W) == 0, (M, N, K)


def test_skinny_reads_only_k_columns_and_rows_are_independent():
    """Row strides beyond K with NaN in the padding columns (never read), and each row's result the same bit for
    bit whether it is computed alone or with 7 others (the per-row reduction order depends on K only)."""
    M, N, K, ld = 8, 1030, 1016, 1032
    A, W = _inputs(M, N, ld, seed=3)
    A[:, K:] = float("nan")
    W[:, K:] = float("nan")
    A, W = A[:, :K], W[:, :K]
    out_full = torch.full((M, N + 6), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc, _ = _skinny(A, W, out_full[:, :N])
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.isnan(out_full[:, N:]).all()          # columns past N untouched
    out = out_full[:, :N]
    assert not torch.isnan(out).any()
    assert _within_rounding(out, A, W) == 0
    for m in range(M):
        rc, one = _skinny(A[m:m + 1], W)
        torch.cuda.synchronize()
        assert rc == 0 and torch.equal(one[0], out[m]), m


def test_engine_mm_routes_small_products_to_the_skinny_kernel():
    """The engine's mm at M <= 8 is hsg_gemm_bf16_skinny's product; with gemm_skinny_rows=0 it is hipBLASLt's."""
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    model = GuardModel.random(cfg, seed=0, device="cuda")
    eng = SlotStreamEngine(model, 4, use_graphs=False)
    eng0 = SlotStreamEngine(model, 4, use_graphs=False, gemm_skinny_rows=0)
    w = eng.layers[0]["w_in"]
    for M in (1, 4, 8, 9):
        x = torch.randn(M, w.shape[1], device="cuda").bfloat16()
        got = eng.mm(x, w, torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda"))
        got0 = eng0.mm(x, w, torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda"))
        rc, ref = _skinny(x, w) if M <= 8 else _run(x, w, eng.gemm_plans.index(M, w.shape[0], w.shape[1]),
                                                    eng.gemm_ws)
        rc0, ref0 = _run(x, w, eng0.gemm_plans.index(M, w.shape[0], w.shape[1]), eng0.gemm_ws)
        torch.cuda.synchronize()
        assert rc == 0 and rc0 == 0
        assert torch.equal(got, ref), M
        assert torch.equal(got0, ref0), M
    with pytest.raises(ValueError):
        SlotStreamEngine(model, 4, use_graphs=False, gemm_skinny_rows=9)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_skinny_silu_equals_silu_mul_then_skinny(M):
    """hsg_gemm_bf16_skinny_silu (the SiLU gate applied while staging A) is bitwise hsg_silu_mul followed by
    hsg_gemm_bf16_skinny, at the MLP's down projection and at ragged shapes with a padded gate|up row stride."""
    from hs_guard._lib import lib
    L = lib()
    st = torch.cuda.current_stream().cuda_stream
    print(f"[gemm] skinny silu M={M}", flush=True)
    for N, K, pad in ((1024, 3584, 0), (1027, 1016, 8), (9, 4104, 16)):
        gen = torch.Generator(device="cuda").manual_seed(100 + M)
        gu = (torch.randn(M, 2 * K + pad, generator=gen, device="cuda") * 2).bfloat16()
        W = (torch.randn(N, K, generator=gen, device="cuda") * 0.02).bfloat16()
        act = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
        assert L.hsg_silu_mul(gu.data_ptr(), gu.stride(0), K, act.data_ptr(), M, st) == 0
        rc, ref = _skinny(act, W)
        got = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        rc2 = L.hsg_gemm_bf16_skinny_silu(gu.data_ptr(), gu.stride(0), W.data_ptr(), K, got.data_ptr(), N, M, N, K,
                                          st)
        torch.cuda.synchronize()
        assert rc == 0 and rc2 == 0, (M, N, K)
        assert torch.equal(got, ref), (M, N, K)
        assert _within_rounding(got, act, W) == 0, (M, N, K)


def test_engine_mm_silu_both_routes():
    """The engine's mm_silu: one fused launch at M <= 8, hsg_silu_mul + mm above; both equal the two-step product."""
    from hs_guard._lib import lib
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    cfg = GuardConfig(vocab_size=1000, hidden_size=1024, num_hidden_layers=4, intermediate_size=1024,
                      linear_num_key_heads=2, linear_num_value_heads=4, num_attention_heads=8,
                      num_key_value_heads=2, window_tokens=32)
    eng = SlotStreamEngine(GuardModel.random(cfg, seed=0, device="cuda"), 4, use_graphs=False)
    w = eng.layers[0]["w_down"]
    N, I = w.shape
    st = torch.cuda.current_stream().cuda_stream
    for M in (1, 8, 16):
        gu = torch.randn(M, 2 * I, device="cuda").bfloat16()
        act = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device="cuda")
        got = eng.mm_silu(gu, w, torch.empty(M, N, dtype=torch.bfloat16, device="cuda"), act)
        act_ref = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
        assert lib().hsg_silu_mul(gu.data_ptr(), 2 * I, I, act_ref.data_ptr(), M, st) == 0
        ref = eng.mm(act_ref, w, torch.empty(M, N, dtype=torch.bfloat16, device="cuda"))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), M
        assert bool(torch.isnan(act).all()) == (M <= 8), M      # the fused route leaves act unwritten


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
def test_skinny_addnorm_equals_add_rmsnorm_then_skinny(M):
    """hsg_gemm_bf16_skinny_addnorm (residual add + RMSNorm while staging A) is bitwise hsg_add_rmsnorm followed by
    hsg_gemm_bf16_skinny: the same product, the new residual in the output buffer, the input residual untouched;
    at the wide projections (two columns per wave) and a narrow ragged N."""
    from hs_guard._lib import lib
    L = lib()
    st = torch.cuda.current_stream().cuda_stream
    H = 1024
    print(f"[gemm] skinny addnorm M={M}", flush=True)
    for N in (8448, 7168, 37):
        gen = torch.Generator(device="cuda").manual_seed(200 + M)
        hidden = (torch.randn(M, H, generator=gen, device="cuda") * 3).bfloat16()
        mix = torch.randn(M, H, generator=gen, device="cuda").bfloat16()
        w1 = 1 + 0.1 * torch.randn(H, generator=gen, device="cuda")
        W = (torch.randn(N, H, generator=gen, device="cuda") * 0.02).bfloat16()
        h_ref, normed = hidden.clone(), torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
        assert L.hsg_add_rmsnorm(h_ref.data_ptr(), mix.data_ptr(), w1.data_ptr(), 1e-6, normed.data_ptr(), M, H,
                                 st) == 0
        rc, ref = _skinny(normed, W)
        h_in = hidden.clone()
        h_out = torch.full((M, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        got = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        rc2 = L.hsg_gemm_bf16_skinny_addnorm(h_in.data_ptr(), H, mix.data_ptr(), H, w1.data_ptr(), 1e-6,
                                             h_out.data_ptr(), H, W.data_ptr(), H, got.data_ptr(), N, M, N, H, None,
                                             st)
        torch.cuda.synchronize()
        assert rc == 0 and rc2 == 0, (M, N)
        assert torch.equal(got, ref), (M, N)
        assert torch.equal(h_out, h_ref), (M, N)
        assert torch.equal(h_in, hidden), (M, N)


def test_skinny_addnorm_with_bias():
    """The add + RMSNorm product with a Linear's bias (the risk heads' first projection after the final norm): the
    same bits as without the bias up to the bias, which enters the fp32 sum before the one rounding; every element
    within the rounding bound of the float64 normed . W^T + b."""
    from hs_guard._lib import lib
    L = lib()
    st = torch.cuda.current_stream().cuda_stream
    H, N = 1024, 1024
    for M in (1, 3, 8):
        gen = torch.Generator(device="cuda").manual_seed(300 + M)
        hidden = (torch.randn(M, H, generator=gen, device="cuda") * 3).bfloat16()
        mix = torch.randn(M, H, generator=gen, device="cuda").bfloat16()
        w1 = 1 + 0.1 * torch.randn(H, generator=gen, device="cuda")
        W = (torch.randn(N, H, generator=gen, device="cuda") * 0.02).bfloat16()
        b = torch.randn(N, generator=gen, device="cuda").bfloat16()
        h_ref, normed = hidden.clone(), torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
        assert L.hsg_add_rmsnorm(h_ref.data_ptr(), mix.data_ptr(), w1.data_ptr(), 1e-6, normed.data_ptr(), M, H,
                                 st) == 0
        h_out = torch.empty(M, H, dtype=torch.bfloat16, device="cuda")
        got = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        rc = L.hsg_gemm_bf16_skinny_addnorm(hidden.data_ptr(), H, mix.data_ptr(), H, w1.data_ptr(), 1e-6,
                                            h_out.data_ptr(), H, W.data_ptr(), H, got.data_ptr(), N, M, N, H,
                                            b.data_ptr(), st)
        torch.cuda.synchronize()
        assert rc == 0
        assert torch.equal(h_out, h_ref)
        ref = normed.double().cpu() @ W.double().cpu().t() + b.double().cpu()
        mag = normed.double().cpu().abs() @ W.double().cpu().abs().t() + b.double().cpu().abs()
        err = (got.double().cpu() - ref).abs()
        assert int((err > 2.0 ** -8 * ref.abs() + 2.0 ** -16 * mag).sum()) == 0, M
