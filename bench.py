"""Benchmark of the streaming slot step on one MI355X (BASELINE.json's metric and config 5).

Workload (config 5, mixed serving): 352 concurrent slots on the full random-init backbone (hidden 1024,
24 layers 3 GDN : 1 attention, GDN 16x128, attention 16q/4kv/256, MLP 3584, vocab 151,936, bf16 weights
N(0, 0.02)), fp32 recurrent state. Every slot first gets an initial context drawn uniformly from
{512, 2048, 8000} tokens, prefilled through step() outside the timed steps (reported as
prefill_352_contexts: once cold, capturing each tick shape's graph, then again into reset slots with the same
lengths, warm). Each step every slot appends c tokens, c = 1 (p 0.8), U{2..16} (p 0.15), U{17..64} (p 0.05);
the step is one engine tick under hipGraph through step_packed, the
call the reference's serving backend makes (examples/demo/runtime_v10.py:114): H2D of the packed tick, graph
replay, D2H of both roles' probabilities, stream sync, probabilities on the host as [R, n, lb, 3]. The same
load through step() (one CPU tensor per request and role, StreamingGuard's call) is reported as api_step.
After each step every slot is reset with p = 0.01 and re-prefilled with a fresh context, untimed (prefill is
outside the reference's timing scope, docs/technical_report.tex:117).

value = streamed tokens / summed host-to-host step time over the K timed steps. Also reported: p50/p95
of those step times, the pure 352 x 1-token decode step and the 1-slot single-token step (20 warm-up +
200 measured each, docs/technical_report.tex:115), the roofline of the dominant kernel (the GDN slot step
at the 352 x 1-token decode shape, HIP events on its launch stream) and the CPU baseline (the repo's CPU
restatement of the same step timed on this host on a bounded sample).
"""
import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "hs-guard_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
REF_L20 = {"min_tokens_per_s_352": 15075.6, "worst_p95_ms_352": 18.368, "single_token_p50_ms": 2.384}


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def percentile(xs, q):
    import numpy as np
    return float(np.percentile(np.asarray(xs), q))


def gdn_roofline(torch, lib, rows=352, iters=100, state_dtype=0):
    """Average duration of hsg_gdn_conv_slot_step_gated (the GDN layers' conv + SiLU and gated slot step in one
    kernel, as the engine runs it) at the decode shape (rows x 1 token, 16 heads x 128x128), HIP events recorded
    on the stream the kernel is launched on. Algorithmic bytes per launch: per (row, head) the state read +
    write 2*K*V*4 B and the 3-row conv history of its 3*128 channels read + written 2 x 3 x 384 x 2 B, per (row,
    head, token) the raw q, k, v, z in and out = 5 x 256 B and a, b = 4 B, and once per launch the conv
    weights 16 x 384 x 4 x 2 B.

    Launch i works on state buffer and conv pool i mod 3, so no launch reads what the previous one wrote: in a step
    each GDN layer's state was last touched a whole step earlier, and one buffer reused back to back would be
    read partly from the 256 MB Infinity Cache, faster than any step sees it."""
    from hs_guard._lib import HSG_GDN_BURST_MIN_DEFAULT
    dev = torch.device("cuda:0")
    H = HV = 16
    K = V = 128
    C = 3 * H * K
    stride = C + HV * V + 2 * HV
    gen = torch.Generator(device=dev).manual_seed(1)
    states, pools = [], []
    for _ in range(3):
        state = (torch.randn(rows + 1, HV, K, V, generator=gen, device=dev) * 0.02)
        states.append(state.half() if state_dtype == 1 else state)
        pools.append(torch.randn(rows + 1, 3, C, generator=gen, device=dev).bfloat16())
    conv_w = (torch.randn(C, 4, generator=gen, device=dev) * 0.3).bfloat16()
    proj = torch.randn(rows, stride, generator=gen, device=dev).bfloat16()
    out = torch.empty(rows, HV * V, dtype=torch.bfloat16, device=dev)
    A = torch.zeros(HV, dtype=torch.bfloat16, device=dev)
    w = torch.ones(V, dtype=torch.bfloat16, device=dev)
    slots = torch.arange(rows, device=dev)
    lens = torch.ones(rows, dtype=torch.long, device=dev)
    offs = torch.arange(rows, device=dev)
    stream = torch.cuda.current_stream(dev)
    base = proj.data_ptr()

    def launch(i):
        rc = lib.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, conv_w.data_ptr(),
                                              pools[i % 3].data_ptr(), C, base + 2 * (C + HV * V + HV),
                                              base + 2 * (C + HV * V), stride, A.data_ptr(), A.data_ptr(),
                                              states[i % 3].data_ptr(), state_dtype, rows + 1, slots.data_ptr(),
                                              lens.data_ptr(), offs.data_ptr(), rows, H, HV, K, V, K ** -0.5,
                                              base + 2 * C, stride, w.data_ptr(), 1e-6, out.data_ptr(),
                                              HSG_GDN_BURST_MIN_DEFAULT, stream.cuda_stream)
        assert rc == 0, rc
    for i in range(9):
        launch(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(iters):
        launch(i)
    t1.record(stream)
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / iters
    elem = 4 if state_dtype == 0 else 2
    per_unit = 2 * K * V * elem + 2 * 3 * 3 * K * 2
    per_token = 5 * 256 + 4
    traffic_alg = rows * HV * (per_unit + per_token) + HV * 3 * K * 4 * 2
    gbs = traffic_alg / (us * 1e-6) / 1e9
    return {"kernel": "gdn_step_kernel conv variant (hsg_gdn_conv_slot_step_gated)",
            "shape": f"{rows} rows x 1 token x 16 heads", "avg_us": round(us, 2), "alg_bytes_per_launch": traffic_alg,
            "achieved_gbs": round(gbs, 1)}


def lone_row_rate(torch, lib, tokens=64, iters=20, burst_min=16):
    """The conv + gated GDN slot step (hsg_gdn_conv_slot_step_gated) on one row of ``tokens`` tokens, 16 heads x
    128, fp32 state, every other row of an 8-row grid empty: a mixed tick's critical path when its longest row
    runs on the slot step (the chip otherwise idle). HIP events on the launch stream around ``iters`` launches.
    ``burst_min`` as the entry point's (0: token by token; 16, the engine's: this row in bursts of 8 tokens on
    MFMA)."""
    dev = torch.device("cuda:0")
    N, H, K = 8, 16, 128
    C = 3 * H * K
    stride = C + H * K + 2 * H + 64
    gen = torch.Generator(device=dev).manual_seed(2)
    proj = torch.randn(tokens, stride, generator=gen, device=dev).bfloat16()
    out = torch.empty(tokens, H * K, device=dev, dtype=torch.bfloat16)
    state = torch.randn(N + 1, H, K, K, generator=gen, device=dev) * 0.02
    pool = torch.randn(N + 1, 3, C, generator=gen, device=dev).bfloat16()
    conv_w = (torch.randn(C, 4, generator=gen, device=dev) * 0.3).bfloat16()
    A = torch.zeros(H, dtype=torch.bfloat16, device=dev)
    w = torch.ones(K, dtype=torch.bfloat16, device=dev)
    slots = torch.arange(N, device=dev)
    lens = torch.zeros(N, dtype=torch.long, device=dev)
    lens[0] = tokens
    offs = torch.zeros(N, dtype=torch.long, device=dev)
    stream = torch.cuda.current_stream(dev)
    base = proj.data_ptr()

    def launch():
        rc = lib.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, conv_w.data_ptr(), pool.data_ptr(),
                                              C, base + 2 * (C + H * K + H), base + 2 * (C + H * K), stride,
                                              A.data_ptr(), A.data_ptr(), state.data_ptr(), 0, N + 1,
                                              slots.data_ptr(), lens.data_ptr(), offs.data_ptr(), N, H, H, K, K,
                                              K ** -0.5, base + 2 * C, stride, w.data_ptr(), 1e-6, out.data_ptr(),
                                              burst_min, stream.cuda_stream)
        assert rc == 0, rc
    launch()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(iters):
        launch()
    t1.record(stream)
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / iters
    return {"tokens": tokens, "burst_min": burst_min, "avg_us": round(us, 2), "us_per_token": round(us / tokens, 3)}


def gdn_tick_rate(torch, lib, rows=352, iters=30, seed=5, burst_mins=(0, 8)):
    """The conv + gated GDN slot step (hsg_gdn_conv_slot_step_gated, as the engine runs every GDN layer of a mixed
    tick) on a config-5 tick: 352 rows, chunk lengths 1 (p 0.8), 2-16 (p 0.15), 17-64 (p 0.05), packed longest
    first, 16 heads x 128, fp32 state, for each burst threshold in ``burst_mins``. HIP events on the launch stream
    around ``iters`` launches. Algorithmic bytes: per (row, head) the state and the conv history read and written,
    per (token, head) q, k, v, z in, the output out and a, b, as the roofline leg counts them. Row r is slot r's
    request, the rows packed as the engine packs a step's requests in slot order (longest first, ties in slot
    order), and launch i works on state buffer and conv pool i mod 3, as in the roofline leg."""
    import numpy as np
    dev = torch.device("cuda:0")
    H = HV = 16
    K = V = 128
    C = 3 * H * K
    stride = C + HV * V + 2 * HV
    rng = np.random.default_rng(seed)
    u = rng.random(rows)
    lens_slot = np.where(u < 0.8, 1, np.where(u < 0.95, rng.integers(2, 17, rows), rng.integers(17, 65, rows)))
    order = np.argsort(-lens_slot, kind="stable")   # the engine's packing: longest first, ties in slot order
    lens_h = lens_slot[order].copy()
    T = int(lens_h.sum())
    gen = torch.Generator(device=dev).manual_seed(seed)
    states = [torch.randn(rows + 1, HV, K, V, generator=gen, device=dev) * 0.02 for _ in range(3)]
    pools = [torch.randn(rows + 1, 3, C, generator=gen, device=dev).bfloat16() for _ in range(3)]
    conv_w = (torch.randn(C, 4, generator=gen, device=dev) * 0.3).bfloat16()
    proj = torch.randn(T, stride, generator=gen, device=dev).bfloat16()
    out = torch.empty(T, HV * V, dtype=torch.bfloat16, device=dev)
    A = torch.zeros(HV, dtype=torch.bfloat16, device=dev)
    w = torch.ones(V, dtype=torch.bfloat16, device=dev)
    slots = torch.from_numpy(order).to(dev)
    lens = torch.from_numpy(lens_h).to(dev)
    offs = torch.from_numpy(np.concatenate([[0], np.cumsum(lens_h)[:-1]])).to(dev)
    stream = torch.cuda.current_stream(dev)
    base = proj.data_ptr()
    res = {"rows": rows, "tokens": T, "multi_token_rows": int((lens_h > 1).sum()), "state_buffers": 3}
    alg = rows * HV * (2 * K * V * 4 + 2 * 3 * 3 * K * 2) + T * HV * (5 * 256 + 4) + HV * 3 * K * 4 * 2
    for bm in burst_mins:
        def launch(i):
            rc = lib.hsg_gdn_conv_slot_step_gated(base, stride, 0, H * K, 2 * H * K, conv_w.data_ptr(),
                                                  pools[i % 3].data_ptr(), C, base + 2 * (C + HV * V + HV),
                                                  base + 2 * (C + HV * V), stride, A.data_ptr(), A.data_ptr(),
                                                  states[i % 3].data_ptr(), 0, rows + 1, slots.data_ptr(),
                                                  lens.data_ptr(), offs.data_ptr(), rows, H, HV, K, V, K ** -0.5,
                                                  base + 2 * C, stride, w.data_ptr(), 1e-6, out.data_ptr(), bm,
                                                  stream.cuda_stream)
            assert rc == 0, rc
        for i in range(6):
            launch(i)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(iters):
            launch(i)
        t1.record(stream)
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / iters
        res[f"burst_min_{bm}"] = {"avg_us": round(us, 2), "hbm_frac": round(alg / (us * 1e-6) / 8e12, 3)}
    res["alg_bytes_per_launch"] = alg
    return res


def calibration_copy(torch, dev):
    """Three plain 512 MiB device-to-device copies (512 MiB read + 512 MiB written each): the known-size kernel
    that scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings of the same run into bytes."""
    src = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def measured_traffic(rows, state_dtype):
    """HBM bytes per launch of the GDN slot step at the decode shape, as rocprofv3's FETCH_SIZE and WRITE_SIZE
    counters read it (each scaled by the same counter's reading for a device copy of known size). The counter
    runs cannot happen inside this process, so the figure comes from the committed counter summary of the
    same command; it exists only for the default shape (352 rows, fp32 state), otherwise None."""
    path = os.path.join(ROOT, "profiles", "gdn_step_352x1_counters.md")
    if rows != 352 or state_dtype != 0 or not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def ring_decode_rate(torch, rows=352, iters=50):
    """Decode ring attention (hsg_ring_decode: one fused launch at 4 query heads per kv head) at the 352 x 1-token
    decode shape, HIP events on the launch stream: config 2's ring fills (uniform in [1, 512]) scaled to 352 rows,
    and full rings (the steady state of a live session). Algorithmic bytes: the visible keys and values (n 256
    dims x 2 B x 2), their positions (8 B each), q, gate and out (3 x 16 heads x 512 B), the new key and value read
    and written to the ring (4 kv heads x 512 B x 4). Launch i reads ring set i mod 3 (the rings of every row, 740 MB a
    set), so no launch reads rings the previous one just read from the 256 MB Infinity Cache: in a step each
    attention layer's rings were last read a whole step earlier."""
    from hs_guard.engine.kernels import ring_attention_v8
    from hs_guard.synthetic import ring_decode_inputs
    out = {}
    for name in ("config2_fills", "full_rings"):
        r = ring_decode_inputs(rows=rows)
        if name == "full_rings":
            W = 512
            r["fill"] = torch.full_like(r["fill"], W)
            rp = torch.full_like(r["ring_pos"], -1)
            for i in range(rows):
                st = int(r["starts"][i])
                cols = torch.arange(st - W, st)
                rp[i, cols % W] = cols
            r["ring_pos"] = rp
        d = {k: v.to("cuda:0") for k, v in r.items() if torch.is_tensor(v)}
        rings = [(d["ring_k"], d["ring_v"])] + [(d["ring_k"].clone(), d["ring_v"].clone()) for _ in range(2)]
        stream = torch.cuda.current_stream()

        def run(i):
            rk, rv = rings[i % 3]
            ring_attention_v8(d["q"], rk, rv, d["new_k"], d["value"], d["gate"], d["ring_pos"],
                              d["slots"], d["starts"], d["lens"], 1 / 16, 512, False)
        for i in range(6):
            run(i)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(iters):
            run(i)
        t1.record(stream)
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / iters
        valid = sum(min(int(f), 511) for f in r["fill"])
        alg = valid * 4 * 256 * 2 * 2 + rows * 16 * 256 * 2 * 3 + rows * 4 * 256 * 2 * 2 + valid * 8
        out[name] = {"avg_us": round(us, 2), "alg_bytes_per_launch": alg,
                     "achieved_gbs": round(alg / (us * 1e-6) / 1e9, 1)}
    return out


def ring_tick_rate(torch, rows=352, iters=50, seed=5):
    """The tiled ring attention (hsg_ring_attention with min_len 2: the multi-token rows of a tick; the engine gives
    the single-token rows to hsg_ring_decode) on a config-5 mixed tick: 352 rows, chunk lengths 1 (p 0.8), 2-16
    (p 0.15), 17-64 (p 0.05), packed layout, 16 q / 4 kv heads of 256, full 512-column rings, ring write off (the
    engine's separate ring_write_kernel). HIP events on the launch stream around ``iters`` launches, launch i on
    ring set i mod 3 (the multi-token rows' rings, 147 MB, would otherwise stay in the Infinity Cache). Algorithmic
    bytes per multi-token row and kv head: its ring keys and values (512 x 256 x 2 B x 2) and positions (512 x 8 B),
    and per token its new key and value (2 x 512 B), 4 queries and gates in and 4 outputs out (12 x 512 B)."""
    import numpy as np
    from hs_guard._lib import lib
    L = lib()
    dev = torch.device("cuda:0")
    hq, hkv, D, W = 16, 4, 256, 512
    G = hq // hkv
    rng = np.random.default_rng(seed)
    u = rng.random(rows)
    lens_h = np.where(u < 0.8, 1, np.where(u < 0.95, rng.integers(2, 17, rows), rng.integers(17, 65, rows)))
    lens_h = np.sort(lens_h)[::-1].copy()                  # the engine packs rows longest first
    T = int(lens_h.sum())
    offs_h = np.concatenate([[0], np.cumsum(lens_h)[:-1]])
    gen = torch.Generator(device=dev).manual_seed(seed)
    att_in = hq * 2 * D + 2 * hkv * D                     # projection row: q | gate interleaved per head, k, v
    proj = torch.randn(T, att_in, generator=gen, device=dev).bfloat16()
    q = torch.randn(T, hq * D, generator=gen, device=dev).bfloat16()
    k = torch.randn(T, hkv * D, generator=gen, device=dev).bfloat16()
    ring_k = torch.randn(rows + 1, hkv, W + 1, D, generator=gen, device=dev).bfloat16()
    ring_v = torch.randn(rows + 1, hkv, W + 1, D, generator=gen, device=dev).bfloat16()
    starts_h = rng.integers(W, 4 * W, rows)
    ring_pos = torch.full((rows + 1, W + 1), -1, dtype=torch.long)
    for i in range(rows):
        cols = np.arange(starts_h[i] - W, starts_h[i])
        ring_pos[i, cols % W] = torch.from_numpy(cols)
    ring_pos = ring_pos.to(dev)
    slots = torch.arange(rows, device=dev)
    starts = torch.from_numpy(starts_h).to(dev)
    lens = torch.from_numpy(lens_h).to(dev)
    offs = torch.from_numpy(offs_h).to(dev)
    out = torch.empty(T, hq * D, dtype=torch.bfloat16, device=dev)
    base = proj.data_ptr()
    stream = torch.cuda.current_stream(dev)

    rings = [(ring_k, ring_v)] + [(ring_k.clone(), ring_v.clone()) for _ in range(2)]

    def run(i):
        rk, rv = rings[i % 3]
        rc = L.hsg_ring_attention(q.data_ptr(), 0, hq * D, G * D, D, rk.data_ptr(), rv.data_ptr(), rows + 1,
                                  W, k.data_ptr(), 0, hkv * D, D, base + 2 * (hq * 2 * D + hkv * D), 0, att_in, D,
                                  base, 0, att_in, G * 2 * D, 2 * D, D, ring_pos.data_ptr(), slots.data_ptr(),
                                  starts.data_ptr(), lens.data_ptr(), offs.data_ptr(), rows, 64, hkv, G, D, D ** -0.5,
                                  0, 2, out.data_ptr(), 0, hq * D, G * D, D, stream.cuda_stream)
        assert rc == 0, rc
    for i in range(6):
        run(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(iters):
        run(i)
    t1.record(stream)
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / iters
    multi = lens_h[lens_h >= 2]
    alg = int(len(multi) * hkv * (W * D * 2 * 2 + W * 8) + int(multi.sum()) * hkv * (2 * 512 + 12 * 512))
    return {"kernel": "ring_attn_mfma_kernel (hsg_ring_attention, min_len 2)", "rows": int(len(multi)),
            "tokens": int(multi.sum()), "avg_us": round(us, 2), "alg_bytes_per_launch": alg,
            "achieved_gbs": round(alg / (us * 1e-6) / 1e9, 1), "hbm_frac": round(alg / (us * 1e-6) / 8e12, 3)}


def chunk_prefill_rate(torch, iters=10):
    """Config 4 on hsg_gdn_chunk_prefill: 16 rows of 512/2048/8000 tokens (53,312 tokens, 833 chunks of 64),
    16 heads x 128, fp32 state; HIP events on the launch stream. Algorithmic work per chunk-head
    2C^2(3dk+2dv) + 6C dk dv + (2/3)C^3 = 11,709,099 FLOP (C=64, dk=dv=128); algorithmic bytes = q, k, v in
    + o out (4 x 256 B) + a, b (4 B) per token-head + the state read and written once per row-head."""
    from hs_guard.engine.kernels import gdn_chunk_prefill
    from hs_guard.synthetic import chunk_prefill_inputs
    H, K = 16, 128
    from hs_guard._lib import lib
    inp = chunk_prefill_inputs(rows=16)
    d = {k: (v.to("cuda:0") if torch.is_tensor(v) else v) for k, v in inp.items()}
    slots = torch.arange(16, device="cuda:0")
    stream = torch.cuda.current_stream()
    max_len = int(inp["lens"].max())
    ws = torch.empty(lib().hsg_gdn_chunk_workspace_bytes(16, max_len, H), dtype=torch.uint8, device="cuda:0")

    def run():
        gdn_chunk_prefill(d["packed"], H * K, H, K, H, K, d["a"], d["b"], d["A_log"], d["dt_bias"], d["state0"],
                          slots, d["lens"], d["offsets"], max_len=max_len, workspace=ws)
    for _ in range(2):
        run()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(iters):
        run()
    t1.record(stream)
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / iters
    T = int(inp["lens"].sum())
    chunks = int(((inp["lens"] + 63) // 64).sum())
    flop = 11709099 * chunks * H
    alg_bytes = T * H * (4 * 256 + 4) + 16 * H * K * K * 4 * 2
    tflops = flop / (us * 1e-6) / 1e12
    ridge = min(MFMA_BF16_PEAK_TFLOPS, flop / alg_bytes * HBM_PEAK_GBS / 1e3)
    return {"avg_us": round(us, 1), "tokens": T, "chunks": chunks, "alg_flop": flop, "alg_bytes": alg_bytes,
            "tflops": round(tflops, 1), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "roof_tflops": round(ridge, 1), "roof_frac": round(tflops / ridge, 4)}


def host_phases(torch, eng, load, steps=100):
    """Where a step_packed tick's host-to-host time goes, on the engine's own calls in the order step_packed makes
    them (requests checked and packed by hs_guard._hostpack, inputs copied, graph replayed, outputs copied, wait,
    padded result): the median per phase in microseconds, and the graph's GPU time between HIP events on the
    launch stream. Mixed config-5 ticks without resets; the engine's graphs are already captured."""
    import numpy as np
    from hs_guard import _hostpack
    from hs_guard.engine.slot_engine import bucket
    names = ("pack", "input_copy", "graph_launch_call", "output_copy", "wait", "result", "total")
    ph = {k: [] for k in names}
    gpu = []
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.inference_mode():
        for i in range(steps):
            req = load.step_requests()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            n, total, max_len = _hostpack.scan(req, eng.max_slots, eng.cfg.vocab_size)
            nb, tb = bucket(n, eng.session_buckets), bucket(total, eng.token_buckets)
            graph, inp, probs, host_in, host_np, host_out, out_np = eng._static(nb, tb)
            lens, offs, slots = (np.empty(n, dtype=np.int64) for _ in range(3))
            _hostpack.fill(req, eng.length, nb, tb, eng.max_slots, eng.cfg.vocab_size, host_np, lens, offs, slots)
            t1 = time.perf_counter()
            inp["all"].copy_(host_in, non_blocking=True)
            t2 = time.perf_counter()
            e0.record(st)
            graph.replay()
            e1.record(st)
            t3 = time.perf_counter()
            host_out.copy_(probs, non_blocking=True)
            t4 = time.perf_counter()
            st.synchronize()
            t5 = time.perf_counter()
            eng.length[slots] += lens
            lb = bucket(max_len, (1, 2, 4, 8, 16, 32, 64))
            out = np.empty((len(eng.roles), n, lb, 3), dtype=np.float32)
            _hostpack.scatter_padded(out_np, len(eng.roles), tb, lens, offs, lb, out)
            t6 = time.perf_counter()
            for k, a, b in zip(names, (t0, t1, t2, t3, t4, t5, t0), (t1, t2, t3, t4, t5, t6, t6)):
                ph[k].append((b - a) * 1e6)
            gpu.append(e0.elapsed_time(e1) * 1e3)
    out = {k: round(float(np.median(v)), 1) for k, v in ph.items()}
    out["graph_gpu"] = round(float(np.median(gpu)), 1)
    out["steps"] = steps
    return out


def config5_leg(torch, cfg_name="v10", slots=352, steps=60, warmup=10, seed=0, state_dtype="float32", reset_p=0.0,
                model=None):
    """The config-5 mixed load on a second engine, reported apart from the headline: ``cfg_name`` "v10" is the
    released geometry (8 q / 2 kv attention heads, vocab 248,320; 754.5M parameters, docs/evaluation.json:623) with
    its own random-init weights; "baseline" is the headline's geometry (pass its ``model`` to share the weights), for
    another state storage (``state_dtype`` "float16": the reference StreamingGuard's, src/hs_guard/runtime.py:157).
    Contexts U{512, 2048, 8000} prefilled untimed, ``steps`` timed mixed steps through step_packed, resets with
    probability ``reset_p`` re-prefilled untimed."""
    from hs_guard.engine.slot_engine import SlotStreamEngine
    from hs_guard.model import GuardConfig, GuardModel
    from hs_guard.synthetic import MixedServingLoad
    dev = torch.device("cuda:0")
    cfg = getattr(GuardConfig, cfg_name)()
    own = model is None
    if own:
        model = GuardModel.random(cfg, seed=seed, device=dev, gen_device=dev)
    eng = SlotStreamEngine(model, slots, state_dtype=state_dtype)
    load = MixedServingLoad(slots=slots, vocab=cfg.vocab_size, seed=seed + 11, reset_p=reset_p)
    eng.step([(s, load.context()) for s in range(slots)])
    mean, sd = 4.175 * slots, 9.48 * slots ** 0.5
    eng.prepare(slots, range(slots, int(mean + 8 * sd) + 1, 16))

    def reprefill():
        gone = load.resets()
        if gone:
            eng.reset(gone)
            eng.step([(s, load.context()) for s in gone])
    for _ in range(warmup):
        eng.step(load.step_requests())
        reprefill()
    times, tokens = [], 0
    for _ in range(steps):
        req = load.step_requests()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.step_packed(req)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
        tokens += sum(len(ids) for _, ids in req)
        reprefill()
    geometry = {"v10": "v10: hidden 1024, 24 layers 3 GDN:1 attn, GDN 16x128, attn 8q/2kv/256 window 512, MLP 3584, "
                       "vocab 248320",
                "baseline": "baseline (the headline's): attn 16q/4kv/256, vocab 151936"}[cfg_name]
    out = {"geometry": geometry, "params": model.num_parameters(), "slots": slots, "state_dtype": state_dtype,
           "reset_p": reset_p, "steps": steps, "tokens_per_s": round(tokens / (sum(times) / 1e3), 1),
           "p50": round(percentile(times, 50), 3), "p95": round(percentile(times, 95), 3)}
    del eng
    if own:
        del model
    torch.cuda.empty_cache()
    return out


def cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, cfg, seed=0, slots=352, steps=10, decode_steps=20):
    """CPU baseline: oracle/torch_cpu.py, the PyTorch float32 restatement of the same step, on this host's cores
    (torch threads = this job's CPU share: OMP_NUM_THREADS, else os.cpu_count()). The reference has no CPU path.
    Legs:
    * config 5 (the headline): ``slots`` slots, initial contexts U{512, 2048, 8000} (the pools filled as after
      them: state, conv history and rings random, ring positions and lengths exact; a step's work does not depend
      on the pools' values), one warm-up step, then ``steps`` timed mixed steps of config 5's chunk sizes.
      tokens/s over those steps; the 2,000-step run of the config is extrapolated from the per-step time;
    * config 3: 64 slots x 1 token after 512-token contexts, ``decode_steps`` steps;
    * config 1: the GDN step alone, 16 slots x 1 token x 64 sequential steps, 16 heads x 128, fp32 state;
    * config 2: one decode step of the window attention with its ring write, 64 slots, 16q / 4kv / 256, W = 512;
    * config 4: the chunk form over 16 rows of 512 / 2048 / 8000 tokens (53,312 tokens), 16 heads x 128."""
    import numpy as np
    import torch
    from hs_guard.synthetic import MixedServingLoad, chunk_prefill_inputs, gdn_step_inputs, ring_decode_inputs
    from oracle.torch_cpu import TorchStream, gdn_chunk_torch, gdn_step_torch, ring_decode_torch
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    legs = {}
    # ---- config 5 ----
    load = MixedServingLoad(slots=slots, vocab=cfg.vocab_size, seed=seed + 7)
    lengths = [int(load.rng.choice(load.contexts)) for _ in range(slots)]
    ts = TorchStream(model.weights, cfg, slots)
    ts.fill_synthetic(lengths, seed=seed)
    ts.tick(load.step_requests())
    tokens, secs = 0, 0.0
    for _ in range(steps):
        req = load.step_requests()
        t0 = time.perf_counter()
        ts.tick(req)
        secs += time.perf_counter() - t0
        tokens += sum(len(ids) for _, ids in req)
    legs["config5"] = {"steps": steps, "tokens": tokens, "s_per_step": round(secs / steps, 3),
                       "tokens_per_s": round(tokens / secs, 1),
                       "extrapolated_2000_steps_s": round(secs / steps * 2000, 1)}
    del ts
    # ---- config 3 ----
    ts = TorchStream(model.weights, cfg, 64)
    ts.fill_synthetic([512] * 64, seed=seed + 1)
    rng = np.random.default_rng(seed)
    ts.tick([(s, [int(rng.integers(0, cfg.vocab_size))]) for s in range(64)])
    t0 = time.perf_counter()
    for _ in range(decode_steps):
        ts.tick([(s, [int(rng.integers(0, cfg.vocab_size))]) for s in range(64)])
    dt = time.perf_counter() - t0
    legs["config3"] = {"steps": decode_steps, "ms_per_step": round(dt / decode_steps * 1e3, 2),
                       "tokens_per_s": round(64 * decode_steps / dt, 1)}
    del ts
    # ---- config 1 ----
    inp = gdn_step_inputs(slots=16, steps=64)
    state = inp["state0"].float().clone()
    A_log, dt_b = inp["A_log"].float(), inp["dt_bias"].float()
    sl = torch.arange(16)
    t0 = time.perf_counter()
    for t in range(64):
        gdn_step_torch(inp["packed"][t, :, 0].float(), 16 * 128, 16, 128, 16, 128, inp["a"][t, :, 0].float(),
                       inp["b"][t, :, 0].float(), A_log, dt_b, state, sl)
    dt = time.perf_counter() - t0
    legs["config1"] = {"steps": 64, "ms_per_step": round(dt / 64 * 1e3, 3),
                       "gbs": round(33948672 * 64 / dt / 1e9, 2)}
    # ---- config 2 ----
    r = ring_decode_inputs(rows=64)
    f = {k: (v.float() if torch.is_tensor(v) and v.is_floating_point() else v) for k, v in r.items()}
    gate = f["gate"].reshape(64, 16, 512)[..., 256:].reshape(64, 4, 4, 256)
    times = []
    for _ in range(4):
        rk, rv = f["ring_k"].clone(), f["ring_v"].clone()
        t0 = time.perf_counter()
        ring_decode_torch(f["q"], rk, rv, f["new_k"][:, :, 0], f["new_v"][:, :, 0], gate, r["ring_pos"], r["slots"],
                          r["starts"], 1 / 16, 512)
        times.append(time.perf_counter() - t0)
    legs["config2"] = {"ms": round(min(times[1:]) * 1e3, 2)}
    # ---- config 4 ----
    inp = chunk_prefill_inputs(rows=16)
    t_all = 0.0
    for L in (512, 2048, 8000):
        rows = [i for i in range(16) if int(inp["lens"][i]) == L]
        pk = torch.stack([inp["packed"][int(inp["offsets"][i]):int(inp["offsets"][i]) + L].float() for i in rows])
        a = torch.stack([inp["a"][int(inp["offsets"][i]):int(inp["offsets"][i]) + L].float() for i in rows])
        b = torch.stack([inp["b"][int(inp["offsets"][i]):int(inp["offsets"][i]) + L].float() for i in rows])
        n = len(rows)
        q = pk[..., :2048].reshape(n, L, 16, 128)
        k = pk[..., 2048:4096].reshape(n, L, 16, 128)
        v = pk[..., 4096:].reshape(n, L, 16, 128)
        t0 = time.perf_counter()
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * 128 ** -0.5
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        g = -torch.nn.functional.softplus(a, threshold=20.0)
        flat = lambda x: x.transpose(1, 2).reshape(n * 16, L, -1)
        S = torch.zeros(n * 16, 128, 128)
        gdn_chunk_torch(flat(q), flat(k), flat(v), g.transpose(1, 2).reshape(n * 16, L),
                        torch.sigmoid(b).transpose(1, 2).reshape(n * 16, L), S)
        t_all += time.perf_counter() - t0
    legs["config4"] = {"ms": round(t_all * 1e3, 1), "tflops": round(156058871472 / t_all / 1e12, 3)}
    c5 = legs["config5"]
    return {"value": c5["tokens_per_s"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle/torch_cpu.py (PyTorch fp32 restatement of the step), config 5 at {slots} slots: "
                      f"{steps} timed mixed steps ({c5['tokens']} tokens, {c5['s_per_step']} s/step; 2,000 steps "
                      f"extrapolated to {c5['extrapolated_2000_steps_s']} s) after contexts emulated in the pools",
            "cpu_model": cpu_model_name(), "os_cpu_count": os.cpu_count(), "configs": legs}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--slots", type=int, default=352)
    ap.add_argument("--state-dtype", default="float32", choices=("float32", "float16"))
    ap.add_argument("--contexts", default="512,2048,8000")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant-kernel measurement (the command profiled under rocprofv3)")
    ap.add_argument("--chunk-only", action="store_true",
                    help="only the config-4 chunked-prefill measurement (profiled under rocprofv3)")
    ap.add_argument("--gdn-tick-only", action="store_true",
                    help="only the GDN slot step on a config-5 tick at several burst thresholds, and a lone 64-token "
                         "row")
    ap.add_argument("--ring-tick-only", action="store_true",
                    help="only the tiled ring attention on a config-5 mixed tick's multi-token rows")
    ap.add_argument("--ring-only", action="store_true",
                    help="only the 352 x 1-token split-K ring decode measurement (profiled under rocprofv3)")
    ap.add_argument("--lone-row-only", action="store_true",
                    help="only the GDN slot step on one 64-token row at --gdn-burst-min (profiled under rocprofv3 "
                         "--pmc)")
    ap.add_argument("--single-token-only", action="store_true",
                    help="only the single-token step latency: slot 0 of the --slots engine after a 512-token context, "
                         "--warmup + --steps timed steps (the command whose kernel statistics give the single-token "
                         "breakdown)")
    ap.add_argument("--mixed-only", action="store_true",
                    help="only the prefill and the mixed steps (no kernel legs, decode legs, context sweep or CPU "
                         "baseline): the command whose kernel statistics give the per-step kernel breakdown")
    ap.add_argument("--reset-p", type=float, default=0.01, help="per-slot reset probability after each step")
    ap.add_argument("--chunk-min-tokens", type=int, default=None,
                    help="SlotStreamEngine's chunk_min_tokens (default: the engine's; 0 puts every GDN row on the "
                         "slot step)")
    ap.add_argument("--gdn-burst-min", type=int, default=None,
                    help="SlotStreamEngine's gdn_burst_min (default: the engine's): slot-step rows of at least this "
                         "many tokens run in 8-token bursts on MFMA (0: every row token by token)")
    ap.add_argument("--sweep-steps", type=int, default=60,
                    help="timed mixed steps per initial-context length in the per-context latency sweep (0: skip)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU: the streaming step shards by slot with no exchange between GPUs, "
              f"and this build measures one GPU's share (asked for --gpus {args.gpus}, WORLD_SIZE {world}).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from hs_guard._lib import HSG_GDN_BURST_MIN_DEFAULT, lib
    from hs_guard.model import GuardConfig, GuardModel
    from hs_guard.runtime import StreamingGuard, random_metadata
    from hs_guard.synthetic import MixedServingLoad

    dev = torch.device("cuda:0")
    log(f"device {torch.cuda.get_device_name(0)}")
    state_code = 0 if args.state_dtype == "float32" else 1
    if args.lone_row_only:   # one threshold per run, so counters of one run describe one path
        bm = HSG_GDN_BURST_MIN_DEFAULT if args.gdn_burst_min is None else args.gdn_burst_min
        print(json.dumps({"gdn_lone_row_64": lone_row_rate(torch, lib(), burst_min=bm)}), flush=True)
        return
    if args.gdn_tick_only:
        print(json.dumps({"gdn_tick": gdn_tick_rate(torch, lib(), rows=args.slots, burst_mins=(0, 8, 16, 32)),
                          "gdn_lone_row_64": lone_row_rate(torch, lib()),
                          "gdn_lone_row_64_token_path": lone_row_rate(torch, lib(), burst_min=0)}), flush=True)
        return
    if args.ring_tick_only:
        print(json.dumps({"ring_attn_tick": ring_tick_rate(torch, rows=args.slots)}), flush=True)
        return
    if args.chunk_only or args.ring_only:
        leg = chunk_prefill_rate(torch) if args.chunk_only else ring_decode_rate(torch, rows=args.slots)
        calibration_copy(torch, dev)
        print(json.dumps({"chunk_prefill_cfg4" if args.chunk_only else "ring_decode_352": leg,
                          "calibration_copy_bytes": 512 << 20}), flush=True)
        return
    if args.mixed_only:
        args.sweep_steps = 0
        args.no_cpu_baseline = True
        roof = ring = chunk = lone = tick = None
    else:
        roof = gdn_roofline(torch, lib(), rows=args.slots, state_dtype=state_code)
        log(f"GDN roofline {roof}")
    if args.roofline_only:
        calibration_copy(torch, dev)
        print(json.dumps({"roofline_only": roof, "calibration_copy_bytes": 512 << 20}), flush=True)
        return
    if not args.mixed_only:
        ring = ring_decode_rate(torch, rows=args.slots)
        log(f"ring decode {ring}")
        tick = ring_tick_rate(torch, rows=args.slots)
        log(f"tiled ring attention, mixed tick {tick}")
        chunk = chunk_prefill_rate(torch)
        log(f"chunk prefill config 4 {chunk}")
        lone = lone_row_rate(torch, lib(), burst_min=(HSG_GDN_BURST_MIN_DEFAULT if args.gdn_burst_min is None
                                                      else args.gdn_burst_min))
        log(f"GDN slot step, one 64-token row {lone}")

    cfg = GuardConfig.baseline()
    t0 = time.time()
    model = GuardModel.random(cfg, seed=args.seed, device=dev, gen_device=dev)
    log(f"model {model.num_parameters() / 1e6:.1f}M params in {time.time() - t0:.1f}s")
    # the public API object (src/hs_guard/runtime.py:148-174); the headline times its engine's step_packed, the
    # serving backend's call, and the guard_step leg times guard.step() itself
    guard = StreamingGuard(model, random_metadata(), max_slots=args.slots, state_dtype=args.state_dtype)
    eng = guard.engine
    if args.chunk_min_tokens is not None:
        eng.chunk_min_tokens = args.chunk_min_tokens   # before the first tick: every graph is captured with it
    if args.gdn_burst_min is not None:
        eng.gdn_burst_min = args.gdn_burst_min   # before the first tick, as chunk_min_tokens
    if args.single_token_only:
        rng1 = np.random.default_rng(args.seed + 1)
        eng.step([(0, rng1.integers(0, cfg.vocab_size, 512).tolist())])
        one = []
        for i in range(args.warmup + args.steps):
            req = [(0, [int(rng1.integers(0, cfg.vocab_size))])]
            torch.cuda.synchronize()
            t = time.perf_counter()
            eng.step_packed(req)
            torch.cuda.synchronize()
            if i >= args.warmup:
                one.append((time.perf_counter() - t) * 1e3)
        print(json.dumps({"single_token_ms": {"p50": round(percentile(one, 50), 3),
                                              "p95": round(percentile(one, 95), 3)},
                          "slots": args.slots, "context": 512, "steps": len(one)}), flush=True)
        return
    load = MixedServingLoad(slots=args.slots, vocab=cfg.vocab_size, seed=args.seed,
                            contexts=tuple(int(x) for x in args.contexts.split(",")), reset_p=args.reset_p)

    # ---- initial contexts through step() (outside the timed steps): first cold (every tick shape captured
    # into its graph on first use), then, into reset slots, the same lengths with fresh token ids (warm) ----
    t0 = time.perf_counter()
    ctx = [(s, load.context()) for s in range(args.slots)]
    eng.step(ctx)
    torch.cuda.synchronize()
    cold_s = time.perf_counter() - t0
    captures = eng.stats["captures"]
    ctx_tokens = sum(len(c) for _, c in ctx)
    log(f"prefilled {ctx_tokens} context tokens in {cold_s:.2f}s ({captures} graphs)")
    rng_ctx = np.random.default_rng(args.seed + 3)
    ctx = [(s, rng_ctx.integers(0, cfg.vocab_size, len(c)).tolist()) for s, c in ctx]
    eng.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.step(ctx)
    torch.cuda.synchronize()
    warm_s = time.perf_counter() - t0
    prefill = {"contexts": args.slots, "tokens": ctx_tokens, "ticks": max(-(-len(c) // eng.max_tick_tokens)
                                                                          for _, c in ctx),
               "cold_s": round(cold_s, 3), "graphs_captured": captures, "warm_s": round(warm_s, 3),
               "warm_tokens_per_s": round(ctx_tokens / warm_s, 1), "chunk_min_tokens": eng.chunk_min_tokens}
    log(f"prefill {prefill}")

    def reprefill(slots):
        if slots:
            eng.reset(slots)
            eng.step([(s, load.context()) for s in slots])

    # ---- warm-up + timed mixed steps ----
    # graphs for every token bucket a mixed tick can plausibly hit (mean 4.175 tok/slot, sd 9.5 per slot),
    # so no capture lands inside a timed step
    t0 = time.time()
    mean, sd = 4.175 * args.slots, 9.48 * args.slots ** 0.5
    eng.prepare(args.slots, range(args.slots, int(mean + 8 * sd) + 1, 16))
    torch.cuda.synchronize()
    log(f"{eng.stats['captures']} graphs captured ({time.time() - t0:.1f}s)")
    for i in range(args.warmup):
        eng.step(load.step_requests())
        reprefill(load.resets())
    torch.cuda.synchronize()
    # the serving loop's own garbage stays collectable; the long-lived objects of the setup (torch, the model,
    # the engine) are moved out of the collector's scans, as a long-running server process would
    gc.collect()
    gc.freeze()
    log("warm-up done")
    times, tokens, step_tokens = [], 0, []
    for i in range(args.steps):
        req = load.step_requests()
        caps = eng.stats["captures"]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.step_packed(req)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        step_tokens.append(sum(len(ids) for _, ids in req))
        tokens += step_tokens[-1]
        if eng.stats["captures"] != caps or times[-1] > 0.05:
            log(f"step {i}: {times[-1] * 1e3:.1f} ms, {eng.stats['captures'] - caps} graph captures, "
                f"{len(req)} rows, max chunk {max(len(ids) for _, ids in req)}")
        caps = eng.stats["captures"]
        reprefill(load.resets())
        if eng.stats["captures"] != caps:
            log(f"after step {i}: re-prefill captured {eng.stats['captures'] - caps} graphs")
        if (i + 1) % 50 == 0:
            log(f"step {i + 1}/{args.steps}: {tokens / sum(times):.0f} tok/s")
    total = sum(times)
    value = tokens / total
    slow = sorted(range(len(times)), key=lambda i: -times[i])[:3]
    log("slowest steps: " + ", ".join(f"#{i} {times[i] * 1e3:.1f} ms ({step_tokens[i]} tokens)" for i in slow))
    step_ms = [t * 1e3 for t in times]
    # the same mixed load through step() (StreamingGuard's call: one CPU tensor per request and role), 60 steps
    api_t, api_tok = [], 0
    for i in range(60):
        req = load.step_requests()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.step(req)
        torch.cuda.synchronize()
        api_t.append(time.perf_counter() - t0)
        api_tok += sum(len(ids) for _, ids in req)
        reprefill(load.resets())
    api_step = {"steps": len(api_t), "tokens_per_s": round(api_tok / sum(api_t), 1),
                "p50": round(percentile([t * 1e3 for t in api_t], 50), 3),
                "p95": round(percentile([t * 1e3 for t in api_t], 95), 3)}
    log(f"step() leg {api_step}")
    # the same load through StreamingGuard.step() (the API the north star names): the reference's per-id checks,
    # the engine's step(), then one record per request with its cut scores 1 - p(safe) as a Python list
    g_t, g_tok = [], 0
    for i in range(60):
        req = load.step_requests()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        guard.step(req, role="assistant")
        g_t.append(time.perf_counter() - t0)
        g_tok += sum(len(ids) for _, ids in req)
        reprefill(load.resets())
    guard_step = {"steps": len(g_t), "tokens_per_s": round(g_tok / sum(g_t), 1),
                  "p50": round(percentile([t * 1e3 for t in g_t], 50), 3),
                  "p95": round(percentile([t * 1e3 for t in g_t], 95), 3)}
    log(f"StreamingGuard.step() leg {guard_step}")
    phases = host_phases(torch, eng, MixedServingLoad(slots=args.slots, vocab=cfg.vocab_size, seed=args.seed + 3,
                                                      reset_p=0.0))
    log(f"host phases of a tick (us) {phases}")
    if args.mixed_only:
        print(json.dumps({"mixed_only": True, "value": round(value, 1), "unit": "tokens/s", "steps": args.steps,
                          "prefill_352_contexts": prefill,
                          "tokens": tokens, "ms_per_step": round(total / args.steps * 1e3, 4),
                          "latency_ms": {"p50": round(percentile(step_ms, 50), 3),
                                         "p95": round(percentile(step_ms, 95), 3)}, "api_step": api_step,
                          "guard_step": guard_step, "host_phases_us": phases}),
              flush=True)
        return

    # ---- per-context latency: every slot restarted with one initial-context length, then timed mixed steps
    # (resets re-prefilled at that length, untimed) ----
    by_context = {}
    if args.sweep_steps > 0:
        for c in (512, 2048, 8000):
            t0 = time.time()
            ctx_load = MixedServingLoad(slots=args.slots, vocab=cfg.vocab_size, seed=args.seed + c, contexts=(c,),
                                        reset_p=args.reset_p)
            eng.reset()
            eng.step([(s, ctx_load.context()) for s in range(args.slots)])
            torch.cuda.synchronize()
            prefill_s = time.time() - t0
            ts, toks = [], 0
            for i in range(args.sweep_steps + 5):
                req = ctx_load.step_requests()
                torch.cuda.synchronize()
                t = time.perf_counter()
                eng.step_packed(req)
                torch.cuda.synchronize()
                if i >= 5:
                    ts.append((time.perf_counter() - t) * 1e3)
                    toks += sum(len(ids) for _, ids in req)
                gone = ctx_load.resets()
                if gone:
                    eng.reset(gone)
                    eng.step([(s, ctx_load.context()) for s in gone])
            by_context[str(c)] = {"steps": len(ts), "tokens_per_s": round(toks / (sum(ts) / 1e3), 1),
                                  "p50": round(percentile(ts, 50), 3), "p95": round(percentile(ts, 95), 3)}
            log(f"context {c}: {by_context[str(c)]} (prefill {prefill_s:.1f}s)")

    # ---- pure decode: 352 x 1 token, and 1 slot x 1 token (20 warm-up + 200 measured) ----
    def timed(make, n=200, warm=20):
        out = []
        for i in range(n + warm):
            req = make()
            torch.cuda.synchronize()
            t = time.perf_counter()
            eng.step_packed(req)
            torch.cuda.synchronize()
            if i >= warm:
                out.append((time.perf_counter() - t) * 1e3)
        return out
    rng = np.random.default_rng(args.seed + 1)
    dec = timed(lambda: [(s, [int(rng.integers(0, cfg.vocab_size))]) for s in range(args.slots)])
    one = timed(lambda: [(0, [int(rng.integers(0, cfg.vocab_size))])])
    log(f"decode 352x1 p50 {percentile(dec, 50):.3f} ms; single-token p50 {percentile(one, 50):.3f} ms")

    # ---- complete-message scorer (one whole forward) on an 8000-token message ----
    from hs_guard.engine.whole import WholeSequenceScorer
    scorer = WholeSequenceScorer(model, shared=eng)
    msg = np.random.default_rng(args.seed + 2).integers(0, cfg.vocab_size, 8000).tolist()
    scorer.forward(msg)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        scorer.forward(msg)
    torch.cuda.synchronize()
    whole_ms = (time.perf_counter() - t0) / 3 * 1e3
    log(f"complete-message scorer, 8000 tokens: {whole_ms:.1f} ms")

    del scorer
    # the headline load with the reference StreamingGuard's fp16 state storage, on the same weights (a second
    # engine; the headline's is left as it is)
    other = "float16" if args.state_dtype == "float32" else "float32"
    state_leg = config5_leg(torch, "baseline", slots=args.slots, steps=100, seed=args.seed, state_dtype=other,
                            reset_p=args.reset_p, model=model)
    log(f"config 5 at {other} state {state_leg}")
    v10 = config5_leg(torch, "v10", slots=args.slots, seed=args.seed, state_dtype=args.state_dtype)
    log(f"v10 geometry {v10}")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(model, cfg, seed=args.seed)
        log(f"cpu baseline {cpu} in {time.time() - t0:.1f}s")

    result = {
        "metric": "stream tokens/s @352 slots + p50/p95 single-token step latency (ms)",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REF_L20["min_tokens_per_s_352"], 3),
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0,0.02), uniform token ids)",
        "config": {"workload": "config5 mixed serving: 352 slots, chunks {1 p.8, 2-16 p.15, 17-64 p.05}, contexts "
                               "U{512,2048,8000} prefilled untimed, resets p=0.01 re-prefilled untimed, hipGraph",
                   "slots": args.slots, "state_dtype": args.state_dtype, "tokens": tokens,
                   "geometry": "hidden 1024, 24 layers 3 GDN:1 attn, GDN 16x128, attn 16q/4kv/256 window 512, "
                               "MLP 3584, vocab 151936", "parallelism": "none (1 GPU)"},
        "latency_ms": {"p50": round(percentile(step_ms, 50), 3), "p95": round(percentile(step_ms, 95), 3),
                       "max": round(max(step_ms), 3)},
        "latency_by_context_ms": by_context,
        "api_step": api_step,
        "guard_step": guard_step,
        "host_phases_us": phases,
        "decode_352x1_ms": {"p50": round(percentile(dec, 50), 3), "p95": round(percentile(dec, 95), 3),
                            "tokens_per_s": round(args.slots / (np.mean(dec) / 1e3), 1)},
        "single_token_ms": {"p50": round(percentile(one, 50), 3), "p95": round(percentile(one, 95), 3)},
        "reference_l20": REF_L20,
        "roofline": {"bound": "hbm", "achieved": roof["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(roof["achieved_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.slots, state_code),
                     "kernel": roof["kernel"], "shape": roof["shape"], "avg_us": roof["avg_us"],
                     "alg_bytes_per_launch": roof["alg_bytes_per_launch"]},
        "ring_decode_352": ring,
        "ring_attn_tick": tick,
        "chunk_prefill_cfg4": chunk,
        "gdn_lone_row_64": lone,
        "prefill_352_contexts": prefill,
        "complete_message_8000": {"ms": round(whole_ms, 2), "tokens_per_s": round(8000 / whole_ms * 1e3, 1)},
        f"config5_{other}_state": state_leg,
        "v10_geometry": v10,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
