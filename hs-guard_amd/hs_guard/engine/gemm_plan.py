"""Deterministic GEMM plans for the engine's projections (hsg_gemm_bf16).

torch.mm runs hipBLASLt's first heuristic candidate. Faster solutions exist for the step's shapes, but choosing
them by timing at start-up picks different solutions in different processes, and solutions differ in
accumulation order, so results would change from run to run. The choice is made once instead, by ``tune`` on an
MI355X, and committed as ``gemm_plans.json``: per (token bucket M, N, K), a hipBLASLt solution index, valid for
the hipBLASLt version recorded with it. The engine looks every product up in that table (``GemmPlans.index``);
shapes the table lacks, or a different hipBLASLt, get index -1 (the heuristic's first candidate).

Regenerate the table on the GPU, from the repository root:

    python -m hs_guard.engine.gemm_plan --out hs-guard_amd/hs_guard/engine/gemm_plans.json

(with ``hs-guard_amd`` on ``PYTHONPATH``).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

from .._lib import lib

PLAN_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_plans.json")
WORKSPACE_BYTES = 32 << 20     # hipBLASLt workspace the engine allocates for these products


class GemmPlans:
    """The committed solution table, keyed by (M, N, K)."""

    def __init__(self, table=None, version=None):
        self.table = dict(table or {})
        self.version = version

    @classmethod
    def load(cls, path=PLAN_PATH):
        """The table at ``path`` if it was generated with the hipBLASLt this process runs, else an empty one."""
        if not os.path.exists(path):
            return cls()
        with open(path) as f:
            data = json.load(f)
        version = int(data.get("blas_version", -1))
        if version != lib().hsg_gemm_blas_version():
            return cls(version=version)
        table = {tuple(int(x) for x in key.split(",")): int(v["index"]) for key, v in data["plans"].items()}
        return cls(table, version)

    def index(self, M, N, K):
        return self.table.get((int(M), int(N), int(K)), -1)

    def drop(self, M, N, K):
        """Forget the entry of (M, N, K): the running hipBLASLt rejected its solution (hsg_gemm_bf16 returned
        HSG_ERR_SHAPE), so the product falls back to the heuristic's first candidate from now on."""
        return self.table.pop((int(M), int(N), int(K)), None)


def engine_shapes(cfg):
    """(N, K) of the engine's bias-free projections for a GuardConfig: GDN in (padded) and out, attention in and
    out, MLP gate|up and down."""
    from .slot_engine import gdn_proj_width
    hq, hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    H, I = cfg.hidden_size, cfg.intermediate_size
    return [(gdn_proj_width(cfg), H), (H, cfg.value_dim), (hq * 2 * D + 2 * hkv * D, H), (H, hq * D),
            (2 * I, H), (H, I)]


def _time(torch, fn, reps, replays=3):
    """GPU time per call of ``fn``: ``reps`` calls captured into one hipGraph (as the engine runs them, so host
    launch cost does not enter), replayed ``replays`` times between HIP events. None if the capture fails."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for _ in range(reps):
                    if fn() != 0:
                        raise RuntimeError("hsg_gemm_bf16 failed under capture")
    except RuntimeError:
        torch.cuda.synchronize()
        return None
    torch.cuda.current_stream().wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * replays)


def tune_problem(torch, M, N, K, candidates=64, reps=10, seed=0):
    """Time hipBLASLt's first ``candidates`` solutions for one problem. A solution qualifies if it runs, two runs
    agree bit for bit and its result is within 2^-7 relative (Frobenius) of the fp32 product. Returns (best
    index, its µs, the first candidate's µs or None when the first does not qualify)."""
    import ctypes
    L = lib()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(seed)
    A = torch.randn(M, K, generator=gen, device=dev).bfloat16()
    W = (torch.randn(N, K, generator=gen, device=dev) * 0.02).bfloat16()
    ref = A.float() @ W.float().t()
    ws = torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    idx = (ctypes.c_int32 * candidates)()
    n = L.hsg_gemm_candidates(M, N, K, idx, None, candidates, WORKSPACE_BYTES)
    if n <= 0:
        return -1, None, None

    def run(i):
        return L.hsg_gemm_bf16(A.data_ptr(), K, W.data_ptr(), K, out.data_ptr(), N, M, N, K, i, ws.data_ptr(),
                               WORKSPACE_BYTES, torch.cuda.current_stream().cuda_stream)
    results = {}
    for c in list(idx[:n]):
        if run(c) != 0:
            continue
        first = out.clone()
        if run(c) != 0:
            continue
        torch.cuda.synchronize()
        if not torch.equal(first, out):
            continue
        err = (out.float() - ref).norm() / ref.norm()
        if not err <= 2.0 ** -7:
            continue
        us = _time(torch, lambda: run(c), reps)
        if us is not None:
            results[c] = us
    if not results:
        return -1, None, None
    best = min(results, key=results.get)
    return best, results[best], results.get(idx[0])


def tune(cfgs, max_slots=352, max_tick_tokens=64, candidates=256, candidates_large=64, large_m=4096, reps=10,
         log=print):
    """Plans for every token bucket of an engine of ``max_slots`` slots and every projection shape of ``cfgs``:
    ``candidates`` solutions searched per problem up to ``large_m`` rows (the streaming ticks), ``candidates_large``
    beyond (prefill ticks, whose products are long enough for the first candidates to be near the best)."""
    import torch

    from .slot_engine import token_buckets
    buckets = token_buckets(max_slots * max_tick_tokens)   # the engine's token buckets (its largest row bucket
    # is max_slots)
    shapes = sorted({s for cfg in cfgs for s in engine_shapes(cfg)})
    plans = {}
    t0 = time.time()
    for M in buckets:
        for N, K in shapes:
            best, us, first_us = tune_problem(torch, M, N, K, candidates if M <= large_m else candidates_large,
                                              reps)
            if best < 0:
                continue
            plans[f"{M},{N},{K}"] = {"index": int(best), "us": round(us, 2),
                                     "first_us": None if first_us is None else round(first_us, 2)}
        log(f"[gemm_plan] M={M}: {len(plans)} plans ({time.time() - t0:.0f} s)")
    return {"blas_version": int(lib().hsg_gemm_blas_version()), "workspace_bytes": WORKSPACE_BYTES,
            "candidates": {"up_to_m": large_m, "small": candidates, "large": candidates_large}, "plans": plans}


def main(argv=None):
    ap = argparse.ArgumentParser(description="generate the engine's GEMM plan table on an MI355X")
    ap.add_argument("--out", default=PLAN_PATH)
    ap.add_argument("--slots", type=int, default=352)
    ap.add_argument("--candidates", type=int, default=256)
    ap.add_argument("--reps", type=int, default=10)
    args = ap.parse_args(argv)
    from ..model import GuardConfig
    data = tune([GuardConfig.baseline(), GuardConfig.v10()], max_slots=args.slots, candidates=args.candidates,
                reps=args.reps, log=lambda m: print(m, file=sys.stderr, flush=True))
    with open(args.out, "w") as f:
        json.dump(data, f, indent=0, sort_keys=True)
    gain = sum(v["first_us"] - v["us"] for v in data["plans"].values() if v["first_us"] is not None)
    print(json.dumps({"plans": len(data["plans"]), "sum_first_minus_best_us": round(gain, 1)}), flush=True)


if __name__ == "__main__":
    main()
