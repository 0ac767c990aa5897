"""GPU parity of the per-token glue kernels of libhsg.so against their oracle functions.

Each kernel sees exactly the oracle's inputs (bf16 values). Outputs are bf16 values that must match the
oracle bit for bit except where fp32 rounding-order differences flip a bf16 rounding: at most 2**-8 relative
on at most 0.5% of the elements (the conv, which rounds to bf16 twice: two bf16 ulps, plus the fp32
accumulation bound where its sum cancels). Pool updates and ring_pos are bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import glue as oglue
from oracle import pack as opack
from oracle.bf16 import bf16
from parity_helpers import close_bf16 as _close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _np(t):
    return t.detach().float().cpu().numpy()


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)


def _stream():
    return torch.cuda.current_stream(DEV).cuda_stream


def test_embed_and_add_rmsnorm():
    from hs_guard._lib import lib
    print("[glue] embed + add rmsnorm", flush=True)
    rng = np.random.default_rng(0)
    T, Hd, V = 37, 1024, 500
    emb = bf16(rng.standard_normal((V, Hd)) * 0.02)
    ids = rng.integers(0, V, T)
    w1 = (1.0 + bf16(rng.standard_normal(Hd) * 0.02)).astype(np.float32)
    emb_d, ids_d = _bf(emb).to(DEV), torch.from_numpy(ids).to(DEV)
    w1_d = torch.from_numpy(w1).to(DEV)
    hid = torch.empty(T, Hd, dtype=torch.bfloat16, device=DEV)
    nrm = torch.empty_like(hid)
    assert lib().hsg_embed_rmsnorm(ids_d.data_ptr(), emb_d.data_ptr(), V, w1_d.data_ptr(), 1e-6, hid.data_ptr(),
                                   nrm.data_ptr(), T, Hd, _stream()) == 0
    np.testing.assert_array_equal(_np(hid), emb[ids])
    _close(_np(nrm), oglue.rmsnorm(emb[ids], w1, 1e-6), "embed rmsnorm", ulps=1)
    mix = bf16(rng.standard_normal((T, Hd)) * 0.05)
    mix_d = _bf(mix).to(DEV)
    assert lib().hsg_add_rmsnorm(hid.data_ptr(), mix_d.data_ptr(), w1_d.data_ptr(), 1e-6, nrm.data_ptr(), T, Hd,
                                 _stream()) == 0
    h_ref, n_ref = oglue.add_rmsnorm(emb[ids], mix, w1, 1e-6)
    np.testing.assert_array_equal(_np(hid), h_ref)
    _close(_np(nrm), n_ref, "add rmsnorm", ulps=1)


def test_gated_rmsnorm():
    """hsg_gated_rmsnorm (the chunk path's gated_finish) against the oracle, strided x / z / out."""
    from hs_guard._lib import lib
    print("[glue] gated rmsnorm", flush=True)
    rng = np.random.default_rng(5)
    T, HV, V = 29, 4, 128
    x = bf16(rng.standard_normal((T, HV * V)))
    z = bf16(rng.standard_normal((T, HV * V + 24)))
    w = bf16(1.0 + rng.standard_normal(V) * 0.1)
    ref = oglue.gated_rmsnorm(x.reshape(T, HV, V), z[:, :HV * V].reshape(T, HV, V), w, 1e-6).reshape(T, HV * V)
    x_d, z_d, w_d = _bf(x).to(DEV), _bf(z).to(DEV), _bf(w).to(DEV)
    out = torch.zeros(T, HV * V + 8, dtype=torch.bfloat16, device=DEV)
    assert lib().hsg_gated_rmsnorm(x_d.data_ptr(), HV * V, z_d.data_ptr(), HV * V + 24, w_d.data_ptr(), 1e-6,
                                   out.data_ptr(), HV * V + 8, T, HV, V, _stream()) == 0
    got = _np(out)
    _close(got[:, :HV * V], ref, "gated rmsnorm")
    assert np.count_nonzero(got[:, HV * V:]) == 0


@pytest.mark.parametrize("packed,rows", [(False, 4), (True, 4), (True, 70), (False, 70)])
def test_conv_silu_update(packed, rows):
    """4 rows spanning 1-3 chunks of 8 tokens; 70 rows, where rows past the first 64 (which get one workgroup
    per chunk) walk their chunks in one workgroup, some longer than 8 tokens."""
    from hs_guard._lib import lib
    print(f"[glue] conv packed={packed} rows={rows}", flush=True)
    rng = np.random.default_rng(1)
    C = 6144
    stride = C + 40
    if rows == 4:
        N, L, S = 4, 21, 6
        slots, lens = np.array([4, 1, 0, 2]), np.array([21, 2, 0, 9])
    else:
        N, L, S = rows, 24, rows + 3
        slots = rng.permutation(S)[:N]
        lens = rng.integers(0, L + 1, N)
        lens[[0, 5, 63, 64, 66, 69]] = [24, 1, 17, 19, 9, 0]
    qkv = bf16(rng.standard_normal((N, L, stride)))
    pool = bf16(rng.standard_normal((S, 3, C)))
    w = bf16(rng.standard_normal((C, 4)) * 0.5)
    ref_out, ref_pool = oglue.conv_silu_update(qkv[..., :C], pool, w, slots, lens)
    # the kernel sums the 4 products in fp32 (as the reference's kernel does), the oracle in float64. The fp32
    # sum is off by up to ~4 * 2^-24 * sum|w x|: where it sits at a bf16 rounding boundary, bf16(acc) flips by
    # one ulp and the output, rounded again after the SiLU, by up to two; where the sum cancels to near zero,
    # that absolute error is many ulps of the tiny output. Bar: 2 bf16 ulps + that absolute bound.
    atol = 4 * 2.0 ** -24 * float(np.abs(w).max()) * float(max(np.abs(qkv).max(), np.abs(pool).max())) * 4
    pool_d = _bf(pool).to(DEV)
    w_d = _bf(w).to(DEV)
    sl_d, ln_d = torch.from_numpy(slots).to(DEV), torch.from_numpy(lens).to(DEV)
    if packed:
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]])
        flat = np.concatenate([qkv[n, :lens[n]] for n in range(N)])
        q_d = _bf(flat).to(DEV)
        out = torch.zeros(len(flat), C, dtype=torch.bfloat16, device=DEV)
        rc = lib().hsg_conv_silu_update(q_d.data_ptr(), stride, pool_d.data_ptr(), S, w_d.data_ptr(), 4,
                                        sl_d.data_ptr(), ln_d.data_ptr(), torch.from_numpy(offs).to(DEV).data_ptr(),
                                        N, 0, C, out.data_ptr(), C, _stream())
        assert rc == 0
        got = _np(out)
        for n in range(N):
            if lens[n]:
                _close(got[offs[n]:offs[n] + lens[n]], ref_out[n, :lens[n]], f"conv row {n}", atol=atol, ulps=2)
    else:
        q_d = _bf(qkv).to(DEV)
        out = torch.zeros(N, L, C, dtype=torch.bfloat16, device=DEV)
        rc = lib().hsg_conv_silu_update(q_d.data_ptr(), stride, pool_d.data_ptr(), S, w_d.data_ptr(), 4,
                                        sl_d.data_ptr(), ln_d.data_ptr(), None, N, L, C, out.data_ptr(), C, _stream())
        assert rc == 0
        _close(_np(out), ref_out, "conv padded (all L positions, as the reference)", atol=atol,
               ulps=2)
    np.testing.assert_array_equal(_np(pool_d), ref_pool)


def test_norm_rope_q_and_k():
    from hs_guard._lib import lib
    print("[glue] norm_rope", flush=True)
    rng = np.random.default_rng(2)
    T, hq, hkv, D, rot = 9, 8, 2, 256, 64
    row = hq * 2 * D + 2 * hkv * D
    proj = bf16(rng.standard_normal((T, row)))
    pos = np.array([0, 1, 2, 511, 512, 4097, 8000, 8191, 77])
    qw1 = (1.0 + bf16(rng.standard_normal(D) * 0.02)).astype(np.float32)
    kw1 = (1.0 + bf16(rng.standard_normal(D) * 0.02)).astype(np.float32)
    inv = oglue.inv_freq(rot, 10000.0)
    cos, sin = oglue.rope_cos_sin(pos, inv)
    q_ref = oglue.norm_rope(proj[:, :hq * 2 * D].reshape(T, hq, 2 * D)[..., :D], qw1, 1e-6, cos, sin)
    k_ref = oglue.norm_rope(proj[:, hq * 2 * D:hq * 2 * D + hkv * D].reshape(T, hkv, D), kw1, 1e-6, cos, sin)
    p_d = _bf(proj).to(DEV)
    q = torch.empty(T, hq * D, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(T, hkv * D, dtype=torch.bfloat16, device=DEV)
    qw, kw = torch.from_numpy(qw1).to(DEV), torch.from_numpy(kw1).to(DEV)
    inv_d = torch.from_numpy(inv).to(DEV)
    pos_d = torch.from_numpy(pos).to(DEV)
    base = p_d.data_ptr()
    rc = lib().hsg_norm_rope(base, row, 2 * D, hq, qw.data_ptr(), 1e-6, q.data_ptr(), hq * D, D,
                             base + 2 * hq * 2 * D, row, D, hkv, kw.data_ptr(), 1e-6, k.data_ptr(), hkv * D, D,
                             pos_d.data_ptr(), inv_d.data_ptr(), rot, T, D, _stream())
    assert rc == 0
    _close(_np(q).reshape(T, hq, D), q_ref, "q norm+rope")
    _close(_np(k).reshape(T, hkv, D), k_ref, "k norm+rope")


def test_silu_mul_and_risk_head():
    from hs_guard._lib import lib
    print("[glue] silu_mul + risk head", flush=True)
    rng = np.random.default_rng(3)
    T, I = 11, 3584
    gu = bf16(rng.standard_normal((T, 2 * I)) * 2)
    gu_d = _bf(gu).to(DEV)
    act = torch.empty(T, I, dtype=torch.bfloat16, device=DEV)
    assert lib().hsg_silu_mul(gu_d.data_ptr(), 2 * I, I, act.data_ptr(), T, _stream()) == 0
    _close(_np(act), oglue.silu_mul(gu[:, :I], gu[:, I:]), "silu_mul")
    # more tokens than one launch's grid holds (65,535 rows): the entry point splits them; a row stride wider than
    # the gate|up pair and widths that are not a multiple of the 2,048-element column block
    for T, I, ld in ((70001, 8, 24), (3, 2056, 4120)):
        gu = bf16(rng.standard_normal((T, ld)) * 2)
        act = torch.empty(T, I, dtype=torch.bfloat16, device=DEV)
        assert lib().hsg_silu_mul(_bf(gu).to(DEV).data_ptr(), ld, I, act.data_ptr(), T, _stream()) == 0
        _close(_np(act), oglue.silu_mul(gu[:, :I], gu[:, I:2 * I]), f"silu_mul {T} x {I}")
    # heads at the model's scale (weights N(0, 0.02)), LayerNorm parameters fp32 values bf16 cannot hold
    T, E, R = 64, 512, 2
    y = bf16(rng.standard_normal((T, R * E)))
    ln_w = (1 + 0.05 * rng.standard_normal((R, E))).astype(np.float32)
    ln_b = (0.05 * rng.standard_normal((R, E))).astype(np.float32)
    w2 = bf16(rng.standard_normal((R, 3, E)) * 0.02)
    b2 = bf16(rng.standard_normal((R, 3)) * 0.02)
    probs = torch.empty(R, T, 3, dtype=torch.float32, device=DEV)
    d = [_bf(y).to(DEV), torch.from_numpy(ln_w).to(DEV), torch.from_numpy(ln_b).to(DEV), _bf(w2).to(DEV),
         _bf(b2).to(DEV)]
    assert lib().hsg_risk_head(d[0].data_ptr(), R * E, d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(),
                               d[4].data_ptr(), 1e-5, R, E, probs.data_ptr(), T, _stream()) == 0
    got = _np(probs)
    for r in range(R):
        # the reference head from the projection output on: LayerNorm -> SiLU -> bf16 -> Linear -> bf16.
        # A bf16 logit of magnitude below 1 is one step of at most 2**-9 from its neighbour, which moves a
        # probability by at most 2**-9 / 4, so fp32-vs-float64 rounding flips stay below 1e-3.
        v = oglue.silu(oglue.layer_norm(y[:, r * E:(r + 1) * E], ln_w[r], ln_b[r]))
        logits = oglue.linear_bf16(bf16(v), w2[r], b2[r]).astype(np.float64)
        assert np.abs(logits).max() < 1.0
        e = np.exp(logits - logits.max(-1, keepdims=True))
        np.testing.assert_allclose(got[r], e / e.sum(-1, keepdims=True), rtol=0, atol=1e-3)


def test_risk_head_f32():
    """hsg_risk_head_f32 (the complete-message readout: fp32 everywhere) against the float64 oracle."""
    from hs_guard._lib import lib
    print("[glue] risk head fp32", flush=True)
    rng = np.random.default_rng(6)
    T, E, R, H = 37, 512, 2, 1024
    h = bf16(rng.standard_normal((T, H)))
    w1 = (rng.standard_normal((R * E, H)) * 0.02).astype(np.float32)
    b1 = (rng.standard_normal(R * E) * 0.02).astype(np.float32)
    ln_w = (1 + 0.05 * rng.standard_normal((R, E))).astype(np.float32)
    ln_b = (0.05 * rng.standard_normal((R, E))).astype(np.float32)
    w2 = (rng.standard_normal((R, 3, E)) * 0.3).astype(np.float32)
    b2 = (rng.standard_normal((R, 3)) * 0.1).astype(np.float32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)
    y = torch.addmm(t(b1), t(h), t(w1).t())             # fp32 GEMM, as the scorer runs it
    probs = torch.empty(R, T, 3, dtype=torch.float32, device=DEV)
    dl = [t(x) for x in (ln_w, ln_b, w2, b2)]
    assert lib().hsg_risk_head_f32(y.data_ptr(), R * E, dl[0].data_ptr(), dl[1].data_ptr(), dl[2].data_ptr(),
                                   dl[3].data_ptr(), 1e-5, R, E, probs.data_ptr(), T, _stream()) == 0
    got = _np(probs)
    for r in range(R):
        ref = oglue.risk_probs_f32(h, w1[r * E:(r + 1) * E], b1[r * E:(r + 1) * E], ln_w[r], ln_b[r], w2[r], b2[r])
        np.testing.assert_allclose(got[r], ref, rtol=0, atol=2e-5)


def test_ring_pos_update_bit_exact():
    from hs_guard._lib import lib
    print("[glue] ring_pos", flush=True)
    rng = np.random.default_rng(4)
    S, W = 7, 32
    rp = np.full((S, W + 1), -1, dtype=np.int64)
    rp_d = torch.from_numpy(rp.copy()).to(DEV)
    length = np.zeros(S - 1, dtype=np.int64)
    for _ in range(30):
        n = int(rng.integers(1, 5))
        slots = rng.permutation(S - 1)[:n]
        lens = rng.integers(1, 17, n)
        nb = n + 1
        sl = np.concatenate([slots, [S - 1]])
        ln = np.concatenate([lens, [0]])
        st = np.concatenate([length[slots], [0]])
        opack.ring_pos_update(rp, sl, st, ln, int(ln.max()), W)
        assert lib().hsg_ring_pos_update(rp_d.data_ptr(), S, W, torch.from_numpy(sl).to(DEV).data_ptr(),
                                         torch.from_numpy(st).to(DEV).data_ptr(),
                                         torch.from_numpy(ln).to(DEV).data_ptr(), nb, 64, _stream()) == 0
        length[slots] += lens
    np.testing.assert_array_equal(rp_d.cpu().numpy(), rp)
