"""Torch-facing wrappers of libhsg.so with the reference's kernel contracts.

Each wrapper keeps the name, argument meaning, output layout and error behaviour of the Triton wrapper it
replaces (AssertionError for layout misuse, as the reference's asserts), allocates its outputs with
``torch.empty`` and launches on the current stream. Nothing here synchronizes, so every wrapper can be
called under hipGraph capture. There is no fallback: a missing library raises RuntimeError.
"""
from __future__ import annotations

import torch

from .._lib import HSG_GDN_BURST_MIN_DEFAULT, check, lib

HSG_STATE_F32 = 0
HSG_STATE_F16 = 1
_STATE_CODES = {torch.float32: HSG_STATE_F32, torch.float16: HSG_STATE_F16}


def _require(cond, msg):
    if not cond:
        raise AssertionError(msg)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _gpu(*tensors):
    for t in tensors:
        _require(t is None or t.is_cuda, "HS-Guard kernels take GPU tensors")


def _bf16_in(*tensors):
    for t in tensors:
        _require(t.dtype == torch.bfloat16, "bf16 tensors expected")
        _require(t.is_contiguous(), "tensors must be contiguous")


def add_square(residual, mixed=None):
    """Replaces fused_kernels.py:44-52: (bf16(residual + mixed), its fp32 squares); with mixed None the squares of
    residual, returned beside residual itself."""
    _gpu(residual, mixed)
    _bf16_in(residual, *(() if mixed is None else (mixed,)))
    _require(mixed is None or mixed.shape == residual.shape, "residual and mixed must have one shape")
    n = residual.shape[-1]
    sq = torch.empty(residual.shape, dtype=torch.float32, device=residual.device)
    out = residual if mixed is None else torch.empty_like(residual)
    check(lib().hsg_add_square(_ptr(residual), _ptr(mixed), None if mixed is None else _ptr(out), _ptr(sq),
                               residual.numel() // n, n, _stream(residual.device)), "hsg_add_square")
    return out, sq


def rms_finish(x, var, w1, eps):
    """Replaces fused_kernels.py:67-72: Qwen3_5RMSNorm of x given var = mean(x.float()**2, -1, keepdim=True) and
    w1 = 1 + weight.float()."""
    _gpu(x, var, w1)
    _bf16_in(x)
    n = x.shape[-1]
    rows = x.numel() // n
    _require(var.dtype == torch.float32 and var.is_contiguous() and var.numel() == rows, "var must be [rows] fp32")
    _require(w1.dtype == torch.float32 and w1.is_contiguous() and w1.numel() == n, "w1 must be [width] fp32")
    out = torch.empty_like(x)
    check(lib().hsg_rms_finish(_ptr(x), _ptr(var), _ptr(w1), float(eps), _ptr(out), rows, n,
                               _stream(x.device)), "hsg_rms_finish")
    return out


def silu_mul(gate, up):
    """Replaces fused_kernels.py:86-90: bf16(bf16(silu(gate)) * up) on two tensors of one shape."""
    _gpu(gate, up)
    _bf16_in(gate, up)
    _require(gate.shape == up.shape, "gate and up must have one shape")
    out = torch.empty_like(gate)
    check(lib().hsg_silu_mul_pair(_ptr(gate), _ptr(up), _ptr(out), gate.numel(), _stream(gate.device)),
          "hsg_silu_mul_pair")
    return out


def conv_silu_update(qkv, pool, weight, slots, lens):
    """Replaces fused_kernels.py:126-136: qkv [N, L, C] bf16; pool [S, K-1, C] bf16 (one layer, updated in place at
    rows slots[n] with lens[n] > 0); weight [C, 1, K] bf16. Returns silu(causal depthwise conv) [N, L, C] bf16
    at every position of every row, as the reference computes it."""
    n, length, c = qkv.shape
    ks = weight.shape[-1]
    _require(qkv.is_contiguous() and pool.is_contiguous() and weight.is_contiguous()
             and pool.shape[1:] == (ks - 1, c), "conv_silu_update: contiguous qkv, pool [S, K-1, C], weight [C, 1, K]")
    _gpu(qkv, pool, weight, slots, lens)
    _bf16_in(qkv, pool, weight)
    out = torch.empty_like(qkv)
    check(lib().hsg_conv_silu_update(_ptr(qkv), c, _ptr(pool), pool.shape[0], _ptr(weight), ks, _ptr(slots),
                                     _ptr(lens), None, n, length, c, _ptr(out), c, _stream(qkv.device)),
          "hsg_conv_silu_update")
    return out


def gated_finish(x, var, weight, z, eps):
    """Replaces fused_kernels.py:228-233: Qwen3_5RMSNormGated(x, z) over the last dim given
    var = mean(x.float()**2, -1, keepdim=True); weight bf16 (the backbone's parameter)."""
    _gpu(x, var, weight, z)
    _bf16_in(x, weight, z)
    n = x.shape[-1]
    rows = x.numel() // n
    _require(z.shape == x.shape and weight.numel() == n, "z must match x and weight its last dim")
    _require(var.dtype == torch.float32 and var.is_contiguous() and var.numel() == rows, "var must be [rows] fp32")
    out = torch.empty_like(x)
    check(lib().hsg_gated_finish(_ptr(x), _ptr(var), _ptr(weight), _ptr(z), float(eps), _ptr(out), rows, n,
                                 _stream(x.device)), "hsg_gated_finish")
    return out


def square_rows(src, tokens, heads, row_stride, head_stride, dim):
    """Replaces fused_kernels.py:245-249: fp32 squares [tokens, heads, dim] of the head rows read at
    src + t*row_stride + h*head_stride (elements)."""
    _gpu(src)
    _bf16_in(src)
    _require(tokens == 0 or (tokens - 1) * row_stride + (heads - 1) * head_stride + dim <= src.numel(),
             "rows reach past src")
    sq = torch.empty(tokens, heads, dim, dtype=torch.float32, device=src.device)
    check(lib().hsg_square_rows(_ptr(src), _ptr(sq), tokens, heads, row_stride, head_stride, dim,
                                _stream(src.device)), "hsg_square_rows")
    return sq


def norm_rope(src, var, w1, cos, sin, eps, n, lb, heads, groups, row_stride, head_stride, dim):
    """Replaces fused_kernels.py:277-284: Qwen3_5RMSNorm per head (given var [n*lb*heads] fp32) then
    apply_rotary_pos_emb with cos/sin [n, lb, rot] bf16, written as [n, heads // groups, groups * lb, dim]: the
    grouped query layout of the ring kernel (groups = 1 gives the key layout [n, Hkv, lb, dim])."""
    _gpu(src, var, w1, cos, sin)
    _require(src.dtype == torch.bfloat16 and cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16,
             "src, cos and sin must be bf16")
    _require(cos.is_contiguous() and sin.is_contiguous() and cos.shape == sin.shape
             and cos.numel() == n * lb * cos.shape[-1], "cos and sin must be contiguous [n, lb, rot]")
    _require(var.dtype == torch.float32 and var.is_contiguous() and var.numel() == n * lb * heads,
             "var must be [n*lb*heads] fp32")
    _require(w1.dtype == torch.float32 and w1.is_contiguous() and w1.numel() == dim, "w1 must be [dim] fp32")
    _require(src.is_contiguous() and (n * lb == 0 or (n * lb - 1) * row_stride + (heads - 1) * head_stride + dim
                                      <= src.numel()), "src must be contiguous and hold every head row")
    _require(heads % groups == 0, "heads must be a multiple of groups")
    rot = cos.shape[-1]
    out = torch.empty(n, heads // groups, groups * lb, dim, dtype=torch.bfloat16, device=src.device)
    check(lib().hsg_norm_rope_grouped(_ptr(src), _ptr(var), _ptr(w1), _ptr(cos), _ptr(sin), rot, float(eps), n, lb,
                                      heads, groups, row_stride, head_stride, dim, _ptr(out), out.stride(0),
                                      out.stride(1), out.stride(2), _stream(src.device)), "hsg_norm_rope_grouped")
    return out


def gdn_slot_v8(packed, key_dim, heads, head_k, value_heads, head_v, a, b, A_log, dt_bias, state, slots, lens,
                bv=32, num_warps=2, burst_min=HSG_GDN_BURST_MIN_DEFAULT):
    """Replaces fused_kernels.py:197-211. packed [N, L, 2*key_dim + value_dim] (conv_silu_update output);
    a, b [N, L, HV]; state [S, HV, K, V] pool (fp32 or fp16) updated in place at rows slots[n] with
    lens[n] > 0. Returns (o [N, L, HV, V] bf16, zeros at padded positions; sq = o.float()**2 fp32).
    ``bv`` and ``num_warps`` are accepted for signature parity; the HIP kernel has one fixed tiling.
    ``burst_min``: rows of at least that many tokens run 8 at a time in the chunk form on MFMA (0: none)."""
    n, length, c = packed.shape
    for tensor in (packed, a, b, state):
        _require(tensor.is_contiguous(), "tensors must be contiguous")
    _gpu(packed, a, b, state, slots, lens)
    _require(packed.dtype == torch.bfloat16, "packed must be bf16")
    _require(state.dtype in _STATE_CODES, "state must be float32 or float16")
    _require(state.shape[1:] == (value_heads, head_k, head_v), "state must be [S, HV, K, V]")
    o = torch.empty(n, length, value_heads, head_v, dtype=packed.dtype, device=packed.device)
    sq = torch.empty(o.shape, dtype=torch.float32, device=packed.device)
    rc = lib().hsg_gdn_slot_step(
        _ptr(packed), c, 0, key_dim, 2 * key_dim, _ptr(a), _ptr(b), value_heads, _ptr(A_log), _ptr(dt_bias),
        _ptr(state), _STATE_CODES[state.dtype], state.shape[0], _ptr(slots), _ptr(lens), None, n, length,
        heads, value_heads, head_k, head_v, head_k ** -0.5, _ptr(o), _ptr(sq), int(burst_min), _stream(packed.device))
    check(rc, "hsg_gdn_slot_step")
    return o, sq


def gdn_slot_recurrent(q, k, v, a, b, A_log, dt_bias, state, slots, lens, scale=None, bv=8, num_warps=1,
                       burst_min=HSG_GDN_BURST_MIN_DEFAULT):
    """Replaces gdn_slot_kernel.py:57-73: q, k [N, L, H, K]; v [N, L, HV, V]; returns o [N, L, HV, V]."""
    n, length, h, kd = k.shape
    hv, vd = v.shape[2], v.shape[3]
    for tensor in (q, k, v, a, b, state):
        _require(tensor.is_contiguous(), "tensors must be contiguous")
    _require(state.dtype in (torch.float32, torch.float16) and state.shape[1:] == (hv, kd, vd),
             "state must be [S, HV, K, V] float32 or float16")
    scale = kd ** -0.5 if scale is None else scale
    qkv = torch.cat([q.reshape(n, length, -1), k.reshape(n, length, -1), v.reshape(n, length, -1)], -1)
    o = torch.empty(n, length, hv, vd, dtype=v.dtype, device=v.device)
    rc = lib().hsg_gdn_slot_step(
        _ptr(qkv), qkv.shape[-1], 0, h * kd, 2 * h * kd, _ptr(a), _ptr(b), hv, _ptr(A_log), _ptr(dt_bias),
        _ptr(state), _STATE_CODES[state.dtype], state.shape[0], _ptr(slots), _ptr(lens), None, n, length,
        h, hv, kd, vd, scale, _ptr(o), None, int(burst_min), _stream(v.device))
    check(rc, "hsg_gdn_slot_step")
    return o


def gdn_chunk_prefill(packed, key_dim, heads, head_k, value_heads, head_v, a, b, A_log, dt_bias, state, slots,
                      lens, offsets=None, scale=None, with_sq=False, max_len=None, workspace=None):
    """Chunked prefill (replaces FLA chunk_gated_delta_rule with initial_state = state[slots] and
    output_final_state written back, bucketed_engine.py:109-111), with gdn_slot_v8's input contract.

    Padded layout (offsets None): packed [N, L, C], a/b [N, L, HV]; returns o [N, L, HV, V] with zeros past
    lens. Packed layout: packed [T, C], a/b [T, HV], row n's tokens at offsets[n] .. offsets[n]+lens[n]-1;
    returns o [T, HV, V]; max_len bounds every row's length (default: lens.max(), a device sync).
    State rows slots[n] (lens > 0) are updated in place. workspace: a uint8 device tensor of at least
    chunk_workspace_bytes(...) bytes, reused across calls (allocated per call when None).
    Returns (o, sq or None)."""
    for tensor in (packed, a, b, state):
        _require(tensor.is_contiguous(), "tensors must be contiguous")
    _gpu(packed, a, b, state, slots, lens, offsets)
    _require(packed.dtype == torch.bfloat16, "packed must be bf16")
    _require(state.dtype in _STATE_CODES, "state must be float32 or float16")
    _require(state.shape[1:] == (value_heads, head_k, head_v), "state must be [S, HV, K, V]")
    if offsets is None:
        n, length, c = packed.shape
        out_shape = (n, length, value_heads, head_v)
    else:
        _require(packed.dim() == 2, "packed layout takes [T, C]")
        c = packed.shape[1]
        n = slots.shape[0]
        length = int(lens.max()) if max_len is None else int(max_len)
        out_shape = (packed.shape[0], value_heads, head_v)
    o = torch.empty(out_shape, dtype=packed.dtype, device=packed.device)
    sq = torch.empty(out_shape, dtype=torch.float32, device=packed.device) if with_sq else None
    scale = head_k ** -0.5 if scale is None else scale
    ws_bytes = lib().hsg_gdn_chunk_workspace_bytes(n, max(length, 1), value_heads)
    if workspace is None:
        workspace = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=packed.device)
    _require(workspace.numel() >= ws_bytes, f"workspace needs {ws_bytes} bytes")
    rc = lib().hsg_gdn_chunk_prefill(
        _ptr(packed), c, 0, key_dim, 2 * key_dim, _ptr(a), _ptr(b), value_heads, _ptr(A_log), _ptr(dt_bias),
        _ptr(state), _STATE_CODES[state.dtype], state.shape[0], _ptr(slots), _ptr(lens), _ptr(offsets), n,
        max(length, 1), heads, value_heads, head_k, head_v, scale, _ptr(o), _ptr(sq), 0, _ptr(workspace),
        workspace.numel(), _stream(packed.device))
    check(rc, "hsg_gdn_chunk_prefill")
    return o, sq


def ring_attention_v8(q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, lens, scale, window,
                      write_ring, block_m=16, block_n=32, num_warps=4, num_stages=1, split_k=True):
    """Replaces fused_kernels.py:358-376. q [N, Hkv, G*Lb, D] and new_k [N, Hkv, Lb, D]; value [N, Lb, Hkv*D]
    (v_proj output, strided rows allowed); gate: q_proj output [N, Lb, Hq*2D] (gate = second half of each
    head). Returns out * sigmoid(gate) as [N, Lb, Hq*D] bf16. write_ring (Lb == 1 only, as the
    reference): also writes this tick's key/value into ring column start % window. Decode ticks (Lb == 1)
    run the decode kernel (hsg_ring_decode) unless split_k is False."""
    n, hkv, m, d = q.shape
    lb = new_k.shape[2]
    groups = m // lb
    _require(window % block_n == 0 and d & (d - 1) == 0 and block_m >= 16 and block_n >= 16, "bad tiling")
    _require(not write_ring or (lb == 1 and m <= block_m), "write_ring needs Lb == 1")
    for tensor in (q, ring_k, ring_v, new_k, value, gate, ring_pos):
        _require(tensor.is_contiguous(), "tensors must be contiguous")
    _gpu(q, ring_k, ring_v, new_k, value, gate, ring_pos, slots, starts, lens)
    out = torch.empty(n, lb, hkv * groups * d, dtype=torch.bfloat16, device=q.device)
    if lb == 1 and split_k:
        # the split-K kernels (more than 8 query heads per kv head) keep their partial results in a workspace; the
        # fused kernel below that needs none
        ws_bytes = lib().hsg_ring_decode_workspace_bytes(n, hkv, groups, window) if groups > 8 else 0
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
        rc = lib().hsg_ring_decode(
            _ptr(q), hkv * m * d, d, m * d, d,
            _ptr(ring_k), _ptr(ring_v), ring_k.shape[0], window,
            _ptr(new_k), hkv * d, d, d,
            _ptr(value), value.stride(0), value.stride(1), d,
            _ptr(gate), gate.stride(0), gate.stride(1), groups * 2 * d, 2 * d, d,
            _ptr(ring_pos), _ptr(slots), _ptr(starts), _ptr(lens), None,
            n, hkv, groups, d, float(scale), int(bool(write_ring)),
            _ptr(out), hkv * groups * d, hkv * groups * d, groups * d, d, _ptr(ws), ws.numel(), _stream(q.device))
        check(rc, "hsg_ring_decode")
        return out
    rc = lib().hsg_ring_attention(
        _ptr(q), hkv * m * d, d, m * d, lb * d,
        _ptr(ring_k), _ptr(ring_v), ring_k.shape[0], window,
        _ptr(new_k), hkv * lb * d, d, lb * d,
        _ptr(value), value.stride(0), value.stride(1), d,
        _ptr(gate), gate.stride(0), gate.stride(1), groups * 2 * d, 2 * d, d,
        _ptr(ring_pos), _ptr(slots), _ptr(starts), _ptr(lens), None,
        n, lb, hkv, groups, d, float(scale), int(bool(write_ring)), 0,
        _ptr(out), lb * hkv * groups * d, hkv * groups * d, groups * d, d, _stream(q.device))
    check(rc, "hsg_ring_attention")
    return out


def ring_attention(q, ring_k, ring_v, new_k, new_v, ring_pos, slots, starts, lens, scale, window,
                   block_m=16, block_n=32, num_warps=4, num_stages=1):
    """Replaces ring_attention_kernel.py:91-105 (same contract as ring_attention_reference): q, out
    [N, Hkv, G*Lb, D]; new_k/new_v [N, Hkv, Lb, D]; the ring is read only."""
    n, hkv, m, d = q.shape
    lb = new_k.shape[2]
    groups = m // lb
    _require(window % block_n == 0 and d & (d - 1) == 0 and block_m >= 16 and block_n >= 16, "bad tiling")
    _require(ring_k.shape[1:] == (hkv, window + 1, d) and new_k.shape == (n, hkv, lb, d), "bad shapes")
    for tensor in (q, ring_k, ring_v, new_k, new_v, ring_pos):
        _require(tensor.is_contiguous(), "tensors must be contiguous")
    out = torch.empty_like(q)
    rc = lib().hsg_ring_attention(
        _ptr(q), hkv * m * d, d, m * d, lb * d,
        _ptr(ring_k), _ptr(ring_v), ring_k.shape[0], window,
        _ptr(new_k), hkv * lb * d, d, lb * d,
        _ptr(new_v), hkv * lb * d, d, lb * d,
        None, 0, 0, 0, 0, 0,
        _ptr(ring_pos), _ptr(slots), _ptr(starts), _ptr(lens), None,
        n, lb, hkv, groups, d, float(scale), 0, 0,
        _ptr(out), hkv * m * d, d, m * d, lb * d, _stream(q.device))
    check(rc, "hsg_ring_attention")
    return out
