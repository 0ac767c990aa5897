"""Torch-facing wrappers of libhsg.so with the reference's kernel contracts.

Each wrapper keeps the name, argument meaning, output layout and error behaviour of the Triton wrapper it
replaces (AssertionError for layout misuse, as the reference's asserts), allocates its outputs with
``torch.empty`` and launches on the current stream. Nothing here synchronizes, so every wrapper can be
called under hipGraph capture. There is no fallback: a missing library raises RuntimeError.
"""
from __future__ import annotations

import torch

from .._lib import check, lib

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


def gdn_slot_v8(packed, key_dim, heads, head_k, value_heads, head_v, a, b, A_log, dt_bias, state, slots, lens,
                bv=32, num_warps=2):
    """Replaces fused_kernels.py:197-211. packed [N, L, 2*key_dim + value_dim] (conv_silu_update output);
    a, b [N, L, HV]; state [S, HV, K, V] pool (fp32 or fp16) updated in place at rows slots[n] with
    lens[n] > 0. Returns (o [N, L, HV, V] bf16, zeros at padded positions; sq = o.float()**2 fp32).
    ``bv`` and ``num_warps`` are accepted for signature parity; the HIP kernel has one fixed tiling."""
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
        heads, value_heads, head_k, head_v, head_k ** -0.5, _ptr(o), _ptr(sq), _stream(packed.device))
    check(rc, "hsg_gdn_slot_step")
    return o, sq


def gdn_slot_recurrent(q, k, v, a, b, A_log, dt_bias, state, slots, lens, scale=None, bv=8, num_warps=1):
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
        h, hv, kd, vd, scale, _ptr(o), None, _stream(v.device))
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
        ws_bytes = lib().hsg_ring_decode_workspace_bytes(n, hkv, groups, window)
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
