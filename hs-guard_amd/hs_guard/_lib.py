"""ctypes binding of libhsg.so (the C ABI declared in include/hsg.h).

The library is required: there is no CPU or torch fallback for any kernel. ``lib()`` raises a
RuntimeError naming the missing file when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os

# torch first: libhsg.so needs libamdhip64.so.7 and libhipblaslt.so.1, and torch's wheel bundles its own copies under
# those sonames. Whichever copy a process loads first serves every later user of the soname, so loading libhsg.so
# before torch would bind /opt/rocm's hipBLASLt and move torch.mm onto it as well. With torch loaded first the
# process runs torch's bundled HIP runtime and hipBLASLt, the ones the committed GEMM plan table was made with.
import torch  # noqa: F401,E402

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhsg.so")

# return codes of include/hsg.h
HSG_OK, HSG_ERR_ARG, HSG_ERR_ALIGN, HSG_ERR_SHAPE, HSG_ERR_BLAS = 0, -1, -2, -3, -4
HSG_GDN_BURST_MIN_DEFAULT = 16   # include/hsg.h
HSG_GEMM_SKINNY_M_MAX = 8        # include/hsg.h

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/hsg.h
SIGNATURES = {
    "hsg_version": (ctypes.c_int, []),
    "hsg_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "hsg_gdn_slot_step": (ctypes.c_int, [
        _P, _I64, _I32, _I32, _I32,          # qkv, qkv_stride, q_off, k_off, v_off
        _P, _P, _I64, _P, _P,                # a, b, ab_stride, A_log, dt_bias
        _P, _I32, _I64,                      # state, state_dtype, state_rows
        _P, _P, _P, _I32, _I32,              # slots, lens, offsets, n_rows, L
        _I32, _I32, _I32, _I32, _F,          # H, HV, K, V, scale
        _P, _P, _I32, _P]),                  # o, sq, burst_min, stream
    "hsg_gdn_chunk_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _I32]),
    "hsg_gdn_chunk_prefill": (ctypes.c_int, [
        _P, _I64, _I32, _I32, _I32,
        _P, _P, _I64, _P, _P,
        _P, _I32, _I64,
        _P, _P, _P, _I32, _I32,
        _I32, _I32, _I32, _I32, _F,
        _P, _P, _I32, _P, ctypes.c_size_t, _P]),   # o, sq, min_len, workspace, workspace_bytes, stream
    "hsg_gdn_chunk_prefill_gated": (ctypes.c_int, [
        _P, _I64, _I32, _I32, _I32,
        _P, _P, _I64, _P, _P,
        _P, _I32, _I64,
        _P, _P, _P, _I32, _I32,
        _I32, _I32, _I32, _I32, _F,
        _P, _P, _I64, _P, _F, _P,            # o, z, z_stride, norm_w, eps, out
        _I32, _P, ctypes.c_size_t, _P]),     # min_len, workspace, workspace_bytes, stream
    "hsg_gdn_slot_step_gated": (ctypes.c_int, [
        _P, _I64, _I32, _I32, _I32,
        _P, _P, _I64, _P, _P,
        _P, _I32, _I64,
        _P, _P, _P, _I32, _I32,
        _I32, _I32, _I32, _I32, _F,
        _P, _I64, _P, _F, _P, _I32, _I32, _I32, _P]),   # z, z_stride, norm_w, eps, out, skip_rows, skip_min_len,
                                                        # burst_min, stream
    "hsg_gdn_conv_slot_step_gated": (ctypes.c_int, [
        _P, _I64, _I32, _I32, _I32,          # proj, proj_stride, q_off, k_off, v_off
        _P, _P, _I32,                        # conv_w, conv_pool, channels
        _P, _P, _I64, _P, _P,                # a, b, ab_stride, A_log, dt_bias
        _P, _I32, _I64,                      # state, state_dtype, state_rows
        _P, _P, _P, _I32,                    # slots, lens, offsets, n_rows
        _I32, _I32, _I32, _I32, _F,          # H, HV, K, V, scale
        _P, _I64, _P, _F, _P, _I32, _P]),    # z, z_stride, norm_w, eps, out, burst_min, stream
    "hsg_ring_attention": (ctypes.c_int, [
        _P, _I64, _I64, _I64, _I64,          # q, q_sn, q_sl, q_sh, q_sg
        _P, _P, _I64, _I32,                  # ring_k, ring_v, ring_rows, window
        _P, _I64, _I64, _I64,                # new_k, nk_sn, nk_sl, nk_sh
        _P, _I64, _I64, _I64,                # new_v, nv_sn, nv_sl, nv_sh
        _P, _I64, _I64, _I64, _I64, _I64,    # gate, g_sn, g_sl, g_sh, g_sg, g_off
        _P, _P, _P, _P, _P,                  # ring_pos, slots, starts, lens, offsets
        _I32, _I32, _I32, _I32, _I32, _F, _I32, _I32,  # n_rows, lb, hkv, groups, head_dim, scale, write_ring,
                                                         # min_len
        _P, _I64, _I64, _I64, _I64, _P]),    # out, o_sn, o_sl, o_sh, o_sg, stream
    "hsg_ring_decode_workspace_bytes": (ctypes.c_size_t, [_I32, _I32, _I32, _I32]),
    "hsg_ring_decode": (ctypes.c_int, [
        _P, _I64, _I64, _I64, _I64,          # q, q_sn, q_sl, q_sh, q_sg
        _P, _P, _I64, _I32,                  # ring_k, ring_v, ring_rows, window
        _P, _I64, _I64, _I64,                # new_k, nk_sn, nk_sl, nk_sh
        _P, _I64, _I64, _I64,                # new_v, nv_sn, nv_sl, nv_sh
        _P, _I64, _I64, _I64, _I64, _I64,    # gate, g_sn, g_sl, g_sh, g_sg, g_off
        _P, _P, _P, _P, _P,                  # ring_pos, slots, starts, lens, offsets
        _I32, _I32, _I32, _I32, _F, _I32,    # n_rows, hkv, groups, head_dim, scale, write_ring
        _P, _I64, _I64, _I64, _I64,          # out, o_sn, o_sl, o_sh, o_sg
        _P, ctypes.c_size_t, _P]),           # workspace, workspace_bytes, stream
    "hsg_ring_decode_rope": (ctypes.c_int, [
        _P, _I64, _I64, _P, _F,              # q_raw, q_row, q_head, q_w1, q_eps
        _P, _I64, _I64, _P, _F,              # k_raw, k_row, k_head, k_w1, k_eps
        _P, _P, _I32, _P, _I64,              # pos, inv_freq, rot, k_out, ko_row
        _P, _P, _I64, _I32,                  # ring_k, ring_v, ring_rows, window
        _P, _I64, _I64,                      # new_v, nv_row, nv_head
        _P, _I64, _I64, _I64, _I64,          # gate, g_row, g_head, g_group, g_off
        _P, _P, _P, _P, _P,                  # ring_pos, slots, starts, lens, offsets
        _I32, _I32, _I32, _I32, _F, _I32,    # n_rows, hkv, groups, head_dim, scale, write_ring
        _P, _I64, _I64, _I64,                # out, o_row, o_head, o_group
        _P, ctypes.c_size_t, _P]),           # workspace, workspace_bytes, stream
    "hsg_ring_decode_noalloc": (ctypes.c_int, [
        _P, _I64, _I64, _I64, _I64,          # q, q_sn, q_sl, q_sh, q_sg
        _P, _P, _I64, _I32,                  # ring_k, ring_v, ring_rows, window
        _P, _I64, _I64, _I64,                # new_k, nk_sn, nk_sl, nk_sh
        _P, _I64, _I64, _I64,                # new_v, nv_sn, nv_sl, nv_sh
        _P, _I64, _I64, _I64, _I64, _I64,    # gate, g_sn, g_sl, g_sh, g_sg, g_off
        _P, _P, _P, _P, _P,                  # ring_pos, slots, starts, lens, offsets
        _I32, _I32, _I32, _I32, _F, _I32,    # n_rows, hkv, groups, head_dim, scale, write_ring
        _P, _I64, _I64, _I64, _I64, _P]),    # out, o_sn, o_sl, o_sh, o_sg, stream
    "hsg_embed_rmsnorm": (ctypes.c_int, [_P, _P, _I64, _P, _F, _P, _P, _I32, _I32, _P]),
    "hsg_add_rmsnorm": (ctypes.c_int, [_P, _P, _P, _F, _P, _I32, _I32, _P]),
    "hsg_conv_silu_update": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _I32, _P, _P, _P, _I32, _I32, _I32, _P,
                                            _I64, _P]),
    "hsg_gated_rmsnorm": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _F, _P, _I64, _I32, _I32, _I32, _P]),
    "hsg_norm_rope": (ctypes.c_int, [_P, _I64, _I64, _I32, _P, _F, _P, _I64, _I64,
                                     _P, _I64, _I64, _I32, _P, _F, _P, _I64, _I64,
                                     _P, _P, _I32, _I32, _I32, _P]),
    "hsg_silu_mul": (ctypes.c_int, [_P, _I64, _I32, _P, _I32, _P]),
    "hsg_add_square": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I32, _P]),
    "hsg_rms_finish": (ctypes.c_int, [_P, _P, _P, _F, _P, _I64, _I32, _P]),
    "hsg_silu_mul_pair": (ctypes.c_int, [_P, _P, _P, _I64, _P]),
    "hsg_gated_finish": (ctypes.c_int, [_P, _P, _P, _P, _F, _P, _I64, _I32, _P]),
    "hsg_square_rows": (ctypes.c_int, [_P, _P, _I64, _I32, _I64, _I64, _I32, _P]),
    "hsg_norm_rope_grouped": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _F, _I32, _I32, _I32, _I32, _I64, _I64,
                                             _I32, _P, _I64, _I64, _I64, _P]),
    "hsg_risk_head": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _F, _I32, _I32, _P, _I32, _P]),
    "hsg_risk_head_f32": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _F, _I32, _I32, _P, _I32, _P]),
    "hsg_ring_pos_update": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _P, _I32, _I32, _P]),
    "hsg_gemm_bf16": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _I32, _P, ctypes.c_size_t,
                                     _P]),                  # A, lda, W, ldw, D, ldd, M, N, K, algo, ws, ws_bytes, stream
    "hsg_gemm_bf16_skinny": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _P]),
    "hsg_gemm_bf16_skinny_silu": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32,
                                                 _P]),   # gate_up, ld_gu, W, ldw, D, ldd, M, N, K, stream
    "hsg_gemm_bf16_skinny_addnorm": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _F, _P, _I64, _P, _I64, _P, _I64, _I32,
                                                    _I32, _I32, _P, _P]),
    "hsg_gemm_candidates": (ctypes.c_int, [_I32, _I32, _I32, _P, _P, _I32, ctypes.c_size_t]),
    "hsg_gemm_blas_version": (ctypes.c_int, []),
}

_lib = None


def lib():
    """Load libhsg.so once and attach the signatures; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HS-Guard HIP library not built: {LIB_PATH} is missing "
                               "(run `python -c 'import __graft_entry__ as g; g.build()'` at the repo root)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(rc, name):
    """Map a non-zero return code of an hsg_* call to an exception (ValueError for rejected arguments)."""
    if rc == 0:
        return
    text = lib().hsg_error_string(rc).decode()
    if rc < 0:
        raise ValueError(f"{name}: {text} (code {rc})")
    raise RuntimeError(f"{name}: HIP launch failed: {text} (code {rc})")
