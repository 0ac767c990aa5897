"""The C-ABI library loads and exports every entry point include/hsg.h declares (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hsg.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hsg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "hsg_gdn_slot_step" in names and "hsg_ring_attention" in names


def test_library_exports_every_declared_symbol():
    from hs_guard._lib import LIB_PATH, SIGNATURES
    if not os.path.exists(LIB_PATH):
        pytest.fail(f"{LIB_PATH} missing: build() first")
    handle = ctypes.CDLL(LIB_PATH)
    for name in _declared():
        assert hasattr(handle, name), f"{name} not exported"
    assert set(SIGNATURES) == set(_declared()), "ctypes signatures out of sync with include/hsg.h"


def test_constants_match_the_header():
    """The Python mirror of the header's constants (return codes, the engine's GDN burst threshold)."""
    from hs_guard import _lib
    text = open(HEADER).read()
    assert int(re.search(r"#define HSG_GDN_BURST_MIN_DEFAULT (\d+)", text).group(1)) == _lib.HSG_GDN_BURST_MIN_DEFAULT
    assert int(re.search(r"#define HSG_GEMM_SKINNY_M_MAX (\d+)", text).group(1)) == _lib.HSG_GEMM_SKINNY_M_MAX
    for name in ("HSG_OK", "HSG_ERR_ARG", "HSG_ERR_ALIGN", "HSG_ERR_SHAPE", "HSG_ERR_BLAS"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m is not None and int(m.group(1)) == getattr(_lib, name), name


def test_version_and_error_strings():
    from hs_guard._lib import lib
    assert lib().hsg_version() >= 100
    assert b"alignment" in lib().hsg_error_string(-2)


def test_argument_errors_are_rejected_before_launch():
    """Invalid shapes return HSG_ERR_* without touching the GPU (null pointers are never dereferenced)."""
    from hs_guard._lib import lib
    L = lib()
    # n_rows > 0 with null pointers -> HSG_ERR_ARG; unsupported head size -> HSG_ERR_SHAPE
    rc = L.hsg_gdn_slot_step(None, 6144, 0, 2048, 4096, None, None, 16, None, None, None, 0, 17, None, None, None,
                             4, 1, 16, 16, 128, 128, 1.0, None, None, 8, None)
    assert rc == -1
    rc = L.hsg_gdn_slot_step(8, 6144, 0, 2048, 4096, 8, 8, 16, 8, 8, 16, 0, 17, 8, 8, None, 4, 1, 16, 16, 64, 128,
                             1.0, 8, None, 8, None)
    assert rc == -3
    rc = L.hsg_gdn_slot_step(8, 6144, 0, 2048, 4096, 8, 8, 16, 8, 8, 16, 0, 17, 8, 8, None, 4, 1, 16, 16, 128, 128,
                             1.0, 8, None, -1, None)
    assert rc == -1          # a negative burst threshold
    rc = L.hsg_ring_attention(16, 0, 256, 0, 0, 16, 16, 5, 512, 16, 0, 256, 0, 16, 0, 256, 0, None, 0, 0, 0, 0, 0,
                              8, 8, 8, 8, None, 2, 1, 4, 4, 128, 1.0, 0, 0, 16, 0, 0, 0, 0, None)
    assert rc == -3
    # decode: head_dim 128 is rejected; on the split-K path (G > 8) a missing or too-small workspace is rejected;
    # n_rows == 0 is a no-op
    need = L.hsg_ring_decode_workspace_bytes(2, 4, 16, 512)
    assert need > 0
    rc = L.hsg_ring_decode(16, 0, 256, 0, 0, 16, 16, 5, 512, 16, 0, 256, 0, 16, 0, 256, 0, None, 0, 0, 0, 0, 0,
                           8, 8, 8, 8, None, 2, 4, 4, 128, 1.0, 1, 16, 0, 0, 0, 0, 16, need, None)
    assert rc == -3
    rc = L.hsg_ring_decode(16, 0, 256, 0, 0, 16, 16, 5, 512, 16, 0, 256, 0, 16, 0, 256, 0, None, 0, 0, 0, 0, 0,
                           8, 8, 8, 8, None, 2, 4, 16, 256, 1.0, 1, 16, 0, 0, 0, 0, 16, need - 1, None)
    assert rc == -3
    rc = L.hsg_ring_decode(16, 0, 256, 0, 0, 16, 16, 5, 512, 16, 0, 256, 0, 16, 0, 256, 0, None, 0, 0, 0, 0, 0,
                           8, 8, 8, 8, None, 2, 4, 16, 256, 1.0, 1, 16, 0, 0, 0, 0, None, need, None)
    assert rc == -1
    assert L.hsg_ring_decode(None, 0, 0, 0, 0, None, None, 5, 512, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0, 0,
                             0, None, None, None, None, None, 0, 4, 4, 256, 1.0, 1, None, 0, 0, 0, 0, None, 0,
                             None) == 0
    # allocation-free decode: split-K sizes (G > 8) beyond its scratch are rejected before any device call (the
    # placeholder pointers are never read); 0 rows is a no-op
    cap = re.search(r"#define HSG_RING_DECODE_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(HEADER).read())
    cap = int(cap.group(1)) << int(cap.group(2))
    unit = L.hsg_ring_decode_workspace_bytes(1, 4, 16, 512)
    rows = cap // unit + 1
    assert L.hsg_ring_decode_workspace_bytes(rows, 4, 16, 512) > cap
    assert L.hsg_ring_decode_noalloc(16, 0, 256, 0, 0, 16, 16, rows + 1, 512, 16, 0, 256, 0, 16, 0, 256, 0, None, 0,
                                     0, 0, 0, 0, 8, 8, 8, 8, None, rows, 4, 16, 256, 1.0, 1, 16, 0, 0, 0, 0,
                                     None) == -3
    assert L.hsg_ring_decode_noalloc(None, 0, 0, 0, 0, None, None, 5, 512, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0,
                                     0, 0, 0, None, None, None, None, None, 0, 4, 4, 256, 1.0, 1, None, 0, 0, 0, 0,
                                     None) == 0
    # chunk prefill: workspace size is rows x ceil(L / 64) x HV units plus the row order (4 bytes per row in
    # 256-byte blocks); a too-small or unaligned workspace and L <= 0 are rejected
    unit = L.hsg_gdn_chunk_workspace_bytes(1, 64, 1) - 256
    assert unit > 0 and unit == L.hsg_gdn_chunk_workspace_bytes(1, 128, 1) - unit - 256
    assert L.hsg_gdn_chunk_workspace_bytes(3, 130, 16) == 3 * 3 * 16 * unit + 256
    assert L.hsg_gdn_chunk_workspace_bytes(70, 64, 1) == 70 * unit + 512
    assert L.hsg_gdn_chunk_workspace_bytes(0, 64, 16) == 0
    need = L.hsg_gdn_chunk_workspace_bytes(4, 100, 16)
    args = [256, 6144, 0, 2048, 4096, 256, 256, 16, 256, 256, 256, 0, 17, 256, 256, None, 4, 100, 16, 16, 128, 128,
            1.0, 256, None]
    assert L.hsg_gdn_chunk_prefill(*args, 0, 256, need - 1, None) == -3
    assert L.hsg_gdn_chunk_prefill(*args, 0, 128, need, None) == -2
    args[17] = 0
    assert L.hsg_gdn_chunk_prefill(*args, 0, 256, need, None) == -1
    # n_rows == 0 is a no-op success
    assert L.hsg_ring_attention(None, 0, 0, 0, 0, None, None, 5, 512, None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                                0, 0, None, None, None, None, None, 0, 1, 4, 4, 256, 1.0, 0, 0, None, 0, 0, 0, 0,
                                None) == 0
    # skinny GEMM: null operands, more than 8 rows, K not a multiple of 8, unaligned A (placeholders, never read)
    assert L.hsg_gemm_bf16_skinny(None, 1024, 256, 1024, 256, 64, 1, 64, 1024, None) == -1
    assert L.hsg_gemm_bf16_skinny(256, 1024, 256, 1024, 256, 64, 9, 64, 1024, None) == -3
    assert L.hsg_gemm_bf16_skinny(256, 1020, 256, 1020, 256, 64, 1, 64, 1020, None) == -2
    assert L.hsg_gemm_bf16_skinny(258, 1024, 256, 1024, 256, 64, 1, 64, 1024, None) == -2
    assert L.hsg_gemm_bf16_skinny(256, 1000, 256, 1024, 256, 64, 1, 64, 1024, None) == -1   # lda < K
    # the SiLU-gated variant needs the gate|up row (2 K) within the row stride
    assert L.hsg_gemm_bf16_skinny_silu(256, 1024, 256, 1024, 256, 64, 1, 64, 1024, None) == -1
    assert L.hsg_gemm_bf16_skinny_silu(256, 2048, 256, 1024, 256, 64, 9, 64, 1024, None) == -3
    # the add + RMSNorm variant: K must be 1024, the residual output a separate buffer
    assert L.hsg_gemm_bf16_skinny_addnorm(256, 1024, 256, 1024, 256, 1e-6, 512, 1024, 256, 1024, 256, 64, 1, 64, 512,
                                          None, None) == -3
    assert L.hsg_gemm_bf16_skinny_addnorm(256, 1024, 256, 1024, 256, 1e-6, 256, 1024, 256, 1024, 256, 64, 1, 64, 1024,
                                          None, None) == -1
    # decode with on-the-fly norm + RoPE: no workspace, another rotary width (placeholders, never read)
    rope = [256, 10240, 512, 256, 1e-6, 256, 10240, 256, 256, 1e-6, 256, 256, 64, 256, 1024, 256, 256, 9, 512, 256,
            10240, 256, 256, 10240, 1024, 512, 256, 256, 256, 256, 256, 256, 2, 4, 4, 256, 0.0625, 1, 256, 4096,
            1024, 256]
    need = L.hsg_ring_decode_workspace_bytes(2, 4, 4, 512)
    assert L.hsg_ring_decode_rope(*rope, None, need, None) == -1
    rope[12] = 32
    assert L.hsg_ring_decode_rope(*rope, 256, need, None) == -3
