"""bf16 / fp16 rounding helpers for the CPU oracle (test infrastructure only).

bf16 rounding is IEEE round-to-nearest-even on the upper 16 bits of an fp32, which is what torch's
``.to(torch.bfloat16)`` and Triton's ``.to(tl.bfloat16)`` do. Pinned in tests against torch's own cast.
"""
import contextlib

import numpy as np

_ROUND = [True]


@contextlib.contextmanager
def exact():
    """Within this context ``bf16`` returns its input in float64 (no rounding): the composition of the
    oracle can then be compared with an unrounded library forward at float64 precision."""
    _ROUND[0] = False
    try:
        yield
    finally:
        _ROUND[0] = True


def bf16(x):
    """Round to the nearest bf16 value (ties to even); returns float32 values."""
    if not _ROUND[0]:
        return np.asarray(x, dtype=np.float64)
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out


def fp16(x):
    """Round to the nearest IEEE half value; returns float32 values."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def silu(x):
    """x / (1 + exp(-x)) (fused_kernels.py:24-26, torch's silu)."""
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-x))
