"""bf16 / fp16 rounding helpers for the CPU oracle (test infrastructure only).

bf16 rounding is IEEE round-to-nearest-even on the upper 16 bits of an fp32, which is what torch's
``.to(torch.bfloat16)`` and Triton's ``.to(tl.bfloat16)`` do. Pinned in tests against torch's own cast.
"""
import contextlib

import numpy as np

_ROUND = [True]
_FLIP_ULPS = [0]


@contextlib.contextmanager
def exact():
    """Within this context ``bf16`` returns its input in float64 (no rounding): the composition of the
    oracle can then be compared with an unrounded library forward at float64 precision."""
    _ROUND[0] = False
    try:
        yield
    finally:
        _ROUND[0] = True


@contextlib.contextmanager
def perturbed(ulps):
    """Within this context ``bf16`` rounds every value that lies within ``ulps`` fp32 ulps of a bf16 rounding tie
    to the other of its two bf16 neighbours. An evaluation of the same formulas in fp32 (as any GPU kernel, the
    reference's Triton kernels included, computes them) carries errors of a few fp32 ulps, so it may round
    exactly these values either way: the oracle run perturbed and unperturbed brackets how far two equally
    valid fp32 implementations can drift apart, which is the noise floor an end-to-end comparison must be read
    against. About (2 ulps + 1) / 65536 of all roundings change."""
    previous = _FLIP_ULPS[0]
    _FLIP_ULPS[0] = int(ulps)
    try:
        yield
    finally:
        _FLIP_ULPS[0] = previous


def bf16(x):
    """Round to the nearest bf16 value (ties to even); returns float32 values."""
    if not _ROUND[0]:
        return np.asarray(x, dtype=np.float64)
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32)
    # uint32 arithmetic: finite values and infinities cannot carry past bit 31; NaNs are restored below
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    if _FLIP_ULPS[0]:
        # within _FLIP_ULPS of the tie (low half 0x8000): take the other neighbour (truncation or the next value
        # up in magnitude, whichever round-to-nearest-even did not pick)
        low = (u & np.uint32(0xFFFF)).astype(np.int64)
        near = (np.abs(low - 0x8000) <= _FLIP_ULPS[0]) & np.isfinite(x)
        if near.any():
            down = u & np.uint32(0xFFFF0000)
            r = np.where(near, np.where(r == down, down + np.uint32(0x10000), down), r)
    out = r.view(np.float32)
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
