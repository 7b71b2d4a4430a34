"""BF16 helpers restated from ``Sources/Plamo/Kernels.metal:5-10`` (test infrastructure only).

``bits(x)``  = ``(u + 0x7fff + ((u >> 16) & 1)) >> 16`` on the FP32 bit pattern, with
no NaN special case (a NaN may become +-inf or another NaN, exactly as the Metal code).
``bf(h)``    = ``h << 16`` reinterpreted as FP32.
``roundbf``  = ``bf(bits(x))``.

Pinned by: the closed form on all 2^16 BF16 patterns (round trip is the identity), and
against PyTorch's own ``torch.bfloat16`` conversion (RNE) on every non-NaN FP32 input of a
dense sample that covers all exponents and the tie cases (tests/test_oracle_bf16.py).
"""
import numpy as np
import torch


def bits_np(x):
    """FP32 array -> uint16 BF16 bits (Kernels.metal:6-9)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf_np(h):
    """uint16 BF16 bits -> FP32 (Kernels.metal:5)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def roundbf_np(x):
    return bf_np(bits_np(x))


def bits_t(x):
    """FP32 tensor -> int32 tensor holding the BF16 bit pattern (0..65535)."""
    u = x.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).to(torch.int32) & 0xFFFF


def bf_t(h):
    """int tensor of BF16 bits -> FP32 tensor."""
    return _from_u32((h.to(torch.int64) & 0xFFFF) << 16)


def roundbf_t(x):
    """roundbf on an FP32 tensor (Kernels.metal:10)."""
    u = x.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return _from_u32(r & 0xFFFFFFFF)


def _from_u32(u64):
    # int64 holding a uint32 pattern -> int32 with the same bits -> FP32
    s = torch.where(u64 >= 2**31, u64 - 2**32, u64).to(torch.int32)
    return s.view(torch.float32)
