"""BF16 rounding of the oracle (Kernels.metal:5-10) pinned against PyTorch's RNE conversion."""
import numpy as np
import torch

from oracle.bf16 import bf_np, bits_np, bits_t, roundbf_np, roundbf_t


def test_round_trip_all_patterns():
    h = np.arange(65536, dtype=np.uint16)
    f = bf_np(h)
    finite = ~np.isnan(f)
    assert np.array_equal(bits_np(f)[finite], h[finite])


def test_matches_torch_rne_on_dense_sample():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    # every exponent plus exact ties (low half 0x8000) and their neighbours
    ties = (np.arange(0, 2**16, dtype=np.uint32) << 16) | 0x8000
    u = np.concatenate([u, ties, ties - 1, ties + 1])
    x = u.view(np.float32)
    ok = ~np.isnan(x) & ~np.isinf(x)
    expect = torch.from_numpy(x[ok]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits_np(x[ok]), expect)


def test_torch_and_numpy_paths_agree():
    x = torch.randn(100000) * 37.0
    assert torch.equal(roundbf_t(x), torch.from_numpy(roundbf_np(x.numpy())))
    assert np.array_equal(bits_t(x).numpy().astype(np.uint16), bits_np(x.numpy()))


def test_no_nan_special_case():
    # 0xFFFFFFFF wraps to 0 exactly like the Metal expression (no NaN handling)
    x = np.array([0xFFFFFFFF, 0x7FFFFFFF, 0x7F7FFFFF], dtype=np.uint32).view(np.float32)
    assert bits_np(x).tolist() == [0x0000, 0x8000, 0x7F80]
