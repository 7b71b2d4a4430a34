""".p12 restatement pinned by the reference's packer self-test, decode KATs and chain cases."""
import numpy as np

from oracle import p12


def test_self_test_vectors_round_trip():
    # pack_weights.py:77-86
    for values in p12.self_test_vectors():
        data, offsets, minima = p12.pack(values)
        entries = p12.tag(offsets, minima)
        codes = entries & 63
        restored = p12.unpack(data, entries & ~np.uint32(63), np.where(codes != 0, codes + 107, 0).astype(np.uint8))
        assert np.array_equal(restored.reshape(-1), values)


def test_all_patterns_block_layout():
    # every BF16 pattern: a block is packed exactly when its nonzero exponents span < 15
    data, offsets, minima = p12.pack(np.arange(65536, dtype=np.uint16))
    blocks = np.arange(65536, dtype=np.uint16).reshape(-1, 128)
    for b in range(512):
        v = blocks[b]
        nz = (v & 0x7FFF) != 0
        e = (v >> 7) & 255
        low = e[nz].min() if nz.any() else 255
        high = e[nz].max() if nz.any() else 0
        ok = 108 <= low <= 170 and high < 255 and int(high) - int(low) < 15
        assert (minima[b] != 0) == ok


def test_decode_known_answers():
    # PackedDecodeTests.swift:8-31: 323,584 words
    payload, table, expected = p12.decode_kat()
    assert expected.size == 323_584
    got = p12.decode_block_words(payload, table, np.arange(expected.size))
    assert np.array_equal(got.astype(np.uint32) << 16, expected)


def test_decode_matches_unpack_on_random_weights():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(128 * 300).astype(np.float32) * 0.02)
    from oracle.bf16 import bits_np
    values = bits_np(w)
    values[:128] = 0x7F80  # a raw block (exponent 255)
    data, offsets, minima = p12.pack(values)
    table = p12.tag(offsets, minima)
    got = p12.decode_block_words(data, table, np.arange(values.size))
    assert np.array_equal(got, values)


def test_chain_validation_cases():
    # PackedFormatTests.swift:25-34 fixed accept/reject answers
    fixed = [([0], 256, True), ([1], 192, True), ([63], 192, True), ([0], 192, False), ([1], 191, False),
             ([65], 192, False), ([0xFFFFFFFF], 192, False)]
    for entries, size, ok in fixed:
        assert p12.validate_chain(entries, size) == ok, (entries, size)
    # PackedFormatTests.swift:58-72 generated cases against its own expectation rule
    for entries, size in p12.chain_cases():
        assert p12.validate_chain(entries, size) == p12.chain_reference(entries, size), (entries, size)
