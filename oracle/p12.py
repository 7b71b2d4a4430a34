"""Restatement of the lossless ``.p12`` BF16 packing (test infrastructure only).

Format (``scripts/pack_weights.py:1-5``): a 2-D BF16 tensor is cut into 128-value blocks.
A block whose nonzero exponents lie in ``[low, low+14]`` with ``108 <= low <= 170`` and no
exponent 255 is stored in 192 bytes: 128 sign/mantissa bytes ``(v & 127) | ((v >> 8) & 128)``
followed by 64 bytes of 4-bit codes ``exponent-low`` (two per byte, even index in the low
nibble; code 15 marks +-0).  Any other block is stored raw (256 bytes).  A u32 table entry
per block holds the 64-byte-aligned byte offset of the block in the payload, with
``low-107`` in its low 6 bits (0 = raw).

Functions and what pins them (tests/test_oracle_p12.py):

* ``pack``/``unpack``/``tag``  -- ``pack_weights.py:19-74``.  Pinned by the reference's own
  self-test vectors (``pack_weights.py:77-86``: all 65,536 BF16 patterns, zero blocks, -0
  blocks, the {0,-0,1,-1} tile) and by the bit-exact round trip it asserts.
* ``decode_block_words``       -- the GPU decode ``packed_bits``/``packed_four``
  (``Kernels.metal:23-44``).  Pinned by the known-answer vectors of
  ``Tests/PlamoTests/PackedDecodeTests.swift:8-31`` (323,584 words: 512 raw blocks holding
  every BF16 pattern, and every tag 108..170 x 32 blocks), rebuilt by ``decode_kat``.
* ``validate_chain``           -- the block-table walk of ``Packed.swift:63-89``.  Pinned by
  the accept/reject cases of ``Tests/PlamoTests/PackedFormatTests.swift:25-72``, whose
  independent ``check`` closure is restated by ``chain_reference``.
"""
import numpy as np

BLOCK = 128
MINIMUM_BASE = 107
HEADER = 65536
FORMAT = "plamo-bf16-pack-v2"
REFERENCE_SOURCE_SHA = "7c9f0066d166c075bdbe83ada3d444e08bd7a6ee3f345f47a1f3c442aa6898c5"


def pack(values):
    """pack_weights.py:19-50 -> (data u8, offsets u32, minima u8)."""
    blocks = np.asarray(values, dtype=np.uint16).reshape(-1, BLOCK)
    exponent = (blocks >> 7) & 255
    nonzero = (blocks & 0x7FFF) != 0
    low = np.where(nonzero, exponent, 255).min(axis=1)
    high = np.where(nonzero, exponent, 0).max(axis=1)
    eligible = (low >= 108) & (low <= 170) & (high < 255) & \
        (high.astype(np.int32) - low.astype(np.int32) < 15)
    minima = np.where(eligible, low, 0).astype(np.uint8)
    sizes = np.where(eligible, 192, 256).astype(np.uint32)
    offsets = np.zeros(len(blocks), dtype=np.uint32)
    if len(blocks) > 1:
        np.cumsum(sizes[:-1], out=offsets[1:])
    data = np.empty(int(sizes.sum()), dtype=np.uint8)
    if eligible.any():
        v = blocks[eligible]
        codes = ((v >> 7) & 255).astype(np.int32) - minima[eligible, None].astype(np.int32)
        codes = np.where((v & 0x7FFF) == 0, 15, codes).astype(np.uint8)
        sm = ((v & 127) | ((v >> 8) & 128)).astype(np.uint8)
        enc = np.concatenate([sm, codes[:, 0::2] | (codes[:, 1::2] << 4)], axis=1)
        data[offsets[eligible, None] + np.arange(192)] = enc
    if (~eligible).any():
        raw = blocks[~eligible].copy().view(np.uint8).reshape(-1, 256)
        data[offsets[~eligible, None] + np.arange(256)] = raw
    if not np.array_equal(unpack(data, offsets, minima), blocks):
        raise AssertionError("Packing changed BF16 bits")
    return data, offsets, minima


def unpack(data, offsets, minima):
    """pack_weights.py:53-68."""
    out = np.empty((len(offsets), BLOCK), dtype=np.uint16)
    packed = minima != 0
    if packed.any():
        enc = data[offsets[packed, None].astype(np.int64) + np.arange(192)]
        sm = enc[:, :128].astype(np.uint16)
        nib = enc[:, 128:]
        codes = np.empty((len(enc), BLOCK), dtype=np.uint16)
        codes[:, 0::2] = nib & 15
        codes[:, 1::2] = nib >> 4
        exp = np.where(codes == 15, 0, codes + minima[packed, None].astype(np.uint16))
        out[packed] = (sm & 127) | ((sm & 128) << 8) | (exp << 7)
    if (~packed).any():
        raw = data[offsets[~packed, None].astype(np.int64) + np.arange(256)].copy()
        out[~packed] = raw.view(np.uint16).reshape(-1, BLOCK)
    return out


def tag(offsets, minima):
    """pack_weights.py:71-74: table entry = offset | (minimum-107)."""
    assert np.all((offsets & 63) == 0)
    assert np.all((minima == 0) | ((minima >= 108) & (minima <= 170)))
    return (offsets | np.where(minima != 0, minima.astype(np.uint32) - MINIMUM_BASE, 0)).astype(np.uint32)


def self_test_vectors():
    """The reference packer's self-test inputs (pack_weights.py:79-81)."""
    return [np.arange(65536, dtype=np.uint16), np.zeros(256, dtype=np.uint16),
            np.full(128, 0x8000, dtype=np.uint16),
            np.tile(np.array([0, 0x8000, 0x3F80, 0xBF80], dtype=np.uint16), 64)]


def decode_block_words(payload, table, index):
    """``packed_bits`` (Kernels.metal:23-31) for an array of element indices -> uint16 bits."""
    payload = np.asarray(payload, dtype=np.uint8)
    table = np.asarray(table, dtype=np.uint32)
    index = np.asarray(index, dtype=np.int64)
    entry = table[index // BLOCK]
    t = entry & 63
    start = (entry & ~np.uint32(63)).astype(np.int64)
    i = index % BLOCK
    last = len(payload) - 1  # packed blocks are 192 B: keep the (unused) raw reads in bounds
    raw = payload[np.minimum(start + 2 * i, last)].astype(np.uint16) | \
        (payload[np.minimum(start + 2 * i + 1, last)].astype(np.uint16) << 8)
    sm = payload[np.minimum(start + i, len(payload) - 1)].astype(np.uint32)
    nib = payload[np.minimum(start + 128 + i // 2, len(payload) - 1)].astype(np.uint32)
    code = (nib >> ((i % 2) * 4).astype(np.uint32)) & 15
    exponent = np.where(code == 15, 0, t.astype(np.uint32) + MINIMUM_BASE + code)
    packed = ((sm & 127) | ((sm & 128) << 8) | (exponent << 7)).astype(np.uint16)
    return np.where(t == 0, raw, packed).astype(np.uint16)


def decode_kat():
    """Known-answer vectors of PackedDecodeTests.swift:8-31 -> (payload, table, expected u32)."""
    payload, table, expected = bytearray(), [], []
    for block in range(512):
        table.append(len(payload))
        for i in range(128):
            b = block * 128 + i
            payload += bytes((b & 255, b >> 8))
            expected.append(b << 16)
    for minimum in range(108, 171):
        for block in range(32):
            table.append(len(payload) | (minimum - 107))
            enc = bytearray(192)
            for i in range(128):
                index = block * 128 + i
                sm, code = index // 16, index % 16
                enc[i] = sm & 255
                enc[128 + i // 2] |= (code << ((i % 2) * 4)) & 255
                exponent = 0 if code == 15 else minimum + code
                expected.append(((sm & 127) | ((sm & 128) << 8) | (exponent << 7)) << 16)
            payload += enc
    return (np.frombuffer(bytes(payload), dtype=np.uint8), np.array(table, dtype=np.uint32),
            np.array(expected, dtype=np.uint32))


def validate_chain(entries, data_size):
    """Packed.swift:63-89, restated as a closed form: block sizes are 256 B (tag 0) or
    192 B, every entry's aligned offset must equal the prefix sum of the sizes before it,
    and the sizes must add up to exactly the data region size."""
    e = np.asarray(entries, dtype=np.uint64)
    sizes = np.where((e & 63) == 0, 256, 192).astype(np.uint64)
    starts = np.concatenate([np.zeros(1, np.uint64), np.cumsum(sizes)[:-1]]) if len(e) else e
    return bool(np.array_equal(e & np.uint64(0xFFFFFFC0), starts) and int(sizes.sum()) == int(data_size))


def chain_reference(entries, data_size):
    """The expectation closure of PackedFormatTests.swift:43-50, restated independently."""
    end, valid = 0, True
    for e in entries:
        offset, size = int(e) & ~63 & 0xFFFFFFFF, (256 if int(e) & 63 == 0 else 192)
        if offset != end or offset > data_size - size:
            valid = False
            break
        end = offset + size
    return valid and end == data_size


def chain_cases():
    """Accept/reject cases of PackedFormatTests.swift:25-34,58-72 -> [(entries, bytes)]."""
    cases = [([0], 256), ([1], 192), ([63], 192), ([0], 192), ([1], 191), ([65], 192),
             ([0xFFFFFFFF], 192)]
    for count in range(20):
        entries, end = [], 0
        for i in range(count):
            t = 0 if i % 3 == 0 else (1 if i % 3 == 1 else 63)
            entries.append(end | t)
            end += 256 if t == 0 else 192
        cases.append((list(entries), end))
        for b in [0, max(0, end - 1), end + 1, end + 64]:
            cases.append((list(entries), b))
        for i in range(len(entries)):
            for change in [1, 63, 64, 256, 0xFFFFFFFF]:
                bad = list(entries)
                bad[i] ^= change
                cases.append((bad, end))
    return cases
