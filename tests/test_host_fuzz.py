"""Seeded mutations of the files the host code reads: safetensors weights
(plamo_check_weights, Runtime.swift:33-101), .p12 archives (plamo_check_packed,
Packed.swift:12-91), auxiliary.safetensors (plamo_check_aux, Auxiliary.swift:14-62) and the
tokenizer file (plamo_tokenizer_open, Tokenizer.swift:90-118).

Every reader takes every mutated file without crashing and either accepts it or returns an
error with a message.  Mutations that break the container (truncation, the header length,
offsets past the end, sizes that overflow) are always rejected.  tests/test_host_asan.py runs
this file against the host code built with AddressSanitizer, so an out-of-bounds read in a
reader on any of these inputs fails there.
"""
import ctypes
import json
import os
import random
import struct

import numpy as np
import pytest

from oracle import p12
from plamo_hip import native, synth

N_MUTATIONS = 40


def _safetensors(tensors):
    header, off, blobs = {}, 0, []
    for name, arr in tensors.items():
        b = arr.astype(np.uint16).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    js = json.dumps(header).encode()
    js += b" " * ((8 - len(js) % 8) % 8)
    return struct.pack("<Q", len(js)) + js + b"".join(blobs)


def _p12(entries, nbytes):
    # a valid chain of `entries` block-table words (PackedFormatTests.swift:10-24)
    start = max(64, (len(entries) * 4 + 63) // 64 * 64)
    header = {"format": "plamo-bf16-pack-v2", "block": 128, "minimum_base": 107, "source_sha256": "s" * 64,
              "payload_bytes": start + nbytes,
              "tensors": {"w": {"shape": [1, len(entries) * 128], "offsets": [0, len(entries) * 4],
                                "data": [start, start + nbytes]}}}
    js = json.dumps(header).encode()
    length = (len(js) + 8 + 63) // 64 * 64 - 8
    blob = struct.pack("<Q", length) + js + b" " * (length - len(js))
    return blob + np.asarray(entries, dtype=np.uint32).tobytes() + bytes(start - len(entries) * 4 + nbytes)


def _header_span(blob):
    n = struct.unpack("<Q", blob[:8])[0]
    return 8, 8 + min(n, len(blob) - 8)


def _json_edits(blob, rng):
    """Semantic edits of the JSON header: numbers replaced by extremes, keys dropped."""
    lo, hi = _header_span(blob)
    try:
        header = json.loads(blob[lo:hi].decode())
    except (UnicodeDecodeError, ValueError):
        return None
    extremes = [-1, 0, 1, 2 ** 31, 2 ** 32 + 7, 2 ** 62, 2 ** 63 - 1, 2 ** 64 + 1, 10 ** 30]

    def edit(node, depth=0):
        if isinstance(node, dict) and node:
            k = rng.choice(sorted(node))
            if rng.random() < 0.15:
                del node[k]
            else:
                node[k] = edit(node[k], depth + 1)
        elif isinstance(node, list) and node:
            i = rng.randrange(len(node))
            node[i] = edit(node[i], depth + 1)
        elif isinstance(node, (int, float)) and not isinstance(node, bool):
            return rng.choice(extremes)
        elif isinstance(node, str):
            return rng.choice(["", "F32", "BF16", node + "x", node[:-1]])
        return node

    header = edit(header)
    js = json.dumps(header).encode()
    js += b" " * (hi - lo - len(js)) if len(js) < hi - lo else b""
    return struct.pack("<Q", len(js)) + js + blob[hi:]


def _mutations(blob, seed, header_only=False):
    """Yields (kind, mutated bytes, must_fail)."""
    rng = random.Random(seed)
    lo, hi = _header_span(blob)
    yield "empty", b"", True
    yield "length only", blob[:8], True
    yield "header length huge", struct.pack("<Q", 2 ** 63 + 5) + blob[8:], True
    yield "header length past the end", struct.pack("<Q", len(blob)) + blob[8:], True
    for _ in range(N_MUTATIONS):
        r = rng.random()
        if r < 0.25:
            cut = rng.randrange(1, len(blob))
            yield "truncated", blob[:cut], True
        elif r < 0.55:
            b = bytearray(blob)
            for _ in range(rng.randint(1, 4)):
                b[rng.randrange(lo, hi)] = rng.randrange(256)
            yield "header bytes", bytes(b), False
        elif r < 0.85:
            m = _json_edits(blob, rng)
            if m is not None:
                yield "header field", m, False
        elif not header_only:
            b = bytearray(blob)
            for _ in range(rng.randint(1, 16)):
                b[rng.randrange(hi, len(blob))] = rng.randrange(256)
            yield "payload bytes", bytes(b), False


def _run(tmp_path, name, blob, check):
    path = str(tmp_path / name)
    with open(path, "wb") as f:
        f.write(blob)
    rc, msg = check(path)
    assert rc == 0 or msg, f"error without a message for {name}"
    return rc


def _err():
    return ctypes.create_string_buffer(512)


def test_weights_reader_mutations(tmp_path):
    # Weights(path:) requires the input embedding at open (Runtime.swift:33-50): the files are
    # the header plus a sparse payload of the embedding's and a small tensor's size
    lib = native.load()
    emb = 107520 * 1536 * 2
    header = {"model.embed_tokens.weight": {"dtype": "BF16", "shape": [107520, 1536], "data_offsets": [0, emb]},
              "a": {"dtype": "BF16", "shape": [4, 16], "data_offsets": [emb, emb + 128]}}
    js = json.dumps(header).encode()
    js += b" " * ((-(8 + len(js))) % 8)
    head = struct.pack("<Q", len(js)) + js
    size = len(head) + emb + 128

    def write(name, head_bytes, total, patches=()):
        path = str(tmp_path / name)
        with open(path, "wb") as f:
            f.write(head_bytes[:total])
            f.truncate(total)
            for off, b in patches:
                if off < total:
                    f.seek(off)
                    f.write(b)
        return path

    def check(path):
        err = _err()
        shape = (ctypes.c_int64 * 2)(4, 16)
        rc = lib.plamo_check_weights(path.encode(), b"a", shape, 2, err, 512)
        msg = err.value.decode(errors="replace")
        assert rc == 0 or msg, path
        os.remove(path)
        return rc

    assert check(write("ok.safetensors", head, size)) == 0
    rng = random.Random(1)
    cases = [("empty", b"", 0, True), ("length only", head, 8, True),
             ("header length huge", struct.pack("<Q", 2 ** 63 + 5) + head[8:], size, True),
             ("header length past the end", struct.pack("<Q", size) + head[8:], size, True)]
    for _ in range(N_MUTATIONS):
        r = rng.random()
        if r < 0.25:
            cases.append(("truncated", head, rng.randrange(1, size), True))
        elif r < 0.55:
            b = bytearray(head)
            for _ in range(rng.randint(1, 4)):
                b[rng.randrange(8, len(head))] = rng.randrange(256)
            cases.append(("header bytes", bytes(b), size, False))
        else:
            m = _json_edits(head + bytes(8), rng)
            if m is not None:
                m = m[:len(m) - 8]
                cases.append(("header field", m, len(m) + emb + 128, False))
    for i, (kind, h, total, must_fail) in enumerate(cases):
        rc = check(write(f"w{i}.safetensors", h, total))
        assert not (must_fail and rc == 0), kind


def test_packed_reader_mutations(tmp_path):
    lib = native.load()
    # the longest valid block-table chain of the reference's chain cases (oracle/p12.py)
    entries, nbytes = max(((e, n) for e, n in p12.chain_cases() if e and p12.validate_chain(e, n)),
                          key=lambda c: len(c[0]))
    blob = _p12(entries, nbytes)

    def check(path):
        err, ok = _err(), ctypes.c_int32()
        shape = (ctypes.c_int64 * 2)(1, len(entries) * 128)
        rc = lib.plamo_check_packed(path.encode(), b"s" * 64, b"w", shape, 2, ctypes.byref(ok), err, 512)
        return rc, err.value.decode(errors="replace")

    assert _run(tmp_path, "ok.p12", blob, check) == 0
    for i, (kind, m, must_fail) in enumerate(_mutations(blob, 2)):
        rc = _run(tmp_path, f"p{i}.p12", m, check)
        assert not (must_fail and rc == 0), kind


def test_auxiliary_reader_mutations(tmp_path, model_dir):
    lib = native.load()
    d, sha = model_dir
    with open(os.path.join(d, "auxiliary.safetensors"), "rb") as f:
        blob = f.read()

    def check(path):
        err = _err()
        rc = lib.plamo_check_aux(path.encode(), sha.encode(), 1, 1, err, 512)
        return rc, err.value.decode(errors="replace")

    assert _run(tmp_path, "ok.aux", blob, check) == 0
    for i, (kind, m, must_fail) in enumerate(_mutations(blob, 3)):
        rc = _run(tmp_path, f"a{i}.safetensors", m, check)
        assert not (must_fail and rc == 0), kind


def test_tokenizer_reader_mutations(tmp_path):
    lib = native.load()
    path, _ = synth.ensure_tokenizer()
    with open(path, "rb") as f:
        text = f.read()
    lines = text.split(b"\n")
    rng = random.Random(4)

    def check(p):
        err, handle = _err(), ctypes.c_void_p()
        rc = lib.plamo_tokenizer_open(p.encode(), ctypes.byref(handle), err, 512)
        if rc == 0:
            lib.plamo_tokenizer_close(handle)
        return rc, err.value.decode(errors="replace")

    cases = [("empty", b"", True), ("one line", lines[0] + b"\n", True)]
    for _ in range(N_MUTATIONS // 2):
        r = rng.random()
        if r < 0.3:
            cases.append(("truncated", text[:rng.randrange(1, len(text))], False))
        elif r < 0.7:
            b = bytearray(text)
            for _ in range(rng.randint(1, 8)):
                b[rng.randrange(len(b))] = rng.choice(b'[]{}",:\\0123456789-eE \x00\xff\xc3')
            cases.append(("bytes", bytes(b), False))
        else:
            ls = list(lines)
            i = rng.randrange(len(ls) - 1)
            ls[i] = rng.choice([b"", b"[]", b'["a"]', b'["a", "x", "NORMAL"]', b'["a", 1e999, "NORMAL"]',
                                b'["", -1.0, "BYTE"]', b'["\\ud800", -1.0, "NORMAL"]', b"[" * 200])
            cases.append(("line", b"\n".join(ls), False))
    for i, (kind, m, must_fail) in enumerate(cases):
        rc = _run(tmp_path, f"t{i}.jsonl", m, check)
        assert not (must_fail and rc == 0), kind
