"""Host-side checks of the C-ABI library that need no GPU."""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

from oracle import p12, sampler
from plamo_hip import native
import plamo_hip


def test_library_exports_every_declared_symbol():
    lib = native.load()
    declared = native.declared_symbols()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.plamo_version().startswith(b"plamo_hip")


# ------------------------------------------------------------------ .p12 archive writer
def _write_safetensors(path, tensors):
    header, off, blobs = {}, 0, []
    for name, arr in tensors.items():
        b = arr.astype(np.uint16).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    js = json.dumps(header).encode()
    js += b" " * ((-(8 + len(js))) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)) + js + b"".join(blobs))


def _sha(path):
    import hashlib
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def test_packer_matches_oracle_bytes(tmp_path):
    rng = np.random.default_rng(5)
    from oracle.bf16 import bits_np
    w = bits_np(rng.standard_normal((64, 1536)).astype(np.float32) * 0.02)
    w[3, :128] = 0x7F80                       # a raw block
    w[5, 128:256] = 0                         # an all-zero block (raw)
    tensors = {"model.embed_tokens.weight": np.zeros((107520, 1536), np.uint16)[:1],  # replaced below
               "a.weight": w, "n.weight": bits_np(np.ones(1536, np.float32))}
    tensors["model.embed_tokens.weight"] = np.zeros((107520, 1536), np.uint16)
    src = str(tmp_path / "m.safetensors")
    _write_safetensors(src, tensors)
    sha = _sha(src)
    out = str(tmp_path / "m.p12")
    rep = native.pack(src, out, sha)
    with open(out, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
        payload = f.read()
    assert n == 65536 - 8 and hdr["format"] == "plamo-bf16-pack-v2" and hdr["source_sha256"] == sha
    assert "model.embed_tokens.weight" not in hdr["tensors"]
    rec = hdr["tensors"]["a.weight"]
    data, offsets, minima = p12.pack(w)
    table = np.frombuffer(payload[rec["offsets"][0]:rec["offsets"][1]], dtype=np.uint32)
    assert np.array_equal(table, p12.tag(offsets, minima))
    assert payload[rec["data"][0]:rec["data"][1]] == data.tobytes()
    raw = hdr["tensors"]["n.weight"]["raw"]
    assert payload[raw[0]:raw[1]] == tensors["n.weight"].tobytes()
    assert rep["blocks"] == 64 * 12 and rep["compressed_blocks"] == int((minima != 0).sum())
    # the archive validates (Packed.tensor) and the table walks
    ok = ctypes.c_int32()
    shape = (ctypes.c_int64 * 2)(64, 1536)
    native.call(native.load().plamo_check_packed, out.encode(), sha.encode(), b"a.weight", shape, 2,
                ctypes.byref(ok))
    assert ok.value == 1
    with pytest.raises(native.PlamoError, match="checksum"):
        native.pack(src, out, "0" * 64)


def _archive(path, entries, nbytes, fmt="plamo-bf16-pack-v2", base=107, table_bytes=None, sha="s" * 64):
    # PackedFormatTests.swift:10-24
    start = max(64, (len(entries) * 4 + 63) // 64 * 64)
    header = {"format": fmt, "block": 128, "minimum_base": base, "source_sha256": sha,
              "payload_bytes": start + nbytes,
              "tensors": {"w": {"shape": [1, len(entries) * 128],
                                "offsets": [0, table_bytes if table_bytes is not None else len(entries) * 4],
                                "data": [start, start + nbytes]}}}
    js = json.dumps(header).encode()
    length = (len(js) + 8 + 63) // 64 * 64 - 8
    blob = struct.pack("<Q", length) + js + b" " * (length - len(js))
    blob += np.asarray(entries, dtype=np.uint32).tobytes() + bytes(start - len(entries) * 4 + nbytes)
    with open(path, "wb") as f:
        f.write(blob)


def _check(path, n, sha="s" * 64):
    ok = ctypes.c_int32()
    shape = (ctypes.c_int64 * 2)(1, n * 128)
    err = ctypes.create_string_buffer(512)
    rc = native.load().plamo_check_packed(path.encode(), sha.encode(), b"w", shape, 2, ctypes.byref(ok), err, 512)
    return rc, err.value.decode()


def test_packed_chain_validation(tmp_path):
    path = str(tmp_path / "a.p12")
    for entries, nbytes in p12.chain_cases():
        if not entries:
            continue
        _archive(path, entries, nbytes)
        rc, msg = _check(path, len(entries))
        assert (rc == 0) == p12.validate_chain(entries, nbytes), (entries, nbytes, msg)
    _archive(path, [1], 192, table_bytes=3)
    assert _check(path, 1)[0] != 0
    for fmt, base in (("plamo-bf16-pack-v1", 107), ("plamo-bf16-pack-v2", 106)):
        _archive(path, [1], 192, fmt=fmt, base=base)
        rc, msg = _check(path, 1)
        assert rc != 0 and "scripts/pack_weights.py" in msg
    _archive(path, [1], 192, sha="t" * 64)
    assert "scripts/pack_weights.py" in _check(path, 1)[1]


def test_malformed_weights(tmp_path):
    # PlamoTests.swift:141-154
    path = str(tmp_path / "bad.safetensors")
    lib = native.load()
    err = ctypes.create_string_buffer(256)
    assert lib.plamo_check_weights(path.encode(), None, None, 0, err, 256) != 0
    for data in [b"", b"\xff" * 16, bytes([8, 0, 0, 0, 0, 0, 0, 0]) + b"{}      "]:
        with open(path, "wb") as f:
            f.write(data)
        assert lib.plamo_check_weights(path.encode(), None, None, 0, err, 256) != 0
        assert lib.plamo_check_packed(path.encode(), None, None, None, 0, None, err, 256) != 0


def test_weights_tensor_validation(model_dir):
    d, _ = model_dir
    lib = native.load()
    err = ctypes.create_string_buffer(256)
    path = os.path.join(d, "model.safetensors").encode()
    good = (ctypes.c_int64 * 2)(2304, 1536)
    assert lib.plamo_check_weights(path, b"model.layers.layers.0.mixer.qkv_proj.weight", good, 2, err, 256) == 0
    bad = (ctypes.c_int64 * 2)(1536, 2304)
    assert lib.plamo_check_weights(path, b"model.layers.layers.0.mixer.qkv_proj.weight", bad, 2, err, 256) != 0
    assert b"Missing or incompatible BF16 tensor" in err.value


def test_synthetic_model_identity(model_dir, golden):
    d, sha = model_dir
    assert sha == golden["synthetic_model"]["sha256"]
    from oracle.model import read_safetensors
    t = read_safetensors(os.path.join(d, "model.safetensors"), names={"model.norm.weight",
                                                                      "model.layers.layers.0.post_mixer_norm.weight",
                                                                      "model.layers.layers.0.post_mlp_norm.weight"})
    from oracle.bf16 import bf_np, roundbf_np
    assert np.all(roundbf_np(bf_np(t["model.norm.weight"]) + np.float32(1.0)) == 1.0)
    assert np.all(roundbf_np(bf_np(t["model.layers.layers.0.post_mixer_norm.weight"]) + np.float32(0.2)) == 1.0)
    off = np.float32(1 / 5.0 ** 1.5)
    assert np.all(roundbf_np(bf_np(t["model.layers.layers.0.post_mlp_norm.weight"]) + off) == 1.0)


def test_open_without_device_fails_loudly(model_dir):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(native.PlamoError, match="HIP device"):
        plamo_hip.Runtime(model_dir[0], 96)


def test_open_with_adapters_validates_in_the_reference_order(model_dir, tmp_path):
    # Runtime.init (Runtime.swift:166-178): the context, then the QSA budget, then
    # auxiliary.safetensors, all before the model or a device is touched (on this CPU-only
    # host the next step is the device check)
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    d, sha = model_dir
    bare = tmp_path / "no_adapters"
    bare.mkdir()
    for name in os.listdir(d):
        if name != "auxiliary.safetensors":
            os.symlink(os.path.join(d, name), bare / name)
    budget = "QSA budget must be a multiple of four in 4...2048"
    missing = "Trained adapters missing; run scripts/train_auxiliary.py --collect"
    for context in (0, 32769):
        with pytest.raises(native.PlamoError, match=r"Context must be 1\.\.\.32768"):
            plamo_hip.Runtime(bare, context, source_sha256=sha, qsa_budget=3)
    for b in (0, 3, 6, 2052, -4):
        with pytest.raises(native.PlamoError, match=budget):
            plamo_hip.Runtime(bare, 64, source_sha256=sha, qsa_budget=b, mtp=True)
    for kw in ({"qsa_budget": 16}, {"mtp": True}, {"qsa_budget": 2048, "mtp": True}):
        with pytest.raises(native.PlamoError, match=missing):
            plamo_hip.Runtime(bare, 64, source_sha256=sha, **kw)
    # adapters trained against another model are refused before the device as well
    with pytest.raises(native.PlamoError, match="Incompatible trained adapters"):
        plamo_hip.Runtime(d, 64, qsa_budget=16)
    # valid adapters pass: the device check comes next
    with pytest.raises(native.PlamoError, match="HIP device"):
        plamo_hip.Runtime(d, 64, source_sha256=sha, qsa_budget=16, mtp=True)


# ---------------------------------------------------------- native decodeBatch (host)
def _bytes_ids(text):
    return [b + 384 if b < 128 else b for b in text.encode()]


def _simulate(texts, limits, run):
    source = [_bytes_ids(t) for t in texts]
    cursor = [0] * len(texts)
    calls = []

    def nxt():
        return [source[i][cursor[i]] if cursor[i] < len(source[i]) else (1 if i % 2 == 0 else 16)
                for i in range(len(source))]

    def step(tokens):
        calls.append(list(tokens))
        for lane, t in enumerate(tokens):
            if t is not None:
                cursor[lane] += 1
        return nxt()

    return run(nxt(), limits, step, stop_on_truncation=True), calls


@pytest.mark.parametrize("texts,limits", [(["AAA", "B", "あ", ""], [20] * 4),
                                          (["AAA", "BBBB", "C", "DDDD"], [20, 2, 20, 20]),
                                          (["AAAA", "BBBB", "CCCC", "D"], [2, 20, 1, 20]),
                                          (["A", "B"], [0, 20])])
def test_native_decode_batch_matches_oracle(texts, limits):
    got, gcalls = _simulate(texts, limits, plamo_hip.decode_batch)
    want, wcalls = _simulate(texts, limits, sampler.decode_batch)
    assert got == want and gcalls == wcalls


def test_native_decode_batch_finish_order():
    calls, finished, pending = [], [], [[1, 16, 100, 201], [1, 16, 100, 202]]

    def step(t):
        calls.append(list(t))
        return pending.pop(0)

    out = plamo_hip.decode_batch([1, 16, 100, 200], [9, 9, 1, 3], step, finish=lambda lane, _: finished.append(lane))
    assert [ids for ids, _ in out] == [[], [], [100], [200, 201, 202]]
    assert [r for _, r in out] == ["stop", "stop", "length", "length"]
    assert calls == [[None, None, None, 200], [None, None, None, 201]]
    assert finished == [0, 1, 2, 3]
    with pytest.raises(native.PlamoError, match="Invalid quad decode inputs"):
        plamo_hip.decode_batch([5], [8192], lambda t: t)
    with pytest.raises(native.PlamoError, match="Invalid quad predictions"):
        plamo_hip.decode_batch([5], [3], lambda t: [107520])


def test_attention_decode_rejects_bad_geometry():
    # plamo_kernel_attention_decode validates its geometry on the host before any device work
    import ctypes
    from plamo_hip import native
    lib = native.load()
    pos = (ctypes.c_int32 * 1)(100)
    # global position past the capacity; local window larger than the ring; five rows
    assert lib.plamo_kernel_attention_decode(1, 1, 1, 1, 1, 100, pos, 1, 1, 1, 1, 1, 0) != 0
    assert lib.plamo_kernel_attention_decode(1, 1, 1, 1, 1, 50, pos, 1, 0, 1, 1, 1, 0) != 0
    pos5 = (ctypes.c_int32 * 5)(1, 1, 1, 1, 1)
    assert lib.plamo_kernel_attention_decode(1, 1, 1, 1, 1, 100, pos5, 5, 1, 1, 1, 1, 0) != 0
    neg = (ctypes.c_int32 * 1)(-1)
    assert lib.plamo_kernel_attention_decode(1, 1, 1, 1, 1, 100, neg, 1, 1, 1, 1, 1, 0) != 0
