"""Repeated runs give identical bits: the same prompt prefilled again and again (two chunks,
.p12 weights, the local ring of 4096 slots) and the same decode steps after it.  Every
bit-exactness claim of the other GPU tests assumes this; a race between workgroups, or a
load into LDS still in flight when a workgroup ends, would show here as a run that differs.
"""
import hashlib

import numpy as np
import pytest

import plamo_hip

pytestmark = pytest.mark.gpu


def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("packed,tokens,context", [(True, 4090, 4400), (False, 2048, 2112)])
def test_prefill_and_decode_repeat_bit_for_bit(model_dir, packed, tokens, context):
    d, sha = model_dir
    prompt = np.random.default_rng(7).integers(1024, 107520, tokens).tolist()
    rt = plamo_hip.Runtime(d, context, packed=packed, source_sha256=sha)
    try:
        first, runs = None, 24
        for r in range(runs):
            rt.reset()
            nxt = rt.prefill(prompt)
            pre = _digest(rt.logit_bits(), rt.hidden().view(np.uint32))
            kv = _digest(*[x[:tokens] for l in (0, 7, 15) for x in rt.kv(l)])
            ids = [nxt]
            for _ in range(4):
                ids.append(rt.forward([ids[-1]]))
            key = (pre, kv, _digest(rt.logit_bits()), tuple(ids))
            if first is None:
                first = key
            assert key == first, (packed, tokens, r, [a == b for a, b in zip(key, first)])
        print(f"  packed={packed} {tokens} tokens: {runs} prefills and decodes identical", flush=True)
    finally:
        rt.close()
