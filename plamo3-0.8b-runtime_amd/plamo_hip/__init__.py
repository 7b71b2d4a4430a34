"""Python mirror of the reference's Swift surface over the HIP C ABI.

Names, argument meaning and error behaviour follow the reference:

* ``Runtime``      -- ``Runtime`` (Sources/Plamo/Runtime.swift:128-553): ``forward``,
                      ``prefill``, ``reset``, ``logits``, ``logit_values``, ``predictions``,
                      ``position``, ``gpu_seconds``.
* ``Batch``        -- ``Batch`` (Sources/Plamo/Batch.swift:4-187) and ``Batch.generate``
                      (BatchDecode.swift:40-47).
* ``decode_batch`` -- ``decodeBatch`` (BatchDecode.swift:8-37), native implementation.
* ``pack``         -- ``scripts/pack_weights.py`` through the native packer.

Every call goes to ``lib/libplamo_hip.so``; there is no CPU fallback.
"""
import collections
import ctypes

import numpy as np

from . import native
from .native import PlamoError, VOCAB, HIDDEN, pack

REASONS = {1: "stop", 2: "length"}


def _u16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


class Runtime:
    """Runtime(directory:context:packed:qsaBudget:mtp:) (Runtime.swift:164).  `qsa_budget`
    and `mtp` load the trained adapters of auxiliary.safetensors, whose teacher checksum must
    equal `source_sha256` (None: the reference's pinned value)."""

    def __init__(self, directory, context, packed=False, source_sha256=None, qsa_budget=None, mtp=False):
        lib = native.load()
        h = ctypes.c_void_p()
        sha = source_sha256.encode() if source_sha256 else None
        if qsa_budget is None and not mtp:
            native.call(lib.plamo_open, str(directory).encode(), int(context), 1 if packed else 0, sha,
                        ctypes.byref(h))
        else:
            # None = dense attention (the C ABI's 0); an explicit 0 is a budget, and refused
            budget = 0 if qsa_budget is None else (int(qsa_budget) if int(qsa_budget) != 0 else -1)
            native.call(lib.plamo_open_aux, str(directory).encode(), int(context), 1 if packed else 0, sha,
                        budget, 1 if mtp else 0, ctypes.byref(h))
        self._h = h
        self._lib = lib

    def close(self):
        if getattr(self, "_h", None):
            self._lib.plamo_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self):
        self._lib.plamo_reset(self._h)

    def forward(self, tokens, output=True, all=False, sequential=False):
        """Runtime.forward(_:output:all:sequential:) (Runtime.swift:321-467) -> next token of the
        last row (-1 without output); with `all`, predictions() holds every row's."""
        tokens = [int(t) for t in tokens]
        nxt = ctypes.c_int32(-1)
        if all or sequential:
            native.call(self._lib.plamo_forward_ex, self._h, native.i32(tokens), len(tokens), 1 if output else 0,
                        1 if all else 0, 1 if sequential else 0, ctypes.byref(nxt))
        else:
            native.call(self._lib.plamo_forward, self._h, native.i32(tokens), len(tokens), 1 if output else 0,
                        ctypes.byref(nxt))
        return nxt.value

    def draft(self, first):
        """Runtime.draft(_:) (Runtime.swift:485-520) -> [draft token]."""
        d = ctypes.c_int32(-1)
        native.call(self._lib.plamo_draft, self._h, int(first), ctypes.byref(d))
        return [d.value]

    def rewind(self, new_position, hidden_index):
        """Runtime.rewind(_:hiddenIndex:) (Runtime.swift:527-538)."""
        native.call(self._lib.plamo_rewind, self._h, int(new_position), int(hidden_index))

    def prefill(self, tokens):
        """Runtime.prefill(_:) (Runtime.swift:469-483)."""
        tokens = [int(t) for t in tokens]
        nxt = ctypes.c_int32(-1)
        native.call(self._lib.plamo_prefill, self._h, native.i32(tokens), len(tokens), ctypes.byref(nxt))
        return nxt.value

    def logit_bits(self, slot=0):
        out = np.empty(VOCAB, dtype=np.uint16)
        native.call(self._lib.plamo_logits_bf16, self._h, int(slot), out.ctypes.data_as(native.c_u16p))
        return out

    def logits(self, slot=0):
        """Runtime.logits(into:slot:) (Runtime.swift:547-552)."""
        return _u16_to_f32(self.logit_bits(slot))

    logit_values = logits

    def hidden(self):
        out = np.empty(HIDDEN, dtype=np.float32)
        native.call(self._lib.plamo_hidden, self._h, out.ctypes.data_as(native.c_f32p))
        return out

    def predictions(self):
        buf = (ctypes.c_int32 * 4)()
        n = ctypes.c_int32()
        self._lib.plamo_predictions(self._h, buf, 4, ctypes.byref(n))
        return [buf[i] for i in range(n.value)]

    def stats(self):
        s = native.Stats()
        self._lib.plamo_get_stats(self._h, ctypes.byref(s))
        return {k: getattr(s, k) for k, _ in native.Stats._fields_}

    @property
    def position(self):
        return self.stats()["position"]

    @property
    def gpu_seconds(self):
        return self.stats()["gpu_seconds"]

    @property
    def context(self):
        return self.stats()["context"]

    def kv(self, layer):
        """Layer KV (BF16 bits [capacity][128]) as the reference tests read layer.keys/values."""
        cap = ctypes.c_int32()
        native.call(self._lib.plamo_kv, self._h, int(layer), None, None, ctypes.byref(cap))
        k = np.empty((cap.value, 128), dtype=np.uint16)
        v = np.empty((cap.value, 128), dtype=np.uint16)
        native.call(self._lib.plamo_kv, self._h, int(layer), k.ctypes.data_as(native.c_u16p),
                    v.ctypes.data_as(native.c_u16p), ctypes.byref(cap))
        return k, v

    def set_sampling(self, repetition_penalty=1.0, frequency_penalty=0.0, presence_penalty=0.0,
                     no_repeat_ngram=0):
        """Options --repetition-penalty/--frequency-penalty/--no-repeat-ngram (Main.swift:236-244)."""
        self._lib.plamo_set_sampling(self._h, float(repetition_penalty), float(frequency_penalty),
                                     float(presence_penalty), int(no_repeat_ngram))

    def observe(self, token):
        """generated.append(token) (Main.swift:280): history the sampling controls see."""
        self._lib.plamo_sampler_observe(self._h, int(token))

    def generate(self, prompt, max_tokens):
        """Device-driven token loop of Main.swift:235-288 -> (ids, 'stop' | None)."""
        prompt = [int(t) for t in prompt]
        out = (ctypes.c_int32 * max(1, max_tokens))()
        n, reason = ctypes.c_int32(), ctypes.c_int32()
        native.call(self._lib.plamo_generate, self._h, native.i32(prompt), len(prompt), int(max_tokens), out,
                    ctypes.byref(n), ctypes.byref(reason))
        return [out[i] for i in range(n.value)], ("stop" if reason.value == 1 else None)

    def bench_decode(self, steps):
        ms = ctypes.c_double()
        native.call(self._lib.plamo_bench_decode, self._h, int(steps), ctypes.byref(ms))
        return ms.value


class Batch:
    """Batch(_ scalar:) (Batch.swift:33-78)."""

    def __init__(self, runtime):
        h = ctypes.c_void_p()
        native.call(runtime._lib.plamo_batch_open, runtime._h, ctypes.byref(h))
        self._h, self._lib, self.runtime = h, runtime._lib, runtime

    def close(self):
        if getattr(self, "_h", None):
            self._lib.plamo_batch_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, prompts):
        """Batch.prefill (Batch.swift:80-107)."""
        flat = [int(t) for p in prompts for t in p]
        nxt = (ctypes.c_int32 * 4)()
        native.call(self._lib.plamo_batch_prefill, self._h, native.i32(flat),
                    native.i32([len(p) for p in prompts]), len(prompts), nxt)
        return [nxt[i] for i in range(len(prompts))]

    def step(self, tokens):
        """Batch.step (Batch.swift:109-180): None marks an inactive lane."""
        t = [-1 if x is None else int(x) for x in tokens]
        nxt = (ctypes.c_int32 * 4)()
        native.call(self._lib.plamo_batch_step, self._h, native.i32(t), len(t), nxt)
        return [nxt[i] for i in range(len(t))]

    def reset(self):
        self._lib.plamo_batch_reset(self._h)

    def fill_kv(self, bits):
        """Fills every lane's KV with the BF16 pattern `bits` (the reference test's memset of
        its Metal KV buffers, BatchMapTests.swift:15-18)."""
        if self._lib.plamo_batch_fill_kv(self._h, int(bits) & 0xFFFF) != 0:
            raise native.PlamoError(1, "fill_kv failed")

    def positions(self):
        buf, n = (ctypes.c_int32 * 4)(), ctypes.c_int32()
        self._lib.plamo_batch_positions(self._h, buf, 4, ctypes.byref(n))
        return [buf[i] for i in range(n.value)]

    def logit_bits(self, lane):
        out = np.empty(VOCAB, dtype=np.uint16)
        native.call(self._lib.plamo_batch_logits_bf16, self._h, int(lane), out.ctypes.data_as(native.c_u16p))
        return out

    def hidden(self, lane):
        out = np.empty(HIDDEN, dtype=np.float32)
        native.call(self._lib.plamo_batch_hidden, self._h, int(lane), out.ctypes.data_as(native.c_f32p))
        return out

    def kv(self, lane, layer):
        cap = ctypes.c_int32()
        native.call(self._lib.plamo_batch_kv, self._h, int(lane), int(layer), None, None, ctypes.byref(cap))
        k = np.empty((cap.value, 128), dtype=np.uint16)
        v = np.empty((cap.value, 128), dtype=np.uint16)
        native.call(self._lib.plamo_batch_kv, self._h, int(lane), int(layer), k.ctypes.data_as(native.c_u16p),
                    v.ctypes.data_as(native.c_u16p), ctypes.byref(cap))
        return k, v

    def generate(self, prompts, limits, stop_on_truncation=False):
        """Batch.generate (BatchDecode.swift:40-47) -> [(ids, reason)]."""
        stride = max(1, max(limits))
        ids = (ctypes.c_int32 * (4 * stride))()
        lengths, reasons, lanes = (ctypes.c_int32 * 4)(), (ctypes.c_int32 * 4)(), ctypes.c_int32()
        flat = [int(t) for p in prompts for t in p]
        native.call(self._lib.plamo_batch_generate, self._h, native.i32(flat), native.i32([len(p) for p in prompts]),
                    native.i32(list(limits)), len(prompts), 1 if stop_on_truncation else 0, ids, stride, lengths,
                    reasons, ctypes.byref(lanes))
        return [([ids[i * stride + k] for k in range(lengths[i])], REASONS[reasons[i]]) for i in range(lanes.value)]

    def translate_ordered(self, parts, tokenizer, limit, emit):
        """Batch.translateOrdered (OrderedOutput.swift:79-115): `emit(text)` receives the
        document's text in order; an exception from `emit` cancels and is re-raised ->
        DocumentOutput as a dict with `sequences` [(ids, reason)]."""
        seg = native.Segments(parts)
        failure = []

        def _cb(_, data, n):
            try:
                emit(ctypes.string_at(data, n).decode("utf-8"))
                return 0
            except Exception as e:  # re-raised below
                failure.append(e)
                return 1

        cb = native.TEXT_FN(_cb)
        docs = max(1, sum(1 for p in parts if p.tokens))
        stride = max(1, int(limit))
        ids = (ctypes.c_int32 * (docs * stride))()
        lengths, reasons = (ctypes.c_int32 * docs)(), (ctypes.c_int32 * docs)()
        out = native.DocumentOutput()
        err = ctypes.create_string_buffer(512)
        rc = self._lib.plamo_batch_translate_ordered(self._h, tokenizer._h, *seg.args(), int(limit),
                                                     ctypes.cast(cb, ctypes.c_void_p), None, ids, stride, lengths,
                                                     reasons, ctypes.byref(out), err, 512)
        if failure:
            raise failure[0]
        if rc != 0:
            raise PlamoError(rc, err.value.decode(errors="replace"))
        seqs = [([ids[i * stride + k] for k in range(lengths[i])], REASONS[reasons[i]]) for i in range(out.sequences)]
        return {"sequences": seqs, "gpu_seconds": out.gpu_seconds, "discarded_tokens": out.discarded_tokens,
                "prefilled_input_tokens": out.prefilled_input_tokens, "prefill_seconds": out.prefill_seconds,
                "decode_seconds": out.decode_seconds}

    def decode(self, initial, limits, stop_on_truncation=False):
        """decodeBatch(initial, limits, step: self.step) (BatchDecode.swift:8-37) as a device loop
        after prefill -> [(ids, reason)]."""
        stride = max(1, max(limits))
        ids = (ctypes.c_int32 * (4 * stride))()
        lengths, reasons, lanes = (ctypes.c_int32 * 4)(), (ctypes.c_int32 * 4)(), ctypes.c_int32()
        native.call(self._lib.plamo_batch_decode, self._h, native.i32([int(t) for t in initial]),
                    native.i32(list(limits)), len(initial), 1 if stop_on_truncation else 0, ids, stride, lengths,
                    reasons, ctypes.byref(lanes))
        return [([ids[i * stride + k] for k in range(lengths[i])], REASONS[reasons[i]]) for i in range(lanes.value)]


def decode_batch(initial, limits, step, emit=None, finish=None, stop_on_truncation=False):
    """decodeBatch (BatchDecode.swift:8-37) through the native scheduler -> [(ids, reason)]."""
    lib = native.load()
    count = len(initial)
    failure = []

    def _step(_, tokens, n, out):
        try:
            res = step([None if tokens[i] < 0 else tokens[i] for i in range(n)])
            for i in range(n):
                out[i] = int(res[i]) if i < len(res) else -1
            return 0
        except Exception as e:  # surfaced after the call returns
            failure.append(e)
            return 1

    def _emit(_, lane, token):
        try:
            if emit:
                emit(lane, token)
            return 0
        except Exception as e:
            failure.append(e)
            return 1

    def _finish(_, lane, ids, n, reason):
        try:
            if finish:
                finish(lane, ([ids[i] for i in range(n)], REASONS[reason]))
            return 0
        except Exception as e:
            failure.append(e)
            return 1

    cb = (native.STEP_FN(_step), native.EMIT_FN(_emit), native.FINISH_FN(_finish))
    stride = max(1, max(limits)) if limits else 1
    ids = (ctypes.c_int32 * (4 * stride))()
    lengths, reasons, lanes = (ctypes.c_int32 * 4)(), (ctypes.c_int32 * 4)(), ctypes.c_int32()
    err = ctypes.create_string_buffer(512)
    rc = lib.plamo_decode_batch(native.i32(list(initial)), native.i32(list(limits)), count, cb[0], cb[1], cb[2], None,
                                1 if stop_on_truncation else 0, ids, stride, lengths, reasons, ctypes.byref(lanes),
                                err, 512)
    if failure:
        raise failure[0]
    if rc != 0:
        raise PlamoError(rc, err.value.decode())
    return [([ids[i * stride + k] for k in range(lengths[i])], REASONS[reasons[i]]) for i in range(lanes.value)]


def _bytes_call(fn, *args):
    """Calls a byte-returning entry point twice when the first buffer is too small."""
    n = ctypes.c_size_t(0)
    buf = ctypes.create_string_buffer(256)
    err = ctypes.create_string_buffer(512)
    rc = fn(*args, buf, 256, ctypes.byref(n), err, 512)
    if rc != 0 and n.value > 256:
        buf = ctypes.create_string_buffer(n.value)
        rc = fn(*args, buf, n.value, ctypes.byref(n), err, 512)
    if rc != 0:
        raise PlamoError(rc, err.value.decode(errors="replace"))
    return buf.raw[:n.value]


class Tokenizer:
    """Tokenizer (Tokenizer.swift:11-282) backed by the native library (host code only)."""

    def __init__(self, path):
        lib = native.load()
        self._lib = lib
        h = ctypes.c_void_p()
        native.call(lib.plamo_tokenizer_open, path.encode(), ctypes.byref(h))
        self._h = h

    def close(self):
        if self._h:
            self._lib.plamo_tokenizer_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text, bos=False):
        """Tokenizer.encode(_:bos:) (Tokenizer.swift:144-190)."""
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        n = ctypes.c_size_t(0)
        cap = 2 * len(data) + 8  # at most four byte tokens per scalar, plus BOS
        ids = (ctypes.c_int32 * cap)()
        native.call(self._lib.plamo_tokenizer_encode, self._h, data, len(data), int(bool(bos)), ids, cap,
                    ctypes.byref(n))
        return list(ids[:n.value])

    def decode_bytes(self, ids):
        """Tokenizer.decode(_:) before the UTF-8 repair (Tokenizer.swift:203-232)."""
        return _bytes_call(self._lib.plamo_tokenizer_decode, self._h, native.i32(ids), len(ids))

    def decode(self, ids):
        return self.decode_bytes(ids).decode("utf-8", errors="replace")

    def stream(self):
        return TokenStream(self)

    @staticmethod
    def prompt(text, target):
        """Tokenizer.prompt(_:target:) (Tokenizer.swift:272-281)."""
        data = text.encode("utf-8")
        return _bytes_call(native.load().plamo_translation_prompt, data, len(data), target.encode()).decode("utf-8")


class TokenStream:
    """Tokenizer.Stream (Tokenizer.swift:236-269): bytes of complete UTF-8 sequences."""

    def __init__(self, tokenizer):
        self._t = tokenizer  # keeps the tokenizer alive
        h = ctypes.c_void_p()
        native.call(tokenizer._lib.plamo_token_stream_open, tokenizer._h, ctypes.byref(h))
        self._h = h

    def push(self, token_id):
        return _bytes_call(self._t._lib.plamo_token_stream_push, self._h, int(token_id))

    def finish(self):
        return _bytes_call(self._t._lib.plamo_token_stream_finish, self._h)

    def close(self):
        if self._h:
            self._t._lib.plamo_token_stream_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


TIMELINE_TAGS, TIMELINE_BLOCKS = 256, 1024
TIMELINE_KINDS = {0: "qkv", 1: "attention", 2: "attention_merge", 3: "o", 4: "gate_up", 5: "down"}


def timeline(clear=True):
    """The step timeline of a library built with `make timeline` (plamo_timeline):
    uint64 [256 tags][1024 blocks][start, end] s_memrealtime ticks (100 MHz), zero where a
    block did not run; `clear` zeroes the device table after the copy."""
    out = np.zeros(TIMELINE_TAGS * TIMELINE_BLOCKS * 2, dtype=np.uint64)
    native.call(native.load().plamo_timeline, out.ctypes.data, out.size, 1 if clear else 0)
    return out.reshape(TIMELINE_TAGS, TIMELINE_BLOCKS, 2)


def timeline_name(tag):
    return {200: "head", 250: "head_merge", 251: "step_begin"}.get(
        tag, f"L{tag // 8}.{TIMELINE_KINDS.get(tag % 8, tag % 8)}")


Segment = collections.namedtuple("Segment", "text tokens")
Segment.__doc__ = "A source piece (Segments.swift:4-7): text with prompt tokens, or a whitespace run (no tokens)."


def document_plan(parts):
    """DocumentPlan (OrderedOutput.swift:3-21) -> (inputs, prefixes, tail)."""
    lib = native.load()
    seg = native.Segments(parts)
    h = ctypes.c_void_p()
    native.call(lib.plamo_document_plan, *seg.args(), ctypes.byref(h))
    try:
        n = lib.plamo_plan_documents(h)
        inputs, prefixes = [], []
        for d in range(n + 1):
            ptr, length = ctypes.c_void_p(), ctypes.c_size_t()
            lib.plamo_plan_prefix(h, d, ctypes.byref(ptr), ctypes.byref(length))
            prefixes.append(ctypes.string_at(ptr, length.value).decode("utf-8") if length.value else "")
            if d < n:
                tp, cnt = ctypes.c_void_p(), ctypes.c_int32()
                lib.plamo_plan_input(h, d, ctypes.byref(tp), ctypes.byref(cnt))
                arr = ctypes.cast(tp, ctypes.POINTER(ctypes.c_int32))
                inputs.append([arr[i] for i in range(cnt.value)])
        return inputs, prefixes[:-1], prefixes[-1]
    finally:
        lib.plamo_plan_close(h)


class OrderedOutput:
    """OrderedOutput (OrderedOutput.swift:24-67): `emit(text)` receives UTF-8 text in document
    order; an exception from `emit` cancels the current append/finish and is re-raised."""

    def __init__(self, tokenizer, prefixes, tail, emit):
        self._t, self._emit, self._failure = tokenizer, emit, []

        def _cb(_, data, n):
            try:
                self._emit(ctypes.string_at(data, n).decode("utf-8"))
                return 0
            except Exception as e:  # re-raised by the caller
                self._failure.append(e)
                return 1

        self._cb = native.TEXT_FN(_cb)
        enc = [p.encode("utf-8") for p in prefixes]
        arr = (ctypes.c_char_p * max(1, len(enc)))(*enc)
        lens = (ctypes.c_size_t * max(1, len(enc)))(*[len(e) for e in enc])
        tb = tail.encode("utf-8")
        h = ctypes.c_void_p()
        self._call(tokenizer._lib.plamo_ordered_open, tokenizer._h, arr, lens, len(enc), tb, len(tb),
                   ctypes.cast(self._cb, ctypes.c_void_p), None, ctypes.byref(h))
        self._h = h

    def _call(self, fn, *args):
        err = ctypes.create_string_buffer(512)
        rc = fn(*args, err, 512)
        if self._failure:
            raise self._failure.pop(0)
        if rc != 0:
            raise PlamoError(rc, err.value.decode(errors="replace"))

    def append(self, lane, token_id):
        self._call(self._t._lib.plamo_ordered_append, self._h, int(lane), int(token_id))

    def finish(self, lane, output):
        """`output` is (ids, reason) as decode_batch returns it."""
        self._call(self._t._lib.plamo_ordered_finish, self._h, int(lane), output[1].encode())

    def close(self):
        if getattr(self, "_h", None):
            self._t._lib.plamo_ordered_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
