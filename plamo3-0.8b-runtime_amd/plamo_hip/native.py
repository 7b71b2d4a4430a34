"""ctypes binding of lib/libplamo_hip.so (include/plamo_hip.h).

The library is the product: there is no Python or CPU fallback.  ``load()`` raises when the
shared library has not been built (``make -C plamo3-0.8b-runtime_amd``).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libplamo_hip.so")
# the same library with the step timeline compiled in (make timeline)
TIMELINE_LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libplamo_hip_timeline.so")
# the host code built with AddressSanitizer (make asan; needs the sanitizer runtime preloaded)
ASAN_LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libplamo_hip_asan.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "plamo_hip.h")

VOCAB, HIDDEN = 107520, 1536
c_i32p = ctypes.POINTER(ctypes.c_int32)
c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_f32p = ctypes.POINTER(ctypes.c_float)


class Stats(ctypes.Structure):
    _fields_ = [("position", ctypes.c_int64), ("gpu_seconds", ctypes.c_double),
                ("device_bytes", ctypes.c_int64), ("weight_bytes", ctypes.c_int64),
                ("linear_bytes", ctypes.c_int64), ("context", ctypes.c_int32),
                ("packed", ctypes.c_int32), ("last_output_rows", ctypes.c_int32),
                ("local_capacity", ctypes.c_int32), ("last_prefill_seconds", ctypes.c_double),
                ("last_decode_seconds", ctypes.c_double), ("auxiliary_bytes", ctypes.c_int64),
                ("sparse_queries", ctypes.c_int64), ("sparse_keys", ctypes.c_int64), ("dense_keys", ctypes.c_int64)]


class PackReport(ctypes.Structure):
    _fields_ = [("original_linear_bytes", ctypes.c_int64), ("packed_linear_bytes", ctypes.c_int64),
                ("archive_bytes", ctypes.c_int64), ("compressed_blocks", ctypes.c_int64),
                ("blocks", ctypes.c_int64)]


STEP_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p)
EMIT_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32)
FINISH_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, c_i32p, ctypes.c_int32, ctypes.c_int32)

_SIGNATURES = {
    "plamo_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_char_p,
                                  ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_open_aux": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_char_p,
                                      ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                      ctypes.c_size_t]),
    "plamo_forward_ex": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, c_i32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_draft": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_i32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_rewind": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_char_p,
                                    ctypes.c_size_t]),
    "plamo_close": (None, [ctypes.c_void_p]),
    "plamo_reset": (None, [ctypes.c_void_p]),
    "plamo_forward": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, ctypes.c_int32, c_i32p,
                                     ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_prefill": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p, ctypes.c_char_p,
                                     ctypes.c_size_t]),
    "plamo_logits": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_f32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_logits_bf16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_u16p, ctypes.c_char_p,
                                         ctypes.c_size_t]),
    "plamo_hidden": (ctypes.c_int, [ctypes.c_void_p, c_f32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_predictions": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p]),
    "plamo_get_stats": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Stats)]),
    "plamo_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_u16p, c_u16p, c_i32p, ctypes.c_char_p,
                                ctypes.c_size_t]),
    "plamo_set_sampling": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                          ctypes.c_int32]),
    "plamo_sampler_observe": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    "plamo_generate": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, ctypes.c_int32, c_i32p, c_i32p,
                                      c_i32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_bench_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_double),
                                          ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_batch_open": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                        ctypes.c_size_t]),
    "plamo_batch_close": (None, [ctypes.c_void_p]),
    "plamo_batch_prefill": (ctypes.c_int, [ctypes.c_void_p, c_i32p, c_i32p, ctypes.c_int32, c_i32p,
                                           ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_batch_step": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p, ctypes.c_char_p,
                                        ctypes.c_size_t]),
    "plamo_batch_reset": (None, [ctypes.c_void_p]),
    "plamo_batch_logits_bf16": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_u16p, ctypes.c_char_p,
                                               ctypes.c_size_t]),
    "plamo_batch_hidden": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, c_f32p, ctypes.c_char_p,
                                          ctypes.c_size_t]),
    "plamo_batch_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, c_u16p, c_u16p, c_i32p,
                                      ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_batch_fill_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint16]),
    "plamo_batch_positions": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p]),
    "plamo_decode_batch": (ctypes.c_int, [c_i32p, c_i32p, ctypes.c_int32, STEP_FN, EMIT_FN, FINISH_FN,
                                          ctypes.c_void_p, ctypes.c_int32, c_i32p, ctypes.c_int32, c_i32p, c_i32p,
                                          c_i32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_batch_generate": (ctypes.c_int, [ctypes.c_void_p, c_i32p, c_i32p, c_i32p, ctypes.c_int32,
                                            ctypes.c_int32, c_i32p, ctypes.c_int32, c_i32p, c_i32p, c_i32p,
                                            ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_batch_decode": (ctypes.c_int, [ctypes.c_void_p, c_i32p, c_i32p, ctypes.c_int32, ctypes.c_int32, c_i32p,
                                          ctypes.c_int32, c_i32p, c_i32p, c_i32p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_pack": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(PackReport),
                                  ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_pack_tensor": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p,
                                         ctypes.c_size_t]),
    "plamo_check_aux": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_check_weights": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                           ctypes.c_int32, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_check_packed": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                          ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, c_i32p, ctypes.c_char_p,
                                          ctypes.c_size_t]),
    "plamo_kernel_linear": (ctypes.c_int, [ctypes.c_uint64] * 4 + [ctypes.c_int32] * 4 + [ctypes.c_uint64]),
    "plamo_kernel_unpack": (ctypes.c_int, [ctypes.c_uint64] * 3 + [ctypes.c_int64, ctypes.c_uint64]),
    "plamo_kernel_argmax": (ctypes.c_int, [ctypes.c_uint64] * 2 + [ctypes.c_int32] * 3 + [ctypes.c_uint64]),
    "plamo_kernel_qsa_select": (ctypes.c_int, [ctypes.c_uint64] + [ctypes.c_int32] * 4 + [ctypes.c_uint64] * 2),
    "plamo_kernel_select": (ctypes.c_int, [ctypes.c_uint64, ctypes.c_int32, ctypes.c_uint64, ctypes.c_int32,
                                           ctypes.c_float, ctypes.c_int32, ctypes.c_float, ctypes.c_float,
                                           ctypes.c_uint64, ctypes.c_uint64]),
    "plamo_kernel_gemm": (ctypes.c_int, [ctypes.c_uint64] * 4 + [ctypes.c_int32] * 4 + [ctypes.c_uint64]),
    "plamo_kernel_attention_prefill": (ctypes.c_int, [ctypes.c_uint64] * 3 + [ctypes.c_int32] * 4 +
                                       [ctypes.c_uint64] * 3),
    "plamo_kernel_attention_decode": (ctypes.c_int, [ctypes.c_uint64] * 5 + [ctypes.c_int32, c_i32p,
                                                                           ctypes.c_int32, ctypes.c_int32] +
                                      [ctypes.c_uint64] * 4),
    "plamo_kernel_attention_decode_static": (ctypes.c_int, [ctypes.c_uint64] * 5 +
                                             [ctypes.c_int32, c_i32p, ctypes.c_int32, ctypes.c_int32] +
                                             [ctypes.c_uint64] * 4 + [ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_rope_table": (ctypes.c_int, [ctypes.POINTER(ctypes.c_double), ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_version": (ctypes.c_char_p, []),
    "plamo_tokenizer_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                            ctypes.c_size_t]),
    "plamo_tokenizer_close": (None, [ctypes.c_void_p]),
    "plamo_tokenizer_encode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_int32,
                                              c_i32p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                              ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_tokenizer_decode": (ctypes.c_int, [ctypes.c_void_p, c_i32p, ctypes.c_size_t, ctypes.c_char_p,
                                              ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p,
                                              ctypes.c_size_t]),
    "plamo_token_stream_open": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                               ctypes.c_size_t]),
    "plamo_token_stream_push": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_char_p, ctypes.c_size_t,
                                               ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_token_stream_finish": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t,
                                                 ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_token_stream_close": (None, [ctypes.c_void_p]),
    "plamo_ordered_open": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_char_p),
                                          ctypes.POINTER(ctypes.c_size_t), ctypes.c_int32, ctypes.c_char_p,
                                          ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p, ctypes.c_size_t]),
    "plamo_ordered_append": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_char_p,
                                            ctypes.c_size_t]),
    "plamo_ordered_finish": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_char_p, ctypes.c_char_p,
                                            ctypes.c_size_t]),
    "plamo_ordered_close": (None, [ctypes.c_void_p]),
    "plamo_translation_prompt": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_char_p,
                                                ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p,
                                                ctypes.c_size_t]),
    "plamo_timeline": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_char_p,
                                      ctypes.c_size_t]),
    "plamo_document_plan": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p,
                                           ctypes.c_size_t]),
    "plamo_plan_documents": (ctypes.c_int32, [ctypes.c_void_p]),
    "plamo_plan_input": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p),
                                        ctypes.POINTER(ctypes.c_int32)]),
    "plamo_plan_prefix": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p),
                                         ctypes.POINTER(ctypes.c_size_t)]),
    "plamo_plan_close": (None, [ctypes.c_void_p]),
    "plamo_batch_translate_ordered": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                                     ctypes.c_void_p, ctypes.c_void_p, c_i32p, ctypes.c_int32, c_i32p,
                                                     c_i32p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]),
}


class DocumentOutput(ctypes.Structure):
    _fields_ = [("sequences", ctypes.c_int32), ("gpu_seconds", ctypes.c_double),
                ("discarded_tokens", ctypes.c_int64), ("prefilled_input_tokens", ctypes.c_int64),
                ("prefill_seconds", ctypes.c_double), ("decode_seconds", ctypes.c_double)]


class Segments:
    """Segment arrays for the C ABI (texts, lengths, token arrays, counts); keeps the
    buffers alive for the duration of a call."""

    def __init__(self, parts):
        self.enc = [p.text.encode("utf-8") for p in parts]
        self.tok = [i32([int(t) for t in p.tokens]) for p in parts]
        n = max(1, len(parts))
        self.texts = (ctypes.c_char_p * n)(*self.enc)
        self.lens = (ctypes.c_size_t * n)(*[len(e) for e in self.enc])
        self.tokens = (ctypes.c_void_p * n)(*[ctypes.cast(t, ctypes.c_void_p) for t in self.tok])
        self.counts = i32([len(p.tokens) for p in parts])
        self.count = len(parts)

    def args(self):
        return (ctypes.cast(self.texts, ctypes.c_void_p), ctypes.cast(self.lens, ctypes.c_void_p),
                ctypes.cast(self.tokens, ctypes.c_void_p), ctypes.cast(self.counts, ctypes.c_void_p), self.count)

TEXT_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t)

_lib = None


class PlamoError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def load():
    """Load the HIP library (raises if it is missing: the product has no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libplamo_hip.so not built: {LIB_PATH} (run make -C plamo3-0.8b-runtime_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def declared_symbols():
    """Function names declared in include/plamo_hip.h."""
    import re
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(plamo_[a-z0-9_]+)\s*\(", text)) - {"plamo_step_fn", "plamo_emit_fn",
                                                                         "plamo_finish_fn"})


def call(fn, *args):
    err = ctypes.create_string_buffer(512)
    rc = fn(*args, err, 512)
    if rc != 0:
        raise PlamoError(rc, err.value.decode(errors="replace"))


def check_aux(path, teacher_sha256=None, mtp=True, qsa=True):
    """Auxiliary.init and its tensor checks (Auxiliary.swift:14-62) without a device."""
    call(load().plamo_check_aux, str(path).encode(), teacher_sha256.encode() if teacher_sha256 else None,
         1 if mtp else 0, 1 if qsa else 0)


def i32(values):
    arr = (ctypes.c_int32 * max(1, len(values)))(*values)
    return arr


def pack(source, output, source_sha256=None):
    """scripts/pack_weights.py (pack_weights.py:89-142) through the native packer."""
    rep = PackReport()
    call(load().plamo_pack, source.encode(), output.encode(),
         source_sha256.encode() if source_sha256 else None, ctypes.byref(rep))
    return {k: getattr(rep, k) for k, _ in PackReport._fields_}


def pack_tensor(bits):
    """pack_weights.py pack()+tag() for one BF16 array -> (payload u8, table u32)."""
    import numpy as np
    bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    payload = np.empty(bits.size * 2, dtype=np.uint8)
    table = np.empty(bits.size // 128, dtype=np.uint32)
    n = ctypes.c_int64()
    call(load().plamo_pack_tensor, bits.ctypes.data, bits.size, payload.ctypes.data, payload.size,
         table.ctypes.data, ctypes.byref(n))
    return payload[:n.value].copy(), table
