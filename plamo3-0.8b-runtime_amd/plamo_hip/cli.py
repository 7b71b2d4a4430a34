"""Command-line surface and metrics schema of the reference's `plamo` executable.

`python -m plamo_hip.cli [options] [TEXT]` mirrors Sources/Plamo/Main.swift:
* ``Options``          -- option rules and error strings (Main.swift:6-97);
* ``parse_ids``        -- Main.swift:100-107;
* ``repetition_period``-- Sampler.repetitionPeriod (Sampler.swift:36-51), for --loop-limit;
* ``split_segments``   -- Segment.split (Segments.swift:8-70);
* ``main``             -- Main.execute (Main.swift:126-348): translation on stdout, one JSON
                          metrics line on stderr with the reference's keys (the keys
                          web/server.ts:22-58 reads: runs[0].stop_reason and the error texts).

Differences, each forced by the platform:
* Segment.split asks Apple's NLTokenizer for sentence ends.  Here a sentence ends after a run
  of '.', '!', '?' followed by closing quotes or brackets and then whitespace or the end of
  the line, or after '。', '！', '？', '．', '｡' (plus closing marks) whatever follows.  Every
  other step (grapheme units, the limit*4 window, halving, whitespace literals) is the
  reference's.
* The .p12 archive and auxiliary.safetensors must carry the original model's checksum; a
  model directory of another model (the synthetic test model) names its own in the
  environment variable PLAMO_SOURCE_SHA256.
* Metal memory keys report HIP device memory held by the runtime; the macOS footprint keys
  report VmRSS / VmHWM from /proc/self/status.
"""
import contextlib
import ctypes
import json
import os
import resource
import sys
import tempfile
import time

import regex

from . import Batch, Runtime, Segment, Tokenizer, TokenStream, document_plan
from .native import VOCAB

END_IDS = (1, 16)
# Unicode White_Space: Character.isWhitespace looks at a grapheme's first scalar.
_WHITE = {chr(c) for c in (*range(0x09, 0x0E), 0x20, 0x85, 0xA0, 0x1680, *range(0x2000, 0x200B),
                          0x2028, 0x2029, 0x202F, 0x205F, 0x3000)}
# Character.isNewline.
_NEWLINE = {chr(c) for c in (0x0A, 0x0B, 0x0C, 0x0D, 0x85, 0x2028, 0x2029)}
_CLOSERS = set("\"')]}»”’）」』】］｝〉》")


class Failure(Exception):
    """Failure.message: printed as `error: <message>` with exit status 1 (Main.swift:117-123)."""


def _is_white(ch):
    return ch[:1] in _WHITE


def _is_newline(ch):
    return ch == "\r\n" or ch[:1] in _NEWLINE


_LIBC = ctypes.CDLL(None)
_LIBC.strtof.restype = ctypes.c_float
_LIBC.strtof.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]


def swift_float(text):
    """Float(text) as Swift parses it for the penalty options (Main.swift:74-75 store a Float):
    the C library's strtof over the whole text (decimal or hexadecimal digits, inf, nan), one
    rounding to FP32, out-of-range magnitudes to infinity; None if the text is empty, starts
    with whitespace or has characters strtof does not read.  Returned as a Python float that
    holds the FP32 value exactly, so every later comparison sees what Swift's Float holds:
    "1.00000001" is 1 (no sampling control), "1e39" is infinite (rejected)."""
    if not text or text[0].isspace() or "\0" in text:
        return None
    raw = text.encode()
    buf = ctypes.create_string_buffer(raw)
    end = ctypes.c_void_p()
    value = _LIBC.strtof(buf, ctypes.byref(end))
    if end.value is None or end.value - ctypes.addressof(buf) != len(raw):
        return None
    return float(value)


class Options:
    """Options (Main.swift:6-97): same defaults, ranges, conflicts and messages."""

    def __init__(self, arguments):
        self.model, self.target, self.max_tokens, self.context = "models/plamo", "ja", 256, None
        self.repeats, self.text, self.tokens, self.dump = 1, None, None, None
        self.qsa, self.qsa_budget, self.mtp = False, 2048, False
        self.repetition_penalty, self.frequency_penalty = 1.0, 0.0
        self.no_repeat_ngram, self.loop_limit = 0, 0
        self.packed = self.stream = self.batch4 = self.tokenize = False
        self.segment_tokens, self.decode = 0, None
        flags = {"--qsa": "qsa", "--mtp": "mtp", "--packed": "packed", "--stream": "stream",
                 "--batch4": "batch4", "--tokenize": "tokenize"}
        i = 0
        while i < len(arguments):
            key = arguments[i]
            if key == "--help":
                raise SystemExit(print(HELP) or 0)
            if key in flags:
                setattr(self, flags[key], True)
                i += 1
                continue
            if key.startswith("--"):
                if i + 1 >= len(arguments):
                    raise Failure(f"Missing value for {key}")
                self._value(key, arguments[i + 1])
                i += 2
            else:
                if self.text is not None:
                    raise Failure("Pass source text as a single argument or through stdin")
                self.text = key
                i += 1
        conflicting = ((self.tokens is not None and self.text is not None)
                       or (self.decode is not None and (self.tokens is not None or self.text is not None or self.tokenize))
                       or (self.tokenize and self.tokens is not None)
                       or (self.stream and (self.tokenize or self.decode is not None))
                       or (self.stream and self.repeats > 1)
                       or (self.segment_tokens > 0 and (self.tokenize or self.decode is not None
                                                        or self.tokens is not None or self.dump is not None))
                       or (self.mtp and (self.repetition_penalty != 1 or self.frequency_penalty != 0
                                         or self.no_repeat_ngram > 1 or self.loop_limit > 0)))
        if conflicting:
            raise Failure("Conflicting input options")
        if self.batch4 and not (self.segment_tokens > 0 and (self.context or 1) < 8192 and not self.qsa
                                and not self.mtp and self.repetition_penalty == 1 and self.frequency_penalty == 0
                                and self.no_repeat_ngram == 0 and self.loop_limit == 0):
            raise Failure("Batch4 requires segmented greedy decoding without QSA, MTP or repetition controls")
        if not (self.max_tokens > 0 or (self.tokens is not None and self.dump is not None)):
            raise Failure("Zero output requires --tokens and --dump-logits")

    def _value(self, key, value):
        def integer(lo, hi, message, step=1):
            try:
                n = int(value, 10)
            except ValueError:
                raise Failure(message) from None
            if not (lo <= n <= hi and n % step == 0) or not value.lstrip("+-").isdigit():
                raise Failure(message)
            return n

        def real(ok, message):
            x = swift_float(value)
            if x is None or x != x or x in (float("inf"), float("-inf")) or not ok(x):
                raise Failure(message)
            return x

        if key == "--qsa-budget":
            self.qsa_budget = integer(4, 2048, "QSA budget must be a multiple of four in 4...2048", 4)
            self.qsa = True
        elif key == "--segment-tokens":
            self.segment_tokens = integer(64, 8192, "Segment tokens must be in 64...8192")
        elif key == "--model":
            self.model = value
        elif key == "--to":
            self.target = value
        elif key == "--max-tokens":
            self.max_tokens = integer(0, 32768, "Invalid max-tokens")
        elif key == "--context":
            self.context = integer(1, 32768, "Invalid context")
        elif key == "--repeat":
            self.repeats = integer(1, 100, "Invalid repeat count")
        elif key == "--repetition-penalty":
            self.repetition_penalty = real(lambda x: x > 0, "Repetition penalty must be a positive finite number")
        elif key == "--frequency-penalty":
            self.frequency_penalty = real(lambda x: x >= 0, "Frequency penalty must be a finite nonnegative number")
        elif key == "--no-repeat-ngram":
            self.no_repeat_ngram = integer(0, 64, "No-repeat n-gram must be in 0...64")
        elif key == "--loop-limit":
            self.loop_limit = integer(0, 1000, "Loop limit must be in 0...1000")
        elif key == "--tokens":
            self.tokens = value
        elif key == "--decode":
            self.decode = value
        elif key == "--dump-logits":
            self.dump = value
        else:
            raise Failure(f"Unknown option: {key}")


HELP = """plamo [--model DIR] [--to ja|en|LANG] [--max-tokens N] [--context N] [--repeat N] [--packed] [--stream] \
[--segment-tokens N] [--batch4] [--repetition-penalty F] [--frequency-penalty F] [--no-repeat-ngram N] \
[--loop-limit N] [--qsa] [--qsa-budget N] [--mtp] [TEXT]
Without TEXT, reads UTF-8 from stdin. Translation goes to stdout; JSON metrics to stderr.
--stream writes each decoded token as it is generated, without a trailing newline; not with --repeat > 1.
--segment-tokens bounds each independently translated prompt (64...8192, default off); segments reset KV
and keep the source whitespace between them; --max-tokens applies per segment.
--batch4 batches up to four segments (greedy only, context below 8192; requires --segment-tokens).
--repetition-penalty F, --frequency-penalty F, --no-repeat-ngram N, --loop-limit N as in the reference.
--qsa/--qsa-budget N select sparse global attention; --mtp drafts and verifies tokens (trained adapters).
Verification: --tokenize TEXT | --decode IDS | --tokens IDS --dump-logits FILE [--max-tokens 0]"""


def parse_ids(text):
    """parseIDs (Main.swift:100-107)."""
    parts = text.split(",")
    ids = []
    for p in parts:
        s = p[1:] if p[:1] in "+-" else p
        if s.isdigit() and s.isascii():
            ids.append(int(p))
    if not ids or len(ids) != len(parts) or not all(0 <= i < VOCAB for i in ids):
        raise Failure(f"Expected comma-separated token IDs in 0..<{VOCAB}")
    return ids


def repetition_period(tokens, repeats):
    """Sampler.repetitionPeriod (Sampler.swift:36-51): the smallest period 1...32 whose block
    fills the tail max(repeats, ceil(24/period)) times, else None."""
    if repeats < 2 or len(tokens) < repeats:
        return None
    for period in range(1, 33):
        span = period * max(repeats, (24 + period - 1) // period)
        if len(tokens) < span:
            continue
        start = len(tokens) - span
        if all(tokens[start + k] == tokens[start + k % period] for k in range(span)):
            return period
    return None


def _sentence_ends(chars):
    """Grapheme offsets just past each sentence (stand-in for NLTokenizer(unit: .sentence))."""
    ends, n, i = [], len(chars), 0
    while i < n:
        c = chars[i]
        if c in ("。", "！", "？", "．", "｡") or c in (".", "!", "?"):
            wide = c not in (".", "!", "?")
            j = i + 1
            while j < n and chars[j] in (".", "!", "?", "。", "！", "？", "．", "｡"):
                j += 1
            while j < n and chars[j] in _CLOSERS:
                j += 1
            if wide or j == n or _is_white(chars[j]):
                ends.append(j)
            i = j
            continue
        i += 1
    if not ends or ends[-1] != n:
        ends.append(n)
    return ends


def split_segments(text, target, limit, tokenizer):
    """Segment.split (Segments.swift:8-70) -> [Segment]: the pieces' texts join to `text`;
    text pieces carry their BOS-prefixed prompt tokens (at most `limit`), whitespace runs and
    line breaks are literal pieces without tokens."""
    Tokenizer.prompt(text, target)
    if limit <= 0:
        raise Failure("No context space for a translation segment")
    parts = []

    def literal(s):
        if not s:
            return
        if parts and not parts[-1].tokens:
            parts[-1] = Segment(parts[-1].text + s, [])
        else:
            parts.append(Segment(s, []))

    def line(chars):
        if all(_is_white(c) for c in chars):
            literal("".join(chars))
            return
        ends = _sentence_ends(chars)
        start, n = 0, len(chars)
        while start < n:
            first = start
            while start < n and _is_white(chars[start]):
                start += 1
            literal("".join(chars[first:start]))
            if start == n:
                break
            upper = min(n, start + limit * 4)
            while True:
                inside = [e for e in ends if start < e <= upper]
                end = inside[-1] if inside else upper
                if not inside and upper < n:
                    spaces = [k for k in range(start, upper) if _is_white(chars[k])]
                    if spaces:
                        end = spaces[-1]
                while end > start and _is_white(chars[end - 1]):
                    end -= 1
                source = "".join(chars[start:end])
                tokens = tokenizer.encode(Tokenizer.prompt(source, target), bos=True)
                if len(tokens) <= limit:
                    parts.append(Segment(source, tokens))
                    start = end
                    break
                if end - start <= 1:
                    raise Failure("A single character exceeds the segment token limit")
                upper = start + (end - start) // 2

    pending = []
    for ch in regex.findall(r"\X", text):
        if _is_newline(ch):
            line(pending)
            pending = []
            literal(ch)
        else:
            pending.append(ch)
    line(pending)
    if not any(p.tokens for p in parts):
        raise Failure("Source must contain text")
    return parts


def _text(chunk):
    """A token stream hands out whole UTF-8 characters as bytes."""
    return chunk.decode("utf-8", "replace") if isinstance(chunk, bytes) else chunk


def _device_name():
    hip = ctypes.CDLL("libamdhip64.so")
    name = ctypes.create_string_buffer(256)
    return name.value.decode() if hip.hipDeviceGetName(name, 256, 0) == 0 else "unknown"


def _proc_status(key):
    with open("/proc/self/status") as f:
        for row in f:
            if row.startswith(key + ":"):
                return int(row.split()[1]) * 1024
    return 0


@contextlib.contextmanager
def _device_init_notices(stderr):
    """The first HIP call of a process loads libdrm, which writes one line about a missing
    marketing-name table ("amdgpu.ids: No such file or directory") to file descriptor 2.
    The reference's stderr carries nothing but the metrics line or an error (web/server.ts
    parses all of it as JSON), so that notice is dropped; anything else written to
    descriptor 2 meanwhile is passed on to `stderr`."""
    sys.stderr.flush()
    saved = os.dup(2)
    with tempfile.TemporaryFile() as tmp:
        os.dup2(tmp.fileno(), 2)
        try:
            yield
        finally:
            os.dup2(saved, 2)
            os.close(saved)
            tmp.seek(0)
            for line in tmp.read().decode("utf-8", "replace").splitlines(True):
                if "amdgpu.ids" not in line:
                    stderr.write(line)


def execute(arguments, stdin, stdout, stderr):
    """Main.execute (Main.swift:126-348)."""
    o = Options(arguments)
    tokenizer = Tokenizer(os.path.join(o.model, "tokenizer.jsonl"))
    if o.decode is not None:
        print(tokenizer.decode(parse_ids(o.decode)), file=stdout)
        return
    parts = []
    if o.tokens is not None:
        inputs = parse_ids(o.tokens)
    else:
        text = o.text
        if text is None:
            try:
                text = stdin.buffer.read().decode("utf-8")
            except UnicodeDecodeError:
                raise Failure("Input is not UTF-8") from None
        if o.tokenize:
            stdout.write(json.dumps(tokenizer.encode(text), separators=(",", ":")) + "\n")
            return
        if o.segment_tokens > 0:
            limit = min(o.segment_tokens, (o.context or (8191 if o.batch4 else 32768)) - o.max_tokens)
            parts = split_segments(text, o.target, limit, tokenizer)
            inputs = max((p.tokens for p in parts), key=len)
        else:
            inputs = tokenizer.encode(Tokenizer.prompt(text, o.target), bos=True)
    if not parts:
        parts = [Segment("", inputs)]
    context = o.context or min(32768, len(inputs) + o.max_tokens)
    if len(inputs) + o.max_tokens > context:
        raise Failure("Input plus output limit exceeds context")
    if o.batch4 and context >= 8192:
        raise Failure("Batch4 context must be below 8192")
    load_start = time.time()
    with _device_init_notices(stderr):
        # the .p12 archive and the adapters carry the original model's checksum; a synthetic
        # model directory names its own in PLAMO_SOURCE_SHA256 (test and bench hook)
        runtime = Runtime(o.model, context, packed=o.packed, source_sha256=os.environ.get("PLAMO_SOURCE_SHA256"),
                          qsa_budget=o.qsa_budget if o.qsa else None, mtp=o.mtp)
        plan = document_plan(parts) if o.batch4 else None
        batch = Batch(runtime) if plan is not None and len(plan[0]) > 1 else None
        device = _device_name()
    load_seconds = time.time() - load_start
    controlled = o.repetition_penalty != 1 or o.frequency_penalty != 0 or o.no_repeat_ngram > 1
    runtime.set_sampling(o.repetition_penalty, o.frequency_penalty, 0.0, o.no_repeat_ngram if controlled else 0)
    zero_aux = {"mtp_proposed_tokens": 0, "mtp_accepted_tokens": 0, "mtp_verifications": 0,
                "qsa_queries": 0, "qsa_selected_keys": 0, "qsa_dense_keys": 0}
    runs, translated = [], ""
    for _ in range(o.repeats):
        translated = ""
        if batch is not None:
            chunks = []

            def emit(s):
                if o.stream:
                    stdout.write(s)
                    stdout.flush()
                else:
                    chunks.append(s)

            out = batch.translate_ordered(parts, tokenizer, o.max_tokens, emit)
            translated = "".join(chunks)
            seqs = out["sequences"]
            segs = [{"input_tokens": len(plan[0][k]), "output_tokens": len(ids), "output_ids": ids, "stop_reason": r}
                    for k, (ids, r) in enumerate(seqs)]
            decoded = sum(max(0, len(ids) - (1 if r == "length" else 0)) for ids, r in seqs)
            runs.append(dict(zero_aux, **{
                "input_tokens": sum(s["input_tokens"] for s in segs),
                "prefilled_input_tokens": out["prefilled_input_tokens"],
                "output_tokens": sum(len(ids) for ids, _ in seqs),
                "output_ids": [t for ids, _ in seqs for t in ids], "stop_reason": seqs[-1][1],
                "prefill_seconds": out["prefill_seconds"], "decode_seconds": out["decode_seconds"],
                "decode_tokens_per_second": decoded / max(out["decode_seconds"], 1e-9),
                "gpu_seconds": out["gpu_seconds"], "segments": segs, "segments_total": len(plan[0]),
                "segments_completed": sum(1 for _, r in seqs if r == "stop"),
                "discarded_output_tokens": out["discarded_tokens"]}))
            continue
        seg_runs, adjacent = [], False
        for part in parts:
            if not part.tokens:
                adjacent = False
                if o.stream:
                    stdout.write(part.text)
                else:
                    translated += part.text
                continue
            if adjacent:
                if o.stream:
                    stdout.write("\n")
                else:
                    translated += "\n"
            adjacent = True
            stream = TokenStream(tokenizer) if o.stream else None
            runtime.reset()
            generated, stop = [], None
            proposed = accepted = verifications = 0

            def emit(token):
                if stream is not None:
                    s = _text(stream.push(token))
                    if s:
                        stdout.write(s)
                        stdout.flush()

            start = time.time()
            nxt = runtime.prefill(part.tokens)
            prefill_end = time.time()
            if o.dump is not None:
                tmp = o.dump + ".tmp"
                runtime.logits().astype("<f4").tofile(tmp)
                os.replace(tmp, o.dump)
            if o.mtp:
                # draft, verify the candidates in one sequential pass, keep the agreeing prefix
                # (Main.swift:254-276): the output is the greedy sequence
                while len(generated) < o.max_tokens:
                    if nxt in END_IDS:
                        stop = "stop"
                        break
                    remaining = o.max_tokens - len(generated)
                    if remaining == 1:
                        generated.append(nxt)
                        emit(nxt)
                        break
                    candidates = [nxt]
                    for token in runtime.draft(nxt)[:remaining - 1]:
                        if token in END_IDS:
                            break
                        candidates.append(token)
                    proposed += len(candidates) - 1
                    start_position = runtime.position
                    runtime.forward(candidates, all=True, sequential=True)
                    verified = runtime.predictions()
                    count = 1
                    while count < len(candidates) and candidates[count] == verified[count - 1]:
                        count += 1
                    for token in candidates[:count]:
                        generated.append(token)
                        emit(token)
                    nxt = verified[count - 1]
                    accepted += count - 1
                    verifications += 1
                    runtime.rewind(start_position + count, count - 1)
            else:
                for i in range(o.max_tokens):
                    if nxt in END_IDS:
                        stop = "stop"
                        break
                    generated.append(nxt)
                    runtime.observe(nxt)
                    emit(nxt)
                    if o.loop_limit > 0 and repetition_period(generated, o.loop_limit) is not None:
                        stop = "repeat"
                        break
                    if i + 1 < o.max_tokens:
                        nxt = runtime.forward([nxt])
            end = time.time()
            counters = runtime.stats()
            count = max(0, len(generated) - (1 if stop is None else 0))
            seg_runs.append(dict(zero_aux, **{
                "mtp_proposed_tokens": proposed, "mtp_accepted_tokens": accepted, "mtp_verifications": verifications,
                "qsa_queries": counters["sparse_queries"], "qsa_selected_keys": counters["sparse_keys"],
                "qsa_dense_keys": counters["dense_keys"],
                "input_tokens": len(part.tokens), "output_tokens": len(generated),
                "prefill_seconds": prefill_end - start, "decode_seconds": end - prefill_end,
                "decode_tokens_per_second": count / max(end - prefill_end, 1e-9),
                "gpu_seconds": runtime.gpu_seconds,
                "stop_reason": "prefill" if o.max_tokens == 0 else (stop or "length"), "output_ids": generated}))
            if stream is not None:
                stdout.write(_text(stream.finish()))
                stream.close()
            else:
                translated += tokenizer.decode(generated)
            if stop != "stop":
                break
        if o.segment_tokens > 0:
            run = dict(seg_runs[0])
            for key in ["input_tokens", "output_tokens"] + list(zero_aux):
                run[key] = sum(r[key] for r in seg_runs)
            for key in ("prefill_seconds", "decode_seconds", "gpu_seconds"):
                run[key] = float(sum(r[key] for r in seg_runs))
            tokens = sum(r["decode_tokens_per_second"] * r["decode_seconds"] for r in seg_runs)
            run["decode_tokens_per_second"] = tokens / max(run["decode_seconds"], 1e-9)
            run["output_ids"] = [t for r in seg_runs for t in r["output_ids"]]
            run["stop_reason"] = seg_runs[-1]["stop_reason"]
            run["segments"] = seg_runs
            run["segments_total"] = sum(1 for p in parts if p.tokens)
            run["segments_completed"] = sum(1 for r in seg_runs if r["stop_reason"] == "stop")
            if o.batch4:
                run["prefilled_input_tokens"] = run["input_tokens"]
                run["discarded_output_tokens"] = 0
            runs.append(run)
        else:
            runs += seg_runs
    if not o.stream:
        print(translated, file=stdout)
    stdout.flush()
    stats = runtime.stats()
    metrics = {
        "device": device, "load_seconds": load_seconds, "packed": o.packed, "qsa": o.qsa,
        "qsa_budget": o.qsa_budget if o.qsa else 0, "mtp": o.mtp,
        "repetition_penalty": o.repetition_penalty, "frequency_penalty": o.frequency_penalty,
        "no_repeat_ngram": o.no_repeat_ngram,
        "peak_rss_bytes": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024,
        "physical_footprint_bytes": _proc_status("VmRSS"), "peak_physical_footprint_bytes": _proc_status("VmHWM"),
        "resident_bytes": _proc_status("VmRSS"),
        "metal_allocated_bytes": stats["device_bytes"], "peak_metal_allocated_bytes": stats["device_bytes"],
        "gpu_weight_bytes": stats["weight_bytes"], "auxiliary_weight_bytes": stats["auxiliary_bytes"],
        "context": context, "segment_tokens": o.segment_tokens, "batch4": o.batch4, "runs": runs}
    stderr.write(json.dumps(metrics, sort_keys=True, separators=(",", ":")) + "\n")
    if batch is not None:
        batch.close()
    runtime.close()
    tokenizer.close()


def main(argv=None):
    try:
        execute(sys.argv[1:] if argv is None else argv, sys.stdin, sys.stdout, sys.stderr)
        return 0
    except Failure as e:
        sys.stderr.write(f"error: {e}\n")
        return 1
    except Exception as e:  # PlamoError and the tokenizer's errors carry the reference's texts
        sys.stderr.write(f"error: {e}\n")
        return 1


if __name__ == "__main__":
    sys.exit(main())
