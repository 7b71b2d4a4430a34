"""The PLaMo unigram tokenizer restated in plain Python (test infrastructure only).

* ``Vocab``          -- ``Tokenizer.init(path:)`` / ``append`` (Tokenizer.swift:59-131): one
  JSON array ``[piece, score, kind]`` per non-empty line; BYTE pieces ``<0xNN>`` (NN read as
  Swift's ``Int(_:radix:16)`` does, sign allowed) map bytes to ids and score 0; other pieces
  score ``round_half_even(score * 1e4)``; a repeated piece keeps its last id; the vocabulary
  must have 107,520 entries, every byte, and ``<|plamo:bos|>`` / ``<|plamo:tag|>`` at 1 / 16.
* ``segments``       -- the boundary regex and U+EE00 split (Tokenizer.swift:41-43,144-151)
  with Python's ``re`` engine and ICU's ``\\s`` (``[\\t\\n\\f\\r\\p{Z}]``) spelled out.
  Pinned by hand cases in ``tests/test_tokenizer.py``.
* ``encode``         -- the Viterbi of Tokenizer.swift:152-186 over every substring looked up
  in a dict (no trie): cost of a scalar's byte fallback 10,000,000, of a piece ``-score``,
  ties to the longer piece.  Pinned by brute force over all segmentations of short inputs
  (minimum total cost) and by hand tie cases.
* ``decode_bytes`` / ``stream`` -- Tokenizer.swift:203-269.  Pinned by round trips and the
  stream invariant (concatenated pushes + finish == decode).
"""
import json
import math
import re

MARK = "\uee00"
_ICU_SPACE = "\t\n\f\r\u0020\u00a0\u1680\u2000-\u200a\u2028\u2029\u202f\u205f\u3000"
BOUNDARY = re.compile(r"(<\|plamo:[^|" + _ICU_SPACE + r"\x1c-\x1f]{0,64}\|>)|(([^\n])\3{3,}| {2,})")
FALLBACK = 10_000_000
VOCAB_SIZE = 107520


def byte_value(piece):
    """Swift's Int(piece.dropFirst(3).dropLast(), radix: 16) for a '<0xNN>' piece, or None."""
    if len(piece) != 6 or not piece.startswith("<0x") or not piece.endswith(">"):
        return None
    body = piece[3:5]
    sign = 1
    if body[0] in "+-":
        sign, body = (-1 if body[0] == "-" else 1), body[1:]
    if not body or any(c not in "0123456789abcdefABCDEF" for c in body):
        return None
    return sign * int(body, 16)


class Vocab:
    def __init__(self, path):
        self.pieces, self.scores, self.bytes = [], [], [-1] * 256
        self.lookup = {}
        self.max_span = 1
        with open(path, encoding="utf-8") as f:
            for line in f.read().split("\n"):
                if not line:
                    continue
                piece, score, kind = json.loads(line)[:3]
                ident = len(self.pieces)
                self.pieces.append(piece)
                if kind == "BYTE":
                    b = byte_value(piece)
                    if b is None or not 0 <= b < 256:
                        raise ValueError("Invalid byte token")
                    self.bytes[b] = ident
                    self.scores.append(0)
                    continue
                scaled = round(score * 1e4)  # Python rounds half to even
                if not math.isfinite(score * 1e4) or not -2 ** 63 <= scaled < 2 ** 63:
                    raise ValueError("Invalid tokenizer score")
                self.scores.append(scaled)
                self.max_span = max(self.max_span, len(piece))
                self.lookup[piece] = ident
        if (len(self.pieces) != VOCAB_SIZE or min(self.bytes) < 0 or self.pieces[1] != "<|plamo:bos|>"
                or self.pieces[16] != "<|plamo:tag|>"):
            raise ValueError("Expected the PLaMo 3 Translate 0.8B vocabulary")


def segments(text):
    marked = BOUNDARY.sub(lambda m: MARK + m.group(0) + MARK, text)
    return [s for s in marked.split(MARK) if s]


def viterbi(v, seg):
    """(tokens, total cost) of one segment (Tokenizer.swift:152-186)."""
    n = len(seg)
    cost = [0] * (n + 1)
    length, token = [1] * n, [-1] * n
    for i in range(n - 1, -1, -1):
        best = cost[i + 1] + FALLBACK
        for j in range(i, min(n, i + v.max_span)):
            t = v.lookup.get(seg[i:j + 1])
            if t is not None and cost[j + 1] - v.scores[t] <= best:
                best = cost[j + 1] - v.scores[t]
                length[i], token[i] = j - i + 1, t
        cost[i] = best
    out, i = [], 0
    while i < n:
        if token[i] >= 0:
            out.append(token[i])
        else:
            out.extend(v.bytes[b] for b in seg[i].encode("utf-8"))
        i += length[i]
    return out, cost[0]


def encode(v, text, bos=False):
    out = [1] if bos else []
    for seg in segments(text):
        out.extend(viterbi(v, seg)[0])
    return out


def brute_min_cost(v, seg):
    """Minimum total cost over every split of `seg` into pieces and byte-fallback scalars."""
    best = [0] + [None] * len(seg)
    for end in range(1, len(seg) + 1):
        cands = [best[end - 1] + FALLBACK]
        for start in range(end):
            t = v.lookup.get(seg[start:end])
            if t is not None:
                cands.append(best[start] - v.scores[t])
        best[end] = min(cands)
    return best[len(seg)]


def decode_bytes(v, ids):
    out = bytearray()
    for i in ids:
        if not 0 <= i < len(v.pieces):
            raise ValueError("Token ID out of range")
        b = byte_value(v.pieces[i])
        out += bytes([b]) if b is not None and 0 <= b < 256 else v.pieces[i].encode("utf-8")
    return bytes(out)
