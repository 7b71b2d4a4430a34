"""Device-measured MFMA accumulators: tests/golden/mfma_accumulate.npz.

The prefill GEMMs accumulate on v_mfma_f32_32x32x16_bf16, whose rounding the CPU oracle
restates (oracle/csrc/mfma_model.h).  The hardware is the authority for that arithmetic, so
this script records what the device returns: raw FP32 accumulators of plamo_kernel_gemm
(output mode 2) for the inputs `cases()` builds from fixed seeds.  Only the outputs are
stored; tests rebuild the inputs with `cases()` (numpy's PCG64 streams are fixed for a
given seed).

    python tests/golden/make_mfma_fixture.py [OUT]   # on a GPU host, from the repository root

Cases:
  groups    8192 rows, K 128 of which only k < 16 are nonzero, X = 1: one or two groups of
            8 with a dominant term and tiny ones, mixed signs, exponent gaps up to 2^34;
  sums      1024 rows, K 256, X = 1: exponent spreads up to 2^30, 15 % exact zeros;
  products  4 tokens x 1024 rows, K 256: products spread over 2^32;
  realistic 48 tokens x 512 rows, K 1536: weights N(0, 0.02), activations N(0, 1) (the
            projection shapes' statistics: long chains where the accumulator dominates);
  crossing  2048 two-group rows, X = 1: the first group leaves the accumulator just inside
            a power of two, the second carries the sum across it (either way, either sign)
            to 2^-9 ulp from a rounding midpoint, so the floor window decides the rounding.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
OUT = os.path.join(ROOT, "tests", "golden", "mfma_accumulate.npz")


def _bits(v):
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _spread(rng, shape, lo, hi):
    mag = rng.uniform(lo, hi, shape)
    sign = np.sign(rng.standard_normal(shape))
    return (sign * 2.0 ** mag * (1 + rng.integers(0, 128, shape) / 128)).astype(np.float32)


def _sgn(rng, n):
    return np.where(rng.random(n) < 0.5, -1.0, 1.0)


def _crossing(rng, n):
    """Rows [n][128] (BF16 bits): group 1 = {2^top, -+d} gives an FP32-exact accumulator just
    inside a power of two 2^top, group 2 = up to six BF16 pieces (8 significant bits each) of
    a sum that carries the total across 2^top to T = 2^top +- (k + 1/2 +- 2^-9) ulp, all
    terms exact in the group's window.  The floor window of the sum then decides between the
    two neighbours of T."""
    rows = []
    for _ in range(n):
        top = int(rng.integers(-3, 3))
        up = rng.random() < 0.5         # accumulator below 2^top, total above; or the reverse
        sg = -1 if rng.random() < 0.5 else 1
        d = int(rng.integers(128, 256)) << int(rng.integers(6, 12))   # in units of 2^(top-32)
        acc = (1 << 32) - d if up else (1 << 32) + 2 * d              # 2^top -+ d (FP32-exact)
        unit = 1 << 9 if up else 1 << 8                               # ulp of T in 2^(top-32)
        k = int(rng.integers(0, 200))
        off = (2 * k + 1) * unit // 2 + (1 if rng.random() < 0.5 else -1)
        t = (1 << 32) + off if up else (1 << 32) - off
        delta = t - acc
        pieces = []
        rem = abs(delta)
        while rem:
            b = rem.bit_length()
            chunk = (rem >> max(0, b - 8)) << max(0, b - 8)
            pieces.append(chunk)
            rem -= chunk
        assert len(pieces) <= 6
        w = np.zeros(128, np.float64)
        w[0] = 2.0 ** top
        w[1] = (-d if up else 2 * d) * 2.0 ** (top - 32)
        for i, c in enumerate(pieces):
            w[8 + i] = (1 if delta > 0 else -1) * c * 2.0 ** (top - 32)
        rows.append(_bits(w * sg))
    return np.array(rows, np.uint16)


def _bits_to_f32(h):
    return (np.asarray(h, np.uint32) << 16).view(np.float32)


def cases():
    """name -> (W bits [m][k], X bits [tokens][k])."""
    out = {}
    rng = np.random.default_rng(5)
    m, k = 8192, 128
    w = np.zeros((m, k), np.uint16)
    for r in range(m):
        fam = r % 4
        if fam == 0:    # one group: a big term, seven small ones
            w[r, 0] = _bits((1 + rng.integers(0, 128) / 128) * _sgn(rng, 1)[0])
            w[r, 1:8] = _bits((1 + rng.integers(0, 128, 7) / 128) * 2.0 ** rng.integers(-34, -12, 7) * _sgn(rng, 7))
        elif fam == 1:  # one group, no dominant term
            w[r, 0:8] = _bits((1 + rng.integers(0, 128, 8) / 128) * 2.0 ** rng.integers(-10, 0, 8) * _sgn(rng, 8))
        elif fam == 2:  # accumulator from group 1, eight small terms in group 2
            w[r, 0] = _bits((1 + rng.integers(0, 128) / 128) * 2.0 ** rng.integers(-4, 4) * _sgn(rng, 1)[0])
            w[r, 8:16] = _bits((1 + rng.integers(0, 128, 8) / 128) * 2.0 ** rng.integers(-30, -4, 8) * _sgn(rng, 8))
        else:           # two groups, random spread
            w[r, 0:16] = _bits((1 + rng.integers(0, 128, 16) / 128) * 2.0 ** rng.integers(-28, 0, 16) * _sgn(rng, 16))
    out["groups"] = (w, np.full((1, k), _bits(1.0), np.uint16))
    rng = np.random.default_rng(11)
    m, k = 1024, 256
    w = _bits(_spread(rng, (m, k), -30, 0))
    w = np.where(rng.random((m, k)) < 0.15, np.uint16(0), w)
    out["sums"] = (w, np.full((1, k), _bits(1.0), np.uint16))
    out["products"] = (_bits(_spread(rng, (1024, 256), -20, 0)), _bits(_spread(rng, (4, 256), -12, 2)))
    out["realistic"] = (_bits(rng.standard_normal((512, 1536)) * 0.02), _bits(rng.standard_normal((48, 1536))))
    out["crossing"] = (_crossing(np.random.default_rng(17), 2048), np.full((1, 128), _bits(1.0), np.uint16))
    return out


def main():
    sys.path[:0] = [ROOT, os.path.join(ROOT, "plamo3-0.8b-runtime_amd")]
    import torch
    from plamo_hip import native
    lib = native.load()
    res = {}
    for name, (w, x) in cases().items():
        m, k = w.shape
        t = x.shape[0]
        wd = torch.from_numpy(w.view(np.int16)).cuda()
        xd = torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()
        y = torch.zeros(t * m, dtype=torch.float32, device="cuda")
        rc = lib.plamo_kernel_gemm(wd.data_ptr(), 0, xd.data_ptr(), y.data_ptr(), k, m, t, 2, 0)
        torch.cuda.synchronize()
        assert rc == 0, (name, rc)
        res[name] = y.cpu().numpy().reshape(t, m)
        print(name, "recorded", res[name].shape, flush=True)
    out = sys.argv[1] if len(sys.argv) > 1 else OUT
    np.savez_compressed(out, **res)
    print("wrote", out, flush=True)


if __name__ == "__main__":
    main()
