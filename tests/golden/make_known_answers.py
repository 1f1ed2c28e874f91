"""Generate tests/golden/known_answers.json: hand-checkable MaxSim cases in
exact rational arithmetic (fractions.Fraction), independent of numpy/torch.

The inputs are small integer vectors (and, for normalize=True, integer
vectors with integer L2 norms, so the normalised dot products are exact
rationals). The expected outputs follow the scalar definition the reference
states in reference.py:13-15:

    score[i, j] = sum_{s : q_mask[i, s]} max_{t : d_mask[j, t]} Q[i, s] . D[j, t]

with an empty max contributing 0 (reference.py:82-85). Residual cases follow
the byte layout of reference.py:124-139 (little-endian within a byte).

Run: python tests/golden/make_known_answers.py  (rewrites the JSON).
"""

import json
import random
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).with_name("known_answers.json")

# integer vectors (padded to d=8) whose L2 norm is an integer
UNIT_BASIS = [
    ([1, 2, 2], 3), ([2, 3, 6], 7), ([1, 4, 8], 9), ([2, 6, 9], 11), ([3, 4, 0], 5),
    ([4, 4, 7], 9), ([1, 2, 2, 4], 5), ([2, 4, 5, 6], 9), ([0, 0, 3, 4], 5), ([6, 2, 3], 7),
]


def maxsim_exact(Q, D, qm, dm):
    out = []
    for i, q in enumerate(Q):
        row = []
        for j, dd in enumerate(D):
            total = Fraction(0)
            for s, qs in enumerate(q):
                if not qm[i][s]:
                    continue
                best = None
                for t, dt in enumerate(dd):
                    if not dm[j][t]:
                        continue
                    v = sum((Fraction(a) * Fraction(b) for a, b in zip(qs, dt)), Fraction(0))
                    best = v if best is None or v > best else best
                total += best if best is not None else 0
            row.append(total)
        out.append(row)
    return out


def rand_unit(rng, d):
    base, n = rng.choice(UNIT_BASIS)
    v = [0] * d
    pos = rng.sample(range(d), len(base))
    for p, b in zip(pos, base):
        v[p] = b * rng.choice([-1, 1])
    return v, n


def main():
    rng = random.Random(1234)
    cases = []
    # 1) raw integers with masks, incl. fully masked doc and query rows
    d = 8
    Q = [[[rng.randint(-3, 3) for _ in range(d)] for _ in range(3)] for _ in range(2)]
    D = [[[rng.randint(-3, 3) for _ in range(d)] for _ in range(5)] for _ in range(4)]
    qm = [[1, 0, 1], [1, 1, 1]]
    dm = [[1, 1, 0, 1, 0], [0, 0, 0, 0, 0], [1, 1, 1, 1, 1], [0, 1, 0, 0, 1]]
    exp = maxsim_exact(Q, D, qm, dm)
    cases.append({"name": "int_masked", "normalize": False, "Q": Q, "D": D, "q_mask": qm, "d_mask": dm,
                  "expected": [[float(x) for x in r] for r in exp]})
    # 2) all dots negative: the max is negative and must be kept (not clamped to 0)
    Qn = [[[1, 0, 0, 0, 0, 0, 0, 0], [0, 2, 0, 0, 0, 0, 0, 0]]]
    Dn = [[[-1, 0, 0, 0, 0, 0, 0, 0], [0, -3, 0, 0, 0, 0, 0, 0], [-2, -1, 0, 0, 0, 0, 0, 0]]]
    exp = maxsim_exact(Qn, Dn, [[1, 1]], [[1, 1, 1]])
    cases.append({"name": "negative_max", "normalize": False, "Q": Qn, "D": Dn, "q_mask": [[1, 1]],
                  "d_mask": [[1, 1, 1]], "expected": [[float(x) for x in r] for r in exp]})
    # 3) normalize=True with integer-norm vectors; stored raw (scaled by k) so the
    #    kernel/oracle must normalise; expected uses the exact unit vectors.
    Qr, Qu, Dr, Du = [], [], [], []
    for _ in range(2):
        rows_r, rows_u = [], []
        for _ in range(4):
            v, n = rand_unit(rng, d)
            k = rng.randint(1, 3)
            rows_r.append([k * x for x in v])
            rows_u.append([Fraction(x, n) for x in v])
        Qr.append(rows_r)
        Qu.append(rows_u)
    for _ in range(3):
        rows_r, rows_u = [], []
        for _ in range(6):
            v, n = rand_unit(rng, d)
            k = rng.randint(1, 4)
            rows_r.append([k * x for x in v])
            rows_u.append([Fraction(x, n) for x in v])
        Dr.append(rows_r)
        Du.append(rows_u)
    qm3 = [[1, 1, 1, 0], [1, 1, 1, 1]]
    dm3 = [[1, 1, 1, 1, 1, 1], [1, 0, 1, 0, 1, 0], [1, 1, 1, 1, 0, 0]]
    exp = maxsim_exact(Qu, Du, qm3, dm3)
    cases.append({"name": "normalized_exact", "normalize": True, "Q": Qr, "D": Dr, "q_mask": qm3, "d_mask": dm3,
                  "expected": [[float(x) for x in r] for r in exp]})

    # residual byte decoding, little-endian within a byte
    resid = []
    for nbits in (2, 4, 8):
        cpb = 8 // nbits
        dd = 16
        codes = [rng.randrange(1 << nbits) for _ in range(dd)]
        packed = [0] * ((dd * nbits + 7) // 8)
        for f, c in enumerate(codes):
            packed[f // cpb] |= c << ((f % cpb) * nbits)
        resid.append({"nbits": nbits, "d": dd, "bytes": packed, "codes": codes})
    # hand example: 0xE4 = 0b11_10_01_00 -> 2-bit fields [0, 1, 2, 3]
    resid.append({"nbits": 2, "d": 4, "bytes": [0xE4], "codes": [0, 1, 2, 3]})
    resid.append({"nbits": 4, "d": 2, "bytes": [0x5A], "codes": [0xA, 0x5]})

    # top-k with ties: expected order = score desc, then lower index
    scores = [3.0, 1.0, 3.0, 2.0, 3.0, 1.0, 0.5, 2.0]
    order = sorted(range(len(scores)), key=lambda i: (-scores[i], i))
    topk = {"scores": scores, "k": 5, "largest_idx": order[:5],
            "smallest_idx": sorted(range(len(scores)), key=lambda i: (scores[i], i))[:5]}

    OUT.write_text(json.dumps({"maxsim": cases, "residual_decode": resid, "topk": topk}, separators=(",", ":")))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
