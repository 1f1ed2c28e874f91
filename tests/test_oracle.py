"""Pins the CPU oracle (oracle/lik_oracle.py) before anything is checked against it.

Each check is independent of the oracle's own formula: pure-Python brute
force loops, exact known answers (tests/golden/known_answers.json, made with
fractions.Fraction), closed forms, cross-identities between entry points,
and torch's fp8 cast as the library routine for e4m3 rounding.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import lik_oracle as O

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def brute(Q, D, qm=None, dm=None):
    """Triple loop, reference tests/test_reference_cpu.py:117-145 pattern."""
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    out = np.zeros((Nq, Nd))
    for i in range(Nq):
        for j in range(Nd):
            tot = 0.0
            for s in range(Lq):
                if qm is not None and not qm[i, s]:
                    continue
                best = -np.inf
                for t in range(Ld):
                    if dm is not None and not dm[j, t]:
                        continue
                    best = max(best, float(sum(float(a) * float(b) for a, b in zip(Q[i, s], D[j, t]))))
                tot += best if best != -np.inf else 0.0
            out[i, j] = tot
    return out


@pytest.mark.parametrize("case", GOLD["maxsim"], ids=lambda c: c["name"])
def test_oracle_known_answers(case):
    got = O.maxsim(np.array(case["Q"], float), np.array(case["D"], float),
                   np.array(case["q_mask"], bool), np.array(case["d_mask"], bool), normalize=case["normalize"])
    np.testing.assert_allclose(got, np.array(case["expected"]), rtol=0, atol=1e-12)


@pytest.mark.parametrize("masks", ["none", "q", "d", "both"])
@pytest.mark.parametrize("normalize", [False, True])
def test_oracle_matches_bruteforce(masks, normalize):
    rng = np.random.default_rng(7)
    Q = rng.standard_normal((3, 5, 8))
    D = rng.standard_normal((4, 7, 8))
    qm = rng.random((3, 5)) > 0.3 if masks in ("q", "both") else None
    dm = rng.random((4, 7)) > 0.3 if masks in ("d", "both") else None
    if dm is not None:
        dm[1] = False  # a fully masked doc
    got = O.maxsim(Q, D, qm, dm, normalize=normalize)
    Qb = Q / np.linalg.norm(Q, axis=-1, keepdims=True) if normalize else Q
    Db = D / np.linalg.norm(D, axis=-1, keepdims=True) if normalize else D
    np.testing.assert_allclose(got, brute(Qb, Db, qm, dm), atol=1e-12)


def test_oracle_closed_forms():
    # identical rows after normalisation: every valid query token's max is 1
    rng = np.random.default_rng(1)
    X = rng.standard_normal((1, 6, 16))
    got = O.maxsim(X * 3.0, X * 0.5, normalize=True)
    assert abs(got[0, 0] - 6.0) < 1e-12
    # orthogonal supports: all dots 0 -> score 0
    Q = np.zeros((1, 2, 4)); Q[0, :, :2] = 1
    D = np.zeros((1, 3, 4)); D[0, :, 2:] = 1
    assert O.maxsim(Q, D)[0, 0] == 0.0
    # fully masked query row and doc contribute 0, never -inf
    got = O.maxsim(rng.standard_normal((2, 3, 4)), rng.standard_normal((2, 3, 4)),
                   np.array([[0, 0, 0], [1, 1, 1]], bool), np.array([[0, 0, 0], [1, 1, 1]], bool))
    assert np.all(got[0] == 0) and np.all(got[:, 0] == 0) and np.isfinite(got).all()
    # zero vector under normalize: eps clamp gives 0, not NaN
    Z = np.zeros((1, 1, 4))
    assert O.maxsim(Z, np.ones((1, 2, 4)), normalize=True)[0, 0] == 0.0


def test_oracle_squeeze_and_1d_masks():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((5, 8))
    d = rng.standard_normal((6, 8))
    assert O.maxsim(q, d).shape == ()
    assert O.maxsim(q, d[None]).shape == (1,)
    assert O.maxsim(q[None], d).shape == (1,)
    qm = np.array([1, 0, 1, 1, 0], bool)
    dm = np.array([1, 1, 0, 1, 0, 1], bool)
    np.testing.assert_allclose(O.maxsim(q[None], d[None], qm, dm), O.maxsim(q[None], d[None], qm[None], dm[None]))


def test_oracle_varlen_pairs_padded_kd_agree():
    rng = np.random.default_rng(3)
    ql = [3, 0, 5]
    dl = [4, 1, 0, 6]
    d = 8
    Qp = rng.standard_normal((sum(ql), d))
    Dp = rng.standard_normal((sum(dl), d))
    cu_q = np.concatenate([[0], np.cumsum(ql)])
    cu_d = np.concatenate([[0], np.cumsum(dl)])
    v = O.maxsim_varlen(Qp, Dp, cu_q, cu_d)
    # padded + masks view of the same data
    Qpad = np.zeros((3, 5, d)); Dpad = np.zeros((4, 6, d))
    for i, L in enumerate(ql):
        Qpad[i, :L] = Qp[cu_q[i]:cu_q[i + 1]]
    for j, L in enumerate(dl):
        Dpad[j, :L] = Dp[cu_d[j]:cu_d[j + 1]]
    qm = np.arange(5)[None] < np.array(ql)[:, None]
    dm = np.arange(6)[None] < np.array(dl)[:, None]
    np.testing.assert_allclose(v, O.maxsim(Qpad, Dpad, qm, dm), atol=1e-12)
    pq = np.array([0, 2, 2, 1, 0])
    pd = np.array([3, 0, 2, 1, 1])
    np.testing.assert_allclose(O.maxsim_pairs(Qp, Dp, cu_q, cu_d, pq, pd), v[pq, pd], atol=1e-12)
    # padded reranking == per-(b, c) loop; KD == per-query loop
    B, C = 2, 3
    Qb = rng.standard_normal((B, 4, d)); Db = rng.standard_normal((B, C, 5, d))
    qlen = np.array([4, 2]); dlen = np.array([[5, 1, 3], [2, 5, 0]])
    want = np.array([[O.maxsim(Qb[b, :qlen[b]], Db[b, c, :dlen[b, c]]) if dlen[b, c] else 0.0 for c in range(C)]
                     for b in range(B)])
    np.testing.assert_allclose(O.maxsim_padded(Qb, Db, qlen, dlen), want, atol=1e-12)
    dm_kd = np.arange(5)[None, None] < dlen[:, :, None]
    qm_kd = np.arange(4)[None] < qlen[:, None]
    np.testing.assert_allclose(O.maxsim_kd(Qb, Db, qm_kd, dm_kd), want, atol=1e-12)


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_oracle_residual_pack_roundtrip(nbits):
    rng = np.random.default_rng(nbits)
    codes = rng.integers(0, 1 << nbits, size=(3, 7, 64))
    packed = O.pack_residuals(codes, nbits)
    assert packed.shape == (3, 7, 64 * nbits // 8)
    np.testing.assert_array_equal(O.unpack_residuals(packed, nbits, 64), codes)


@pytest.mark.parametrize("case", GOLD["residual_decode"], ids=lambda c: f"{c['nbits']}b-{len(c['bytes'])}")
def test_oracle_residual_known_bytes(case):
    got = O.unpack_residuals(np.array(case["bytes"], np.uint8), case["nbits"], case["d"])
    np.testing.assert_array_equal(got, case["codes"])


def test_oracle_residual_identity_buckets_is_dense_maxsim():
    # reference tests/test_reference_cpu.py:81-104
    rng = np.random.default_rng(4)
    cent = rng.standard_normal((16, 64))
    codes = rng.integers(0, 16, (3, 10))
    res = np.zeros((3, 10, 64), np.uint8)
    Q = rng.standard_normal((2, 6, 64))
    got = O.maxsim_residual(Q, codes, res, np.full(3, 10), cent, np.zeros(256), 8, normalize=False)
    np.testing.assert_allclose(got, O.maxsim(Q, cent[codes]), atol=1e-10)


def test_oracle_residual_decode_formula_on_hand_values():
    cent = np.array([[1.0, 2.0, 3.0, 4.0], [10.0, 20.0, 30.0, 40.0]])
    bw = np.array([-0.5, 0.0, 0.25, 1.0])
    # token codes 1; bucket fields [3, 0, 2, 1] -> byte 0b01_10_00_11 = 0x63
    emb = O.decode_residual_tokens(np.array([1]), np.array([[0x63]], np.uint8), cent, bw, 2)
    np.testing.assert_array_equal(emb, [[11.0, 19.5, 30.25, 40.0]])


def test_oracle_residual_varlen_matches_padded():
    rng = np.random.default_rng(5)
    cent = rng.standard_normal((32, 16))
    bw = np.linspace(-0.1, 0.1, 4)
    lens = np.array([5, 0, 8, 3])
    L = 8
    codes = rng.integers(0, 32, (4, L))
    res = O.pack_residuals(rng.integers(0, 4, (4, L, 16)), 2)
    Q = rng.standard_normal((3, 4, 16))
    padded = O.maxsim_residual(Q, codes, res, lens, cent, bw, 2)
    keep = np.arange(L)[None] < lens[:, None]
    cu = np.concatenate([[0], np.cumsum(lens)])
    var = O.maxsim_residual_varlen(Q, codes[keep], res[keep], cu, cent, bw, 2)
    np.testing.assert_allclose(var, padded, atol=1e-12)


def test_oracle_e4m3_round_matches_torch_cast():
    import torch

    grid = np.concatenate([
        O._E4M3_POS, -O._E4M3_POS,
        (O._E4M3_POS[1:] + O._E4M3_POS[:-1]) / 2,  # exact midpoints: ties-to-even
        np.random.default_rng(0).uniform(-448, 448, 20000),
        np.random.default_rng(1).uniform(-0.02, 0.02, 20000),
    ]).astype(np.float32)
    want = torch.from_numpy(grid).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    np.testing.assert_array_equal(O.e4m3_round(grid), want)


def test_oracle_quantize_fp8_matches_torch_formula():
    import torch

    X = np.random.default_rng(2).standard_normal((4, 9, 16)).astype(np.float32)
    q, s = O.quantize_fp8_per_tensor(X)
    Xt = torch.from_numpy(X)
    st = Xt.abs().amax().clamp_min(1e-6) / 448.0
    qt = (Xt / st).clamp(-448, 448).to(torch.float8_e4m3fn).double().numpy()
    assert np.float32(s) == np.float32(st.item())
    np.testing.assert_array_equal(q, qt)
    q2, s2 = O.quantize_fp8_per_token(X)
    st2 = Xt.abs().amax(-1).clamp_min(1e-6) / 448.0
    qt2 = (Xt / st2[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(s2, st2.numpy())
    np.testing.assert_array_equal(q2, qt2)


def test_oracle_topk_known_answer():
    t = GOLD["topk"]
    s = np.array([t["scores"]])
    _, i = O.topk_stable(s, t["k"])
    assert i[0].tolist() == t["largest_idx"]
    _, i = O.topk_stable(s, t["k"], largest=False)
    assert i[0].tolist() == t["smallest_idx"]


@pytest.mark.parametrize("largest", [True, False])
def test_oracle_topk_matches_sorted_and_chunking(largest):
    rng = np.random.default_rng(6)
    s = rng.integers(0, 6, (5, 97)).astype(np.float32)  # many ties
    k = 13
    for r in range(5):
        want = sorted(range(97), key=lambda c: ((-s[r, c]) if largest else s[r, c], c))[:k]
        _, i = O.topk_stable(s[r:r + 1], k, largest=largest)
        assert i[0].tolist() == want
    full = O.retrieve_chunked(s, k, None, largest=largest)
    for chunk in (1, 4, 10, 13, 50, 96):
        got = O.retrieve_chunked(s, k, chunk, largest=largest)
        np.testing.assert_array_equal(got[1], full[1])
        np.testing.assert_array_equal(got[0], full[0])


def _torch_max(vals):
    """torch.max over a row: NaN if any element is NaN (torch propagates it), else the max."""
    best = -np.inf
    for v in vals:
        if v != v:
            return float("nan")
        best = max(best, v)
    return best


def brute_nonfinite(Q, D, qm=None, dm=None):
    """reference.py:75-94 step by step with IEEE scalar arithmetic: masked doc
    tokens are -inf, the row max propagates NaN, a non-finite max scores 0,
    masked query tokens are multiplied by 0 after that."""
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    out = np.zeros((Nq, Nd))
    with np.errstate(invalid="ignore", over="ignore"):
        for i in range(Nq):
            for j in range(Nd):
                tot = 0.0
                for s in range(Lq):
                    row = []
                    for t in range(Ld):
                        acc = 0.0
                        for a, b in zip(Q[i, s], D[j, t]):
                            acc += float(a) * float(b)
                        row.append(acc if dm is None or dm[j, t] else -np.inf)
                    best = _torch_max(row)
                    best = best if np.isfinite(best) else 0.0
                    tot += best * (1.0 if qm is None or qm[i, s] else 0.0)
                out[i, j] = tot
    return out


@pytest.mark.parametrize("normalize", [False, True])
def test_oracle_nonfinite_inputs(normalize):
    """NaN / +inf / -inf tokens in Q and D (masked and kept): the oracle follows
    torch's semantics (reference.py:83-85), pinned by a scalar loop."""
    rng = np.random.default_rng(11)
    Q = rng.standard_normal((3, 5, 8))
    D = rng.standard_normal((5, 7, 8))
    Q[0, 1, 3] = np.nan
    Q[1, 2, 0] = np.inf
    Q[2, 4, 5] = -np.inf
    Q[2, 0, 1] = np.nan  # masked below: contributes 0
    D[0, 2, 4] = np.nan
    D[1, 0, 0] = np.inf
    D[2, 6, 7] = -np.inf
    D[3, 3, 2] = np.nan  # masked below: ignored
    D[4, 1, 1] = -np.inf
    D[4, 5, 6] = np.inf  # masked below
    qm = np.ones((3, 5), bool)
    qm[2, 0] = False
    dm = np.ones((5, 7), bool)
    dm[3, 3] = False
    dm[4, 5] = False
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        got = O.maxsim(Q, D, qm, dm, normalize=normalize)
        Qb = Q / np.linalg.norm(Q, axis=-1, keepdims=True) if normalize else Q
        Db = D / np.linalg.norm(D, axis=-1, keepdims=True) if normalize else D
    want = brute_nonfinite(Qb, Db, qm, dm)
    assert np.all(np.isfinite(got))
    np.testing.assert_allclose(got, want, atol=1e-12)
    # the NaN doc token poisons every query token's max over doc 0


def test_oracle_packed_entry_points_nonfinite():
    """varlen / pairs / padded / KD on poisoned tokens score like the scalar loop
    (and like each other): one isfinite rule for every entry point."""
    rng = np.random.default_rng(12)
    Q = rng.standard_normal((3, 4, 8))
    D = rng.standard_normal((4, 6, 8))
    Q[0, 1, 3] = np.nan
    Q[1, 2, 0] = np.inf
    D[0, 2, 4] = np.nan
    D[2, 5, 1] = -np.inf
    D[3, 0, 0] = np.inf
    lens = np.array([6, 3, 6, 5])
    dm = np.arange(6)[None] < lens[:, None]
    with np.errstate(invalid="ignore", over="ignore"):
        want = brute_nonfinite(Q, D, None, dm)
        Dp = np.concatenate([D[j, : lens[j]] for j in range(4)])
        cu_d = np.concatenate([[0], np.cumsum(lens)])
        cu_q = np.arange(4) * 4
        got_v = O.maxsim_varlen(Q.reshape(-1, 8), Dp, cu_q, cu_d)
        pq, pd = np.repeat(np.arange(3), 4), np.tile(np.arange(4), 3)
        got_p = O.maxsim_pairs(Q.reshape(-1, 8), Dp, cu_q, cu_d, pq, pd)
        got_pad = O.maxsim_padded(Q, np.broadcast_to(D[None], (3, 4, 6, 8)), np.full(3, 4), np.tile(lens, (3, 1)))
        got_kd = O.maxsim_kd(Q, np.broadcast_to(D[None], (3, 4, 6, 8)), None, np.broadcast_to(dm[None], (3, 4, 6)))
    for got in (got_v, got_p.reshape(3, 4), got_pad, got_kd):
        assert np.all(np.isfinite(got))
        np.testing.assert_allclose(got, want, atol=1e-12)


def test_oracle_plaid_approx_nonfinite():
    """A NaN or +inf score in a gathered qcs row makes that query token's max
    non-finite: it scores 0 (reference.py:118-120); -inf loses the max."""
    qcs = np.arange(24, dtype=float).reshape(6, 4) / 10.0
    qcs[2, 1] = np.nan
    qcs[3, 2] = np.inf
    qcs[4, 3] = -np.inf
    codes = np.array([[0, 2, 1], [3, 0, 0], [4, 1, 0], [2, 2, 2]])
    lens = np.array([3, 2, 1, 0])
    got = O.plaid_approx_score(qcs, codes, lens)
    want = []
    for b in range(4):
        tot = 0.0
        for s in range(4):
            m = _torch_max([qcs[c, s] for c in codes[b, : lens[b]]])
            tot += m if np.isfinite(m) else 0.0
        want.append(tot)
    np.testing.assert_allclose(got, want, atol=1e-12)


def test_oracle_plaid_approx():
    rng = np.random.default_rng(8)
    qcs = rng.standard_normal((20, 6))
    codes = rng.integers(-2, 22, (4, 7))  # includes out-of-range codes
    lens = np.array([0, 3, 7, 1])
    got = O.plaid_approx_score(qcs, codes, lens)
    assert got[0] == 0.0
    for b in range(1, 4):
        cc = [c if 0 <= c < 20 else 0 for c in codes[b, : lens[b]]]
        want = sum(max(qcs[c, s] for c in cc) for s in range(6))
        assert abs(got[b] - want) < 1e-12
    # padding beyond the length does not matter
    codes2 = codes.copy(); codes2[1, 3:] = 0
    np.testing.assert_allclose(O.plaid_approx_score(qcs, codes2, lens)[1], got[1])


# --------------------------------------------------------------------------- #
# gradients (training backward)                                               #
# --------------------------------------------------------------------------- #


def _brute_argmax(Q, D, dm):
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    out = []
    for i in range(Nq):
        for j in range(Nd):
            row = []
            for s in range(Lq):
                best, bi = None, -1
                for t in range(Ld):
                    if not dm[j, t]:
                        continue
                    v = float(np.dot(Q[i, s], D[j, t]))
                    if best is None or v > best:
                        best, bi = v, t
                row.append(bi)
            out.append(row)
    return np.array(out)


def test_oracle_argmax_matches_scan_and_ties():
    rng = np.random.default_rng(4)
    Q = rng.standard_normal((2, 3, 5))
    D = rng.standard_normal((3, 6, 5))
    D[1, 4] = D[1, 2]  # exact tie: the lower index wins
    dm = np.ones((3, 6), bool)
    dm[2] = False  # all-masked doc -> -1
    dm[0, 1] = False
    got = O.maxsim_argmax(Q, D, dm)
    assert np.array_equal(got, _brute_argmax(Q, D, dm))
    assert (got.reshape(2, 3, 3)[:, 2] == -1).all()
    assert not (got.reshape(2, 3, 3)[:, 1] == 4).any()


@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("kd", [False, True])
def test_oracle_grads_match_finite_differences(normalize, kd):
    rng = np.random.default_rng(11 + normalize + 2 * kd)
    Nq, Lq, d, Ld = 2, 3, 4, 5
    Nd = Nq * 2 if kd else 3
    Q = rng.standard_normal((Nq, Lq, d))
    D = rng.standard_normal((Nd, Ld, d))
    qm = np.ones((Nq, Lq), bool)
    qm[1, 2] = False
    dm = np.ones((Nd, Ld), bool)
    dm[0, 3] = False
    docs = Nd // Nq if kd else Nd
    G = rng.standard_normal((Nq, docs))

    def loss(Qx, Dx):
        if kd:
            sc = O.maxsim_kd(Qx, Dx.reshape(Nq, docs, Ld, d), qm, dm.reshape(Nq, docs, Ld), normalize=normalize)
        else:
            sc = O.maxsim(Qx, Dx, qm, dm, normalize=normalize)
        return float((G * sc).sum())

    am = O.maxsim_argmax(Q, D, dm, normalize=normalize, kd=kd)
    gQ, gD = O.maxsim_grads(G, Q, D, am, qm, normalize=normalize, kd=kd)
    eps = 1e-6
    for X, gX, which in ((Q, gQ, 0), (D, gD, 1)):
        num = np.zeros_like(X)
        it = np.nditer(X, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            Xp, Xm = X.copy(), X.copy()
            Xp[idx] += eps
            Xm[idx] -= eps
            fp = loss(Xp, D) if which == 0 else loss(Q, Xp)
            fm = loss(Xm, D) if which == 0 else loss(Q, Xm)
            num[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(gX, num, rtol=1e-5, atol=1e-6)
    assert np.all(gQ[1, 2] == 0)  # masked query token
    assert np.all(gD[0, 3] == 0)  # masked doc token


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_oracle_colbert_encoding_is_bit_reversed_little_endian(nbits):
    rng = np.random.default_rng(nbits)
    codes = rng.integers(0, 2**nbits, (7, 128))
    colbert = O.pack_residuals_colbert(codes, nbits)
    assert colbert.shape == (7, 128 * nbits // 8)
    np.testing.assert_array_equal(O.reverse_bits_bytes(colbert), O.pack_residuals(codes, nbits))
    np.testing.assert_array_equal(O.unpack_residuals(O.reverse_bits_bytes(colbert), nbits, 128), codes)


def test_oracle_colbert_encoding_hand_bytes():
    # nbits=2, codes [1, 2, 3, 0]: bits LSB-first 10 01 11 00 -> packbits 0b10011100
    assert O.pack_residuals_colbert(np.array([[1, 2, 3, 0]]), 2)[0, 0] == 0b10011100
    assert O.reverse_bits_bytes(np.array([0b10011100]))[0] == 0b00111001
    assert O.reverse_bits_bytes(np.array([0x01, 0x80, 0xF0]).astype(np.uint8)).tolist() == [0x80, 0x01, 0x0F]
