"""GPU parity on non-finite inputs: NaN, +inf and -inf tokens.

reference.py:75-94 takes the max over doc tokens with torch's max, which
propagates NaN, and then scores a non-finite max (NaN, +inf, or -inf for an
all-masked row) as 0; masked doc tokens are replaced by -inf before the max
(so whatever they hold is ignored), masked query tokens are multiplied by 0
after the isfinite rule. So:

* one NaN element in a kept doc token makes every query token's max over that
  doc NaN: the doc scores 0 against every query;
* a +inf similarity scores its query token 0; a -inf similarity loses the max;
* with normalize=True an inf element normalises to NaN (inf / inf);
* NaN / inf in a masked doc token or a masked query token changes nothing.

The kernels take row maxima with a NaN-propagating max (v_maximum3_f32), zero
masked doc rows before the -inf bias is added, and select -inf for rows past a
tile's end; fp32 splits keep inf products free of inf * 0. Each case is
compared with the oracle (oracle/lik_oracle.py, pinned on the same inputs by a
scalar loop in tests/test_oracle.py) on exactly the values the kernel reads,
within the dtype's tolerance, and the fully poisoned docs are checked to be
exactly 0.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err
from late_interaction_kernels._lib import launch_options

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2, torch.float16: 1e-2}
NAN, INF = float("nan"), float("inf")


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().double().cpu().numpy()


def _oracle(fn, *a, **k):
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        return fn(*a, **k)


def _poison_dense(Q, D):
    """NaN / +inf / -inf at fixed spots of Q [Nq, Lq, d] and D [Nd, Ld, d] (CPU fp32).
    Returns the doc indices that hold a kept NaN token (they score 0 for every query)."""
    Q[0, 3, 5] = NAN
    Q[1, 7, 0] = INF
    Q[2, 1, 9] = -INF
    D[1, 10, 3] = NAN
    D[2, 5, 0] = INF
    D[3, 0, 7] = -INF
    D[4, 12, 2] = -INF
    D[4, 13, 2] = INF
    return [1]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("mask", ["none", "prefix", "holes"])
@pytest.mark.parametrize("Nq,Lq,Nd,Ld,d", [(16, 32, 40, 130, 128), (3, 20, 9, 77, 64)])
def test_dense_nonfinite(dtype, normalize, mask, Nq, Lq, Nd, Ld, d):
    from late_interaction_kernels import maxsim

    _case(f"nonfinite dense {dtype} norm={normalize} mask={mask} {Nq},{Lq},{Nd},{Ld},{d}")
    g = torch.Generator().manual_seed(Nq + Ld + d)
    Q = torch.randn(Nq, Lq, d, generator=g)
    D = torch.randn(Nd, Ld, d, generator=g)
    poisoned = _poison_dense(Q, D)
    qm = dm = None
    if mask != "none":
        lens = torch.randint(20, Ld + 1, (Nd,), generator=g)
        dm = torch.arange(Ld)[None] < lens[:, None]
        dm[5, :] = False  # all masked: 0
        D[6, int(lens[6]) - 1 if int(lens[6]) < Ld else Ld - 1, 0] = NAN
        if mask == "holes":
            dm &= torch.rand(Nd, Ld, generator=g) > 0.2
            dm[1, 10] = True  # the poisoned token stays kept
            D[7, 2, 1] = NAN  # masked NaN tokens: ignored
            D[7, 3, 4] = INF
            dm[7, 2:4] = False
        else:
            D[7, int(lens[7]):, :] = NAN  # past the prefix: ignored
        qm = torch.rand(Nq, Lq, generator=g) > 0.2
        qm[0, 3] = True
        Q[2, 4, :] = NAN  # masked query token: 0
        qm[2, 4] = False
    Qd, Dd = Q.to(dtype), D.to(dtype)
    got = maxsim(Qd.cuda(), Dd.cuda(), None if qm is None else qm.cuda(), None if dm is None else dm.cuda(),
                 normalize=normalize)
    ref = _oracle(O.maxsim, _np(Qd), _np(Dd), None if qm is None else qm.numpy(),
                  None if dm is None else dm.numpy(), normalize=normalize)
    gn = _np(got)
    assert np.all(np.isfinite(gn))
    for j in poisoned:
        assert np.all(gn[:, j] == 0.0)
    assert rel_err(gn, ref) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("normalize", [False, True])
def test_training_forward_nonfinite(dtype, normalize):
    """The argmax-saving forward (Q requires grad) gives the same scores."""
    from late_interaction_kernels import maxsim

    _case(f"nonfinite train fwd {dtype} norm={normalize}")
    g = torch.Generator().manual_seed(5)
    Q = torch.randn(6, 32, 128, generator=g)
    D = torch.randn(9, 70, 128, generator=g)
    poisoned = _poison_dense(Q, D)
    Qd, Dd = Q.to(dtype), D.to(dtype)
    got = maxsim(Qd.cuda().requires_grad_(), Dd.cuda(), normalize=normalize)
    ref = _oracle(O.maxsim, _np(Qd), _np(Dd), normalize=normalize)
    gn = _np(got)
    assert np.all(np.isfinite(gn)) and np.all(gn[:, poisoned] == 0.0)
    assert rel_err(gn, ref) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("normalize", [False, True])
def test_kd_varlen_pairs_nonfinite(dtype, normalize):
    from late_interaction_kernels import maxsim, maxsim_pairs, maxsim_varlen

    _case(f"nonfinite kd/varlen/pairs {dtype} norm={normalize}")
    g = torch.Generator().manual_seed(9)
    Nq, Lq, K, Ld, d = 5, 32, 6, 75, 128
    Q = torch.randn(Nq, Lq, d, generator=g)
    D = torch.randn(Nq, K, Ld, d, generator=g)
    Q[0, 3, 5] = NAN
    Q[1, 7, 0] = INF
    D[0, 1, 10, 3] = NAN
    D[2, 2, 5, 0] = INF
    D[3, 0, 7, 9] = -INF
    Qd, Dd = Q.to(dtype), D.to(dtype)
    # KD layout (the streaming one-block kernel for Lq <= 32)
    got = _np(maxsim(Qd.cuda(), Dd.cuda(), normalize=normalize))
    ref = _oracle(O.maxsim_kd, _np(Qd), _np(Dd), normalize=normalize)
    assert np.all(np.isfinite(got)) and got[0, 1] == 0.0
    assert rel_err(got, ref) < TOL[dtype]
    # pairs (query i, its doc 1): maxsim_pairs
    got_p = _np(maxsim_pairs(Qd.cuda(), Dd[:, 1].contiguous().cuda(), normalize=normalize))
    assert np.all(np.isfinite(got_p)) and got_p[0] == 0.0
    assert rel_err(got_p, ref[:, 1]) < TOL[dtype]
    # varlen: packed docs of ragged lengths (normalise folded into the inputs)
    Qn = Qd.float()
    Dn = Dd.float().reshape(Nq * K, Ld, d)
    if normalize:
        Qn = torch.nn.functional.normalize(Qn, dim=-1)
        Dn = torch.nn.functional.normalize(Dn, dim=-1)
    Qn, Dn = Qn.to(dtype), Dn.to(dtype)
    lens = torch.randint(1, Ld + 1, (Nq * K,), generator=g)
    lens[1] = 11  # keeps the NaN token (row 10) of doc 1
    Dp = torch.cat([Dn[j, : int(lens[j])] for j in range(Nq * K)])
    cu_d = torch.zeros(Nq * K + 1, dtype=torch.int32)
    cu_d[1:] = lens.cumsum(0).to(torch.int32)
    cu_q = torch.arange(Nq + 1, dtype=torch.int32) * Lq
    Qp = Qn.reshape(-1, d)
    got_v = _np(maxsim_varlen(Qp.cuda(), Dp.cuda(), cu_q.cuda(), cu_d.cuda()))
    ref_v = _oracle(O.maxsim_varlen, _np(Qp), _np(Dp), cu_q.numpy(), cu_d.numpy())
    assert np.all(np.isfinite(got_v)) and np.all(got_v[:, 1] == 0.0)
    assert rel_err(got_v, ref_v) < TOL[dtype]


def test_wide_rows_nonfinite():
    """d = 600: the one-wavefront-per-pair kernel for rows wider than a column block."""
    from late_interaction_kernels import maxsim

    _case("nonfinite wide d=600")
    g = torch.Generator().manual_seed(600)
    Q = torch.randn(4, 20, 600, generator=g)
    D = torch.randn(6, 40, 600, generator=g)
    poisoned = _poison_dense(Q, D)
    dm = torch.rand(6, 40, generator=g) > 0.2
    dm[1, 10] = True
    D[5, 3, 3] = NAN
    dm[5, 3] = False
    for dtype in (torch.bfloat16, torch.float32):
        for normalize in (False, True):
            Qd, Dd = Q.to(dtype), D.to(dtype)
            got = _np(maxsim(Qd.cuda(), Dd.cuda(), d_mask=dm.cuda(), normalize=normalize))
            ref = _oracle(O.maxsim, _np(Qd), _np(Dd), None, dm.numpy(), normalize=normalize)
            assert np.all(np.isfinite(got)) and np.all(got[:, poisoned] == 0.0)
            assert rel_err(got, ref) < TOL[dtype], (dtype, normalize)


@pytest.mark.parametrize("per_token", [False, True])
def test_fp8_nonfinite(per_token):
    """e4m3fn has NaN (0x7f) but no inf: a NaN byte in a kept doc token zeroes the doc."""
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_tensor, quantize_fp8_per_token

    _case(f"nonfinite fp8 per_token={per_token}")
    g = torch.Generator().manual_seed(8)
    Q = torch.nn.functional.normalize(torch.randn(20, 24, 128, generator=g), dim=-1)
    D = torch.nn.functional.normalize(torch.randn(30, 150, 128, generator=g), dim=-1)
    quant = quantize_fp8_per_token if per_token else quantize_fp8_per_tensor
    Qf, sq = quant(Q.cuda())
    Df, sd = quant(D.cuda())
    Qf.view(torch.uint8)[0, 3, 5] = 0x7F
    Df.view(torch.uint8)[1, 10, 3] = 0xFF
    Df.view(torch.uint8)[4, 100, 0] = 0x7F
    dm = torch.ones(30, 150, dtype=torch.bool)
    dm[4, 100] = False  # masked NaN: ignored
    dm[6, 50:] = False
    got = _np(maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd, d_mask=dm.cuda()))
    sqn = sq.cpu().double().numpy()[..., None] if per_token else sq.item()
    sdn = sd.cpu().double().numpy()[..., None] if per_token else sd.item()
    ref = _oracle(O.maxsim, _np(Qf) * sqn, _np(Df) * sdn, None, dm.numpy())
    assert np.all(np.isfinite(got)) and np.all(got[:, 1] == 0.0)
    assert rel_err(got, ref) < 2e-3


def _plaid_index(Nd, max_ld, d, nbits, seed, ncent=64):
    g = torch.Generator().manual_seed(seed)
    cent = torch.nn.functional.normalize(torch.randn(ncent, d, generator=g), dim=-1)
    cent[7, 11] = NAN  # a NaN centroid
    bw = torch.linspace(-0.1, 0.1, 2**nbits)
    lens = torch.randint(1, max_ld + 1, (Nd,), generator=g)
    lens[0] = 0
    lens[3] = 40
    lens[5] = 10
    T = int(lens.sum())
    codes = torch.randint(0, ncent, (T,), generator=g, dtype=torch.int32)
    codes[codes == 7] = 8
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    codes[int(cu[3]) + 1] = 7  # doc 3 holds one token of the NaN centroid
    codes[int(cu[5])] = 7      # doc 5 too, at its first token
    bcodes = np.random.default_rng(seed).integers(0, 2**nbits, (T, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    return cent, bw, codes, res, cu


@pytest.mark.parametrize("route", ["auto", "exact_gather", "per_lane", "tile", "decode", "prepared"])
@pytest.mark.parametrize("nq", [1, 3, 40])
def test_plaid_nan_centroid(route, nq):
    from late_interaction_kernels.plaid import ResidualIndex, maxsim_residual_varlen

    _case(f"nonfinite plaid route={route} nq={nq}")
    nbits, d = 2, 128
    cent, bw, codes, res, cu = _plaid_index(300, 90, d, nbits, 17)
    cent = cent.to(torch.bfloat16)
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    g = torch.Generator().manual_seed(nq)
    Q = torch.randn(nq, 32, d, generator=g).to(torch.bfloat16).cuda()
    variant = {"exact_gather": 2, "per_lane": 1, "tile": 3}.get(route, 0)
    for normalize in (True, False):
        if route == "prepared":
            got = ResidualIndex(*args).score(Q, normalize=normalize)
        else:
            with launch_options(plaid_variant=variant, plaid_route="decode" if route == "decode" else "auto"):
                got = maxsim_residual_varlen(Q, *args, normalize=normalize)
        ref = _oracle(O.maxsim_residual_varlen, _np(Q), codes.numpy(), res.numpy(), cu.numpy(),
                      cent.double().numpy(), bw.numpy(), nbits, normalize=normalize)
        gn = _np(got)
        assert np.all(np.isfinite(gn)), (route, normalize)
        assert np.all(gn[:, 3] == 0.0) and np.all(gn[:, 5] == 0.0), (route, normalize)
        assert rel_err(gn, ref) < 1e-2, (route, normalize)


def test_plaid_approx_nonfinite():
    from late_interaction_kernels.plaid import plaid_approx_score

    _case("nonfinite plaid_approx_score")
    g = torch.Generator().manual_seed(3)
    qcs = torch.randn(64, 32, generator=g)
    qcs[5, 3] = NAN
    qcs[6, 4] = INF
    qcs[9, 0] = -INF
    codes = torch.randint(0, 64, (20, 30), generator=g, dtype=torch.int32)
    codes[2, 4] = 5
    codes[3, 0] = 6
    codes[4, 1] = 9
    lens = torch.randint(0, 31, (20,), generator=g)
    lens[2:5] = 30
    got = _np(plaid_approx_score(qcs.cuda(), codes.cuda(), lens.cuda()))
    ref = _oracle(O.plaid_approx_score, qcs.numpy(), codes.numpy(), lens.numpy())
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_head_nonfinite(dtype):
    """maxsim_from_hidden (fused projection head): a NaN hidden state projects to
    a NaN doc row and zeroes its doc; a masked NaN row is ignored."""
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    _case(f"nonfinite fused head {dtype}")
    g = torch.Generator().manual_seed(21)
    Nq, Lq, Nd, Ld, dmod, dout = 3, 32, 6, 120, 256, 128
    Q = torch.nn.functional.normalize(torch.randn(Nq, Lq, dout, generator=g), dim=-1).to(dtype)
    H = torch.randn(Nd, Ld, dmod, generator=g)
    H[1, 30, 7] = NAN
    H[4, 3, 0] = NAN
    W = (torch.randn(dout, dmod, generator=g) * dmod**-0.5).to(dtype)
    dm = torch.ones(Nd, Ld, dtype=torch.bool)
    dm[4, 3] = False
    H = H.to(dtype)
    with torch.no_grad():
        got = _np(maxsim_from_hidden(Q.cuda(), H.cuda(), W.cuda(), None, d_mask=dm.cuda()))
    D = H.float() @ W.float().t()
    D = (D / D.norm(dim=-1, keepdim=True).clamp_min(1e-12)).to(dtype).double()
    S = torch.einsum("isd,jtd->ijst", Q.double(), D).masked_fill(~dm[None, :, None, :], float("-inf"))
    m = S.max(dim=-1).values
    ref = torch.where(torch.isfinite(m), m, torch.zeros_like(m)).sum(-1).numpy()
    assert np.all(np.isfinite(got)) and np.all(got[:, 1] == 0.0)
    assert rel_err(got, ref) < 2e-3
