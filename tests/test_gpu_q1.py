"""One-column-block launches (the KD layout, one short query, packed docs for
one query) run the streaming kernel of lik_q1.hip: doc tiles loaded by
coalesced, non-temporal buffer_load ... lds into a per-wavefront LDS ring,
no workgroup barriers.

* The same bits as the tile kernel (forced with cfg=(4, 1): a forced
  multi-wave block is the tile kernel's): same MFMA sequence per tile, exact
  maxima, the tile kernel's column-sum order (also for two queries sharing
  a block, Lq = 16).
* Against the float64 oracle (lik_oracle.maxsim / maxsim_kd / maxsim_varlen,
  reference.py:26-98) on the same 16-bit values within 1e-4.
* The training forward (argmax) and doc normalisation at d = 128 run here
  too: KD-layout winner indices equal, bitwise, those of the same queries
  scored against all docs on the tile kernel (two queries, docs
  pre-normalised there by its pre-pass), and so do the scores of the
  query whose column sums start at the same chunk (the other: within fp32
  reordering), with query masks, prefix masks at the tile edges and a NaN
  doc token (score 0, winner -1).
* Doc lengths around the tile edges (0, 1, 31, 32, 33, 63, 64, 65, Ld),
  masks with holes (their docs go to the masked tile kernel in the same
  call), query-only normalisation, d = 128 and 64 (full 256- and 128-byte
  rows), d = 96, 48 and 40 (dims past d; rows shorter than the padded
  width) and d = 100 (a row stride that is not a multiple of 16 bytes).
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err
from late_interaction_kernels._lib import launch_options

pytestmark = pytest.mark.gpu

EDGE = [0, 1, 31, 32, 33, 63, 64, 65]


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().float().cpu().numpy()


def _normed(shape, g, dtype):
    return torch.nn.functional.normalize(torch.randn(*shape, generator=g), dim=-1).to(dtype)


def _tile(fn):
    # a forced four-wave block: the tile kernel (unit t of a group keeps its
    # place, so its column sums run in the same order)
    with launch_options(cfg=(4, 1)):
        return fn()


def _lens(shape, ld, g):
    lens = torch.randint(0, ld + 1, shape, generator=g)
    flat = lens.view(-1)
    flat[: len(EDGE)] = torch.tensor(EDGE)
    flat[len(EDGE)] = ld
    return lens


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("normalize", [False, 1])
def test_kd_prefix_masks(dtype, normalize):
    from late_interaction_kernels import maxsim

    _case(f"q1 kd {dtype} normalize={normalize}")
    g = torch.Generator().manual_seed(3)
    Nq, K, Ld, d = 6, 40, 130, 128
    Q = torch.randn(Nq, 32, d, generator=g).to(dtype)
    D = _normed((Nq, K, Ld, d), g, dtype)
    dm = torch.arange(Ld)[None, None] < _lens((Nq, K), Ld, g)[..., None]
    Qc, Dc, dmc = Q.cuda(), D.cuda(), dm.cuda()
    got = maxsim(Qc, Dc, None, dmc, normalize=normalize)
    assert torch.equal(got, _tile(lambda: maxsim(Qc, Dc, None, dmc, normalize=normalize)))
    Qn = _np(Q)
    if normalize:
        Qn = Qn / np.maximum(np.linalg.norm(Qn.astype(np.float64), axis=-1, keepdims=True), 1e-12)
    ref = O.maxsim_kd(Qn, _np(D), None, dm.numpy())
    assert rel_err(_np(got), ref) < 1e-4
    assert got[dmc.sum(-1) == 0].abs().max().item() == 0.0


def test_kd_mask_holes_and_query_mask():
    from late_interaction_kernels import maxsim

    _case("q1 kd holes")
    g = torch.Generator().manual_seed(5)
    Nq, K, Ld, d = 4, 30, 100, 128
    Q = _normed((Nq, 32, d), g, torch.bfloat16)
    D = _normed((Nq, K, Ld, d), g, torch.bfloat16)
    dm = torch.arange(Ld)[None, None] < _lens((Nq, K), Ld, g)[..., None]
    dm[:, ::3] &= torch.rand(Nq, (K + 2) // 3, Ld, generator=g) > 0.3  # holes in every third doc
    qm = torch.arange(32)[None] < torch.tensor([32, 20, 1, 7])[:, None]
    args = (Q.cuda(), D.cuda(), qm.cuda(), dm.cuda())
    got = maxsim(*args)
    assert torch.equal(got, _tile(lambda: maxsim(*args)))
    ref = O.maxsim_kd(_np(Q), _np(D), qm.numpy(), dm.numpy())
    assert rel_err(_np(got), ref) < 1e-4


@pytest.mark.parametrize("nq,lq,d", [(1, 32, 128), (2, 16, 128), (1, 5, 128), (1, 32, 64), (2, 16, 64), (1, 32, 512)])
def test_short_queries_cross_product(nq, lq, d):
    from late_interaction_kernels import maxsim

    _case(f"q1 cross nq={nq} lq={lq} d={d}")
    g = torch.Generator().manual_seed(7 + lq + d)
    Nd, Ld = 300, 90
    Q = _normed((nq, lq, d), g, torch.bfloat16)
    D = _normed((Nd, Ld, d), g, torch.bfloat16)
    dm = torch.arange(Ld)[None] < _lens((Nd,), Ld, g)[:, None]
    args = (Q.cuda(), D.cuda(), None, dm.cuda())
    got = maxsim(*args)
    assert torch.equal(got, _tile(lambda: maxsim(*args)))
    ref = O.maxsim(_np(Q), _np(D), None, dm.numpy())
    assert rel_err(_np(got), ref) < 1e-4


def test_varlen_one_query():
    from late_interaction_kernels import maxsim_varlen

    _case("q1 varlen")
    g = torch.Generator().manual_seed(11)
    d = 128
    ld = _lens((200,), 150, g)
    cu_d = torch.zeros(len(ld) + 1, dtype=torch.int32)
    cu_d[1:] = ld.cumsum(0)
    cu_q = torch.tensor([0, 32], dtype=torch.int32)
    Qp = _normed((32, d), g, torch.bfloat16)
    Dp = _normed((int(cu_d[-1]), d), g, torch.bfloat16)
    args = (Qp.cuda(), Dp.cuda(), cu_q.cuda(), cu_d.cuda())
    got = maxsim_varlen(*args)
    assert torch.equal(got, _tile(lambda: maxsim_varlen(*args)))
    ref = O.maxsim_varlen(_np(Qp), _np(Dp), cu_q.numpy(), cu_d.numpy())
    assert rel_err(_np(got), ref) < 1e-4
    assert got[:, ld.cuda() == 0].abs().max().item() == 0.0


@pytest.mark.parametrize("d", [96, 100, 64, 48, 40])
def test_narrow_rows(d):
    from late_interaction_kernels import maxsim

    _case(f"q1 kd d={d}")
    g = torch.Generator().manual_seed(d)
    Nq, K, Ld = 3, 20, 70
    Q = _normed((Nq, 32, d), g, torch.bfloat16)
    D = _normed((Nq, K, Ld, d), g, torch.bfloat16)
    dm = torch.arange(Ld)[None, None] < _lens((Nq, K), Ld, g)[..., None]
    args = (Q.cuda(), D.cuda(), None, dm.cuda())
    got = maxsim(*args)
    assert torch.equal(got, _tile(lambda: maxsim(*args)))
    ref = O.maxsim_kd(_np(Q), _np(D), None, dm.numpy())
    assert rel_err(_np(got), ref) < 1e-4


@pytest.mark.parametrize("d", [256, 512, 300, 200])
def test_wide_rows(d):
    """Rows of 512 and 1024 bytes move through the ring as 256-byte units.
    One query (the streaming kernel) gives the bits of the same query scored
    next to a second one (64 columns: the tile kernel); KD against the
    oracle."""
    from late_interaction_kernels import maxsim

    _case(f"q1 wide d={d}")
    g = torch.Generator().manual_seed(d + 1)
    Nd, Ld = 150, 80
    Q = _normed((2, 32, d), g, torch.bfloat16)
    D = _normed((Nd, Ld, d), g, torch.bfloat16)
    dm = torch.arange(Ld)[None] < _lens((Nd,), Ld, g)[:, None]
    Qc, Dc, dmc = Q.cuda(), D.cuda(), dm.cuda()
    one = maxsim(Qc[:1], Dc, None, dmc)
    two = maxsim(Qc, Dc, None, dmc)
    assert torch.equal(one[0], two[0])
    ref = O.maxsim(_np(Q), _np(D), None, dm.numpy())
    assert rel_err(_np(two), ref) < 1e-4
    Dk = _normed((2, 30, Ld, d), g, torch.bfloat16)
    dmk = torch.arange(Ld)[None, None] < _lens((2, 30), Ld, g)[..., None]
    got = maxsim(Qc, Dk.cuda(), None, dmk.cuda())
    ref = O.maxsim_kd(_np(Q), _np(Dk), None, dmk.numpy())
    assert rel_err(_np(got), ref) < 1e-4


def test_one_query_c3_scale():
    """One query over C3's corpus (65,536 packed docs, log-uniform lengths in
    [16, 2048]): the same bits as the tile kernel; sampled docs against the
    oracle."""
    import math

    from late_interaction_kernels import maxsim_varlen

    _case("q1 one query x 65536 varlen docs")
    g = torch.Generator(device="cuda").manual_seed(13)
    Nd, d = 65536, 128
    u = torch.rand(Nd, generator=g, device="cuda")
    lens = torch.floor(torch.exp(math.log(16) + u * (math.log(2049) - math.log(16)))).clamp(16, 2048).long()
    cu_d = torch.zeros(Nd + 1, dtype=torch.int32, device="cuda")
    cu_d[1:] = lens.cumsum(0).to(torch.int32)
    tot = int(cu_d[-1].item())
    Dp = torch.empty(tot, d, device="cuda", dtype=torch.bfloat16)
    for s in range(0, tot, 1 << 22):
        e = min(tot, s + (1 << 22))
        Dp[s:e] = torch.nn.functional.normalize(torch.randn(e - s, d, generator=g, device="cuda"), dim=-1)
    Qp = torch.nn.functional.normalize(torch.randn(32, d, generator=g, device="cuda"), dim=-1).to(torch.bfloat16)
    cu_q = torch.tensor([0, 32], dtype=torch.int32, device="cuda")
    got = maxsim_varlen(Qp, Dp, cu_q, cu_d, max_seqlen_q=32, max_seqlen_d=2048)
    assert torch.equal(got, _tile(lambda: maxsim_varlen(Qp, Dp, cu_q, cu_d, max_seqlen_q=32, max_seqlen_d=2048)))
    dj = [0, 1, 777, 30000, int(lens.argmax()), Nd - 1]
    cu_h = cu_d.cpu()
    for j in dj:
        a, b = int(cu_h[j]), int(cu_h[j + 1])
        ref = O.maxsim(_np(Qp)[None], _np(Dp[a:b])[None])
        assert rel_err(_np(got[:, j:j + 1]), ref) < 1e-4, j
    del Dp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype,norm,d", [(torch.bfloat16, 0, 128), (torch.bfloat16, 1, 128), (torch.bfloat16, 2, 128),
                                          (torch.bfloat16, 3, 128), (torch.float16, 0, 128), (torch.float16, 3, 128),
                                          (torch.bfloat16, 3, 96), (torch.float16, 2, 96)])
def test_kd_training_forward_matches_tile_kernel(dtype, norm, d):
    from late_interaction_kernels._core import dense_maxsim_train

    _case(f"q1 kd training forward {dtype} norm={norm} d={d}")
    g = torch.Generator().manual_seed(11 + norm + d)
    Nq, K, Lq, Ld = 2, 40, 32, 130
    Q = torch.randn(Nq, Lq, d, generator=g).to(dtype)
    D = (torch.randn(Nq * K, Ld, d, generator=g) * 3.0).to(dtype)
    D[7, 3, 5] = float("nan")  # doc 7: every query token's max is NaN
    dm = torch.arange(Ld)[None] < _lens((Nq * K,), Ld, g)[:, None]
    dm[7, :10] = True
    qm = torch.arange(Lq)[None] < torch.tensor([32, 21])[:, None]
    args = (Q.cuda(), D.cuda(), qm.cuda(), dm.cuda())
    s_kd, am_kd = dense_maxsim_train(*args, norm=norm, kd=True)[:2]   # streaming kernel
    s_x, am_x = dense_maxsim_train(*args, norm=norm, kd=False)[:2]    # tile kernel, all docs
    am_kd = am_kd.view(Nq, K, Lq)
    am_x = am_x.view(Nq, Nq * K, Lq)
    for i in range(Nq):
        sl = slice(i * K, (i + 1) * K)
        assert torch.equal(am_kd[i], am_x[i, sl]), i
        if i == 0:
            assert torch.equal(s_kd[i], s_x[i, sl])
        else:
            # query i is unit i of the cross product's group, whose column
            # sum starts at 4-column chunk i: the same maxima in another order
            torch.testing.assert_close(s_kd[i], s_x[i, sl], rtol=1e-6, atol=0)
    assert s_kd[0, 7].item() == 0.0 and bool((am_kd[0, 7] == -1).all())

