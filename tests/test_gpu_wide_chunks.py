"""GPU parity for the shapes past one column block and the bounded workspace.

* Pair lists with queries longer than the kernel's query block (Lq = 700 at
  d = 128: query-token chunks whose partial sums are added launch by launch)
  and rows wider than the tile kernel (d = 768: the one-wave-per-pair
  kernel), forward and backward, against torch autograd on an fp32
  restatement (reference score_pairs.py:78-101 loops over query blocks the
  same way: any Lq).
* Training through rows wider than 512 (d = 768, fp32 and bf16): the wide
  kernel's argmax against the oracle's where the winner is separated, and
  gradients end to end against torch autograd.
* Normalised cross-product scoring whose pre-normalised doc copy exceeds the
  512 MiB workspace cap: scored in slices, bitwise equal to scoring each
  slice's docs in calls of their own, scores and argmax.
* forward.maxsim_forward: the raw forward entry point (reference
  forward.py:349-398), scores equal to maxsim's, argmax to the oracle's.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().double().cpu().numpy()


def _pairs_ref(Qr, Dr, cu_q, cu_d, pq, pd, nq, nd):
    out = []
    for a, b in zip(pq.tolist(), pd.tolist()):
        if a >= nq or b >= nd or cu_q[a + 1] == cu_q[a] or cu_d[b + 1] == cu_d[b]:
            out.append(Qr.sum() * 0)
            continue
        qi = Qr[cu_q[a] : cu_q[a + 1]]
        dj = Dr[cu_d[b] : cu_d[b + 1]]
        out.append((qi @ dj.T).max(-1).values.sum())
    return torch.stack(out)


@pytest.mark.parametrize("d,lq", [(128, [700, 12, 0, 530]), (768, [40, 3, 0, 65]), (64, [1100, 9, 600, 0])])
def test_pairs_long_queries_and_wide_rows(d, lq):
    from late_interaction_kernels.score_pairs import score_pairs_packed

    _case(f"pairs d={d} lq={lq}")
    g = torch.Generator().manual_seed(d + sum(lq))
    lqs = torch.tensor(lq)
    ld = torch.tensor([40, 2, 0, 77, 33, 130])
    cu_q = torch.cat([torch.zeros(1, dtype=torch.long), lqs.cumsum(0)]).to(torch.int32)
    cu_d = torch.cat([torch.zeros(1, dtype=torch.long), ld.cumsum(0)]).to(torch.int32)
    pq = torch.tensor([0, 0, 1, 2, 3, 3, 0, 1, 3, 7])
    pd = torch.tensor([0, 3, 3, 1, 5, 2, 5, 4, 0, 1])
    Q = torch.randn(int(lqs.sum()), d, generator=g) / d**0.5
    D = torch.randn(int(ld.sum()), d, generator=g)
    G = torch.randn(len(pq), generator=g).cuda()
    Qc = Q.cuda().requires_grad_()
    Dc = D.cuda().requires_grad_()
    s = score_pairs_packed(Qc, Dc, cu_q.cuda(), cu_d.cuda(), pq.cuda(), pd.cuda())
    (s * G).sum().backward()
    Qr = Q.cuda().requires_grad_()
    Dr = D.cuda().requires_grad_()
    sr = _pairs_ref(Qr, Dr, cu_q, cu_d, pq, pd, len(lq), len(ld))
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 1e-4
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < 1e-3
    # inference path (no argmax) gives the same scores
    with torch.no_grad():
        s2 = score_pairs_packed(Q.cuda(), D.cuda(), cu_q.cuda(), cu_d.cuda(), pq.cuda(), pd.cuda())
    assert torch.equal(s2, s.detach())
    # bf16 against the oracle
    Qb, Db = Q.to(torch.bfloat16), D.to(torch.bfloat16)
    sb = score_pairs_packed(Qb.cuda(), Db.cuda(), cu_q.cuda(), cu_d.cuda(), pq.cuda(), pd.cuda())
    keep = (pq < len(lq)) & (pd < len(ld))
    ref = np.zeros(len(pq))
    ref[keep.numpy()] = O.maxsim_pairs(_np(Qb), _np(Db), cu_q.numpy(), cu_d.numpy(), pq[keep].numpy(),
                                       pd[keep].numpy())
    assert rel_err(_np(sb), ref) < 1e-2


def _separated(Q, D, dm, normalize, gap):
    """[Nq * Nd, Lq] mask: the best doc token beats the runner-up by > gap."""
    Qn = _np(Q) if not normalize else _np(torch.nn.functional.normalize(Q.double(), dim=-1))
    Dn = _np(D) if not normalize else _np(torch.nn.functional.normalize(D.double(), dim=-1))
    Nq, Lq, _ = Qn.shape
    Nd = Dn.shape[0]
    ok = np.ones((Nq * Nd, Lq), bool)
    for i in range(Nq):
        for j in range(Nd):
            S = np.where(dm.numpy()[j][None], Qn[i] @ Dn[j].T, -np.inf)
            if dm[j].sum() >= 2:
                t2 = np.sort(S, axis=1)[:, -2:]
                ok[i * Nd + j] = (t2[:, 1] - t2[:, 0]) > gap
    return ok


def _torch_ref(Q, D, qm, dm, normalize):
    if normalize:
        Q = torch.nn.functional.normalize(Q, dim=-1)
        D = torch.nn.functional.normalize(D, dim=-1)
    S = torch.einsum("isd,jtd->ijst", Q, D)
    S = S.masked_fill(~dm[None, :, None, :], float("-inf"))
    m = S.max(-1).values
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    return (m * qm[:, None, :]).sum(-1)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("normalize", [False, True])
def test_wide_rows_training(dtype, tol, normalize):
    from late_interaction_kernels import maxsim
    from late_interaction_kernels._core import dense_maxsim_train

    d = 768
    _case(f"wide training d={d} {dtype} normalize={normalize}")
    g = torch.Generator().manual_seed(5 + normalize)
    Nq, Lq, Nd, Ld = 4, 20, 6, 45
    Q = torch.randn(Nq, Lq, d, generator=g).to(dtype)
    D = torch.randn(Nd, Ld, d, generator=g).to(dtype)
    qm = torch.rand(Nq, Lq, generator=g) > 0.2
    dm = torch.arange(Ld)[None] < torch.randint(1, Ld + 1, (Nd,), generator=g)[:, None]
    dm[0] = False
    dm[1, 0] = False
    _, am, *_ = dense_maxsim_train(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), norm=3 if normalize else 0, kd=False)
    ref_am = O.maxsim_argmax(_np(Q), _np(D), dm.numpy(), normalize=normalize)
    got = am.cpu().numpy()
    # compare where the best beats the runner-up clearly and the query token is kept
    gap = (1e-3 if dtype == torch.float32 else 3e-2) * (1.0 if normalize else d**0.5)
    ok = np.repeat(qm.numpy(), Nd, axis=0) & _separated(Q, D, dm, normalize, gap)
    assert np.array_equal(got[ok], ref_am[ok])
    assert np.array_equal(got == -1, ref_am == -1)

    Qc = Q.float().cuda().to(dtype).requires_grad_()
    Dc = D.float().cuda().to(dtype).requires_grad_()
    G = torch.randn(Nq, Nd, generator=g).cuda()
    s = maxsim(Qc, Dc, qm.cuda(), dm.cuda(), normalize=normalize)
    (s * G).sum().backward()
    Qr = Q.float().cuda().requires_grad_()
    Dr = D.float().cuda().requires_grad_()
    (_torch_ref(Qr, Dr, qm.cuda(), dm.cuda(), normalize) * G).sum().backward()
    sr = _torch_ref(Qr.detach(), Dr.detach(), qm.cuda(), dm.cuda(), normalize)
    assert rel_err(_np(s), _np(sr)) < tol
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < 3 * tol
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < 3 * tol


def test_prenormalised_docs_in_slices():
    """normalize=True over 9,000 padded bf16 docs of 300 x 128 (a 691 MB
    normalised copy, above the 512 MiB cap) with 3 query groups: two slices.
    Scores and the training argmax are bitwise those of separate calls on the
    two halves (each fits one slice)."""
    from late_interaction_kernels import maxsim
    from late_interaction_kernels._core import dense_maxsim_train

    _case("prenorm slices 9000 docs")
    g = torch.Generator(device="cuda").manual_seed(3)
    Q = torch.randn(40, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    D = torch.randn(9000, 300, 128, generator=g, device="cuda").to(torch.bfloat16)
    lens = torch.randint(1, 301, (9000,), generator=g, device="cuda")
    dm = torch.arange(300, device="cuda")[None] < lens[:, None]
    dm[17, 5] = False  # a doc with a hole: the masked second launch per slice
    full = maxsim(Q, D, d_mask=dm, normalize=True)
    h = 4500
    a = maxsim(Q, D[:h], d_mask=dm[:h], normalize=True)
    b = maxsim(Q, D[h:], d_mask=dm[h:], normalize=True)
    assert torch.equal(full, torch.cat([a, b], 1))
    s, am, *_ = dense_maxsim_train(Q, D, None, dm, norm=3, kd=False)
    assert rel_err(_np(s), _np(full)) < 1e-5
    _, am_a, *_ = dense_maxsim_train(Q, D[:h], None, dm[:h], norm=3, kd=False)
    _, am_b, *_ = dense_maxsim_train(Q, D[h:], None, dm[h:], norm=3, kd=False)
    am3 = am.view(40, 9000, 32)
    assert torch.equal(am3[:, :h], am_a.view(40, h, 32))
    assert torch.equal(am3[:, h:], am_b.view(40, 9000 - h, 32))
    j = torch.tensor([0, 17, 4499, 4500, 8999])
    ref = O.maxsim(_np(Q), _np(D[j.cuda()]), None, dm[j.cuda()].cpu().numpy(), normalize=True)
    assert rel_err(_np(full[:, j.cuda()]), ref) < 1e-2


@pytest.mark.parametrize("normalize", [False, True])
def test_maxsim_forward_entry_point(normalize):
    from late_interaction_kernels import maxsim
    from late_interaction_kernels.forward import maxsim_forward

    _case(f"maxsim_forward normalize={normalize}")
    g = torch.Generator().manual_seed(9)
    Q = torch.randn(3, 16, 64, generator=g)
    D = torch.randn(5, 30, 64, generator=g)
    qm = torch.rand(3, 16, generator=g) > 0.2
    dm = torch.arange(30)[None] < torch.tensor([30, 1, 17, 0, 9])[:, None]
    s, am = maxsim_forward(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), normalize=normalize)
    assert am is None
    assert torch.equal(s, maxsim(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), normalize=normalize))
    s2, am2 = maxsim_forward(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), save_argmax=True, normalize=normalize)
    assert am2.shape == (15, 16) and am2.dtype == torch.int32
    assert rel_err(_np(s2), O.maxsim(_np(Q), _np(D), qm.numpy(), dm.numpy(), normalize=normalize)) < 1e-4
    ref_am = O.maxsim_argmax(_np(Q), _np(D), dm.numpy(), normalize=normalize)
    keep = np.repeat(qm.numpy(), 5, axis=0) & _separated(Q, D, dm, normalize, 1e-3)
    assert np.array_equal(am2.cpu().numpy()[keep], ref_am[keep])
    assert np.array_equal(am2.cpu().numpy() == -1, ref_am == -1)
    # 2-D inputs squeeze like maxsim
    s3, _ = maxsim_forward(Q[0].cuda(), D[1].cuda())
    assert s3.shape == ()
    s4, _ = maxsim_forward(Q[0].cuda(), D.cuda())
    assert s4.shape == (5,)
