"""GPU parity of the training path: argmax-saving forward and the HIP backward.

* The saved argmax equals the oracle's (lowest index among maximal scores,
  -1 for an all-masked doc) wherever the oracle's best and second-best scores
  are separated by more than the compute precision. Entries of masked query
  tokens are unspecified (their score terms and gradients are zero).
* Given the kernel's own argmax, grad_Q / grad_D match the float64 oracle
  (oracle/lik_oracle.maxsim_grads, pinned against finite differences in
  tests/test_oracle.py): rel 1e-5 for fp32 inputs, 1e-2 for bf16.
* End to end, autograd through maxsim matches torch autograd on a plain
  fp32 restatement of the forward; masked tokens get zero gradient; two
  backward runs are bitwise identical (no atomics).
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


def _inputs(Nq, Nd, Lq, Ld, d, dtype, seed, masks=True):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(Nq, Lq, d, generator=g).to(dtype)
    D = torch.randn(Nd, Ld, d, generator=g).to(dtype)
    qm = dm = None
    if masks:
        qm = torch.rand(Nq, Lq, generator=g) > 0.2
        dm = torch.arange(Ld)[None] < torch.randint(1, Ld + 1, (Nd,), generator=g)[:, None]
        dm[0] = False  # fully masked doc
        dm[1, 0] = False  # a hole
    return Q, D, qm, dm


def _separated(Q, D, dm, normalize, kd, gap):
    """Mask of (i*docs+j, s) entries whose best score beats the runner-up by > gap."""
    Qn = _np(Q) if not normalize else _np(torch.nn.functional.normalize(Q.double(), dim=-1))
    Dn = _np(D) if not normalize else _np(torch.nn.functional.normalize(D.double(), dim=-1))
    Nq, Lq, _ = Qn.shape
    Nd, Ld, _ = Dn.shape
    docs = Nd // Nq if kd else Nd
    dmn = np.ones((Nd, Ld), bool) if dm is None else dm.numpy()
    ok = np.ones((Nq * docs, Lq), bool)
    for i in range(Nq):
        for jl in range(docs):
            j = i * docs + jl if kd else jl
            S = np.where(dmn[j][None], Qn[i] @ Dn[j].T, -np.inf)
            if dmn[j].sum() >= 2:
                top2 = np.sort(S, axis=1)[:, -2:]
                ok[i * docs + jl] = (top2[:, 1] - top2[:, 0]) > gap
    return ok


@pytest.mark.parametrize("dtype,tol,gap", [(torch.float32, 1e-5, 1e-4), (torch.bfloat16, 1e-2, 5e-2)])
@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("kd", [False, True])
def test_argmax_and_grads_match_oracle(dtype, tol, gap, normalize, kd):
    from late_interaction_kernels._core import dense_maxsim_train, maxsim_backward

    _case(f"bwd {dtype} norm={normalize} kd={kd}")
    Nq, Lq, d, Ld = 5, 24, 64, 50
    Nd = Nq * 3 if kd else 7
    Q, D, qm, dm = _inputs(Nq, Nd, Lq, Ld, d, dtype, 7 + normalize + 2 * kd)
    scores, am, Qp, Dp, qmi = dense_maxsim_train(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), norm=3 if normalize else 0, kd=kd)
    ref_am = O.maxsim_argmax(_np(Q), _np(D), dm.numpy(), normalize=normalize, kd=kd)
    got_am = am.cpu().numpy()
    sep = _separated(Q, D, dm, normalize, kd, gap)
    # masked query tokens score nothing; their winner entries are unspecified
    docs = Nd // Nq if kd else Nd
    sep &= np.repeat(qm.numpy(), docs, axis=0)
    assert np.array_equal(got_am[sep], ref_am[sep])
    assert np.array_equal(got_am == -1, ref_am == -1)
    G = torch.randn(Nq, docs)
    gq, gd = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=3 if normalize else 0, kd=kd)
    rq, rd = O.maxsim_grads(G.numpy(), _np(Q), _np(D), got_am, qm.numpy(), normalize=normalize, kd=kd)
    assert rel_err(_np(gq), rq) < tol
    assert rel_err(_np(gd), rd) < tol
    assert np.all(_np(gd)[0] == 0)  # fully masked doc: no winners, zero grad


@pytest.mark.parametrize("Nq,kd", [(1, False), (2, False), (3, True)])
def test_grad_q_doc_splits(Nq, kd):
    """Few query tokens and many docs: grad_q splits each token's docs into
    chunks walked by separate wavefronts and adds the chunk sums in order.
    Against the oracle (fp32 inputs, 1e-5), chunk edges not on a 64-doc
    boundary, and bitwise equal on a second run."""
    from late_interaction_kernels._core import dense_maxsim_train, maxsim_backward

    _case(f"bwd grad_q splits Nq={Nq} kd={kd}")
    Lq, d, Ld = 20, 64, 30
    Nd = Nq * 333 if kd else 701
    Q, D, qm, dm = _inputs(Nq, Nd, Lq, Ld, d, torch.float32, 40 + Nq)
    scores, am, Qp, Dp, qmi = dense_maxsim_train(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), norm=3, kd=kd)
    docs = Nd // Nq if kd else Nd
    G = torch.randn(Nq, docs)
    gq, gd = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=3, kd=kd)
    rq, rd = O.maxsim_grads(G.numpy(), _np(Q), _np(D), am.cpu().numpy(), qm.numpy(), normalize=True, kd=kd)
    assert rel_err(_np(gq), rq) < 1e-5
    assert rel_err(_np(gd), rd) < 1e-5
    gq2, _ = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=3, kd=kd)
    assert torch.equal(gq, gq2)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("normalize", [False, True])
def test_grad_d_sorted_entries(dtype, tol, normalize):
    """Cross product with many (query, token) pairs per doc (Nq * Lq >= 8192):
    grad_D from the winner entries sorted by doc row, against the oracle given
    the kernel's winners; masked query tokens, a fully masked doc, holes;
    bitwise equal on a second run."""
    from late_interaction_kernels._core import dense_maxsim_train, maxsim_backward

    _case(f"bwd sorted grad_d {dtype} norm={normalize}")
    Nq, Lq, Nd, Ld, d = 256, 32, 5, 40, 64
    Q, D, qm, dm = _inputs(Nq, Nd, Lq, Ld, d, dtype, 31 + normalize)
    norm = 3 if normalize else 0
    _, am, Qp, Dp, qmi = dense_maxsim_train(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), norm=norm, kd=False)
    G = torch.randn(Nq, Nd, generator=torch.Generator().manual_seed(5))
    G[3, 4] = 0.0  # a zero upstream gradient drops its pairs
    gq, gd = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=norm, kd=False)
    rq, rd = O.maxsim_grads(G.numpy(), _np(Q), _np(D), am.cpu().numpy(), qm.numpy(), normalize=normalize, kd=False)
    assert rel_err(_np(gq), rq) < tol
    assert rel_err(_np(gd), rd) < tol
    assert np.all(_np(gd)[0] == 0)
    gq2, gd2 = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=norm, kd=False)
    assert torch.equal(gd, gd2) and torch.equal(gq, gq2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_cross_product_grad_d_matches_row_blocks(dtype):
    """A cross product with Nq * Lq <= 64 takes the per-doc grad_D kernel; the
    same problem with one masked query token more (66 pairs) takes the
    row-block kernel: grad_D bitwise equal (same pairs, same order)."""
    from late_interaction_kernels._core import dense_maxsim_train, maxsim_backward

    _case(f"small cross grad_d vs row blocks {dtype}")
    Nq, Lq, Nd, Ld, d = 2, 32, 7, 600, 128
    Q, D, qm, dm = _inputs(Nq, Nd, Lq, Ld, d, dtype, 23)
    G = torch.randn(Nq, Nd, generator=torch.Generator().manual_seed(3))
    Q2 = torch.cat([Q, torch.randn(Nq, 1, d).to(dtype)], dim=1)
    qm2 = torch.cat([qm, torch.zeros(Nq, 1, dtype=torch.bool)], dim=1)
    outs = []
    for Qx, qmx in ((Q, qm), (Q2, qm2)):
        _, am, Qp, Dp, qmi = dense_maxsim_train(Qx.cuda(), D.cuda(), qmx.cuda(), dm.cuda(), norm=3, kd=False)
        outs.append((am.view(Nq, Nd, -1)[..., :Lq], maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=3, kd=False)[1]))
    (am1, gd1), (am2, gd2) = outs
    keep = qm.cuda()[:, None, :].expand(Nq, Nd, Lq)
    assert torch.equal(am1[keep], am2[keep])
    assert torch.equal(gd1, gd2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kd_grad_d_matches_per_query_cross_product(dtype):
    """KD-layout grad_D (one wavefront per doc: its winning rows summed in
    token order, the rest written as zeros) equals, bitwise, grad_D of each
    query scored alone against its K docs on the cross-product path (the
    row-block kernel, same token order), given the same winners; long docs
    (Ld 700) and masks."""
    from late_interaction_kernels._core import dense_maxsim_train, maxsim_backward

    _case(f"kd grad_d vs per-query cross product {dtype}")
    Nq, K, Lq, Ld, d = 3, 5, 32, 700, 128
    Q, D, qm, dm = _inputs(Nq, Nq * K, Lq, Ld, d, dtype, 17)
    G = torch.randn(Nq, K, generator=torch.Generator().manual_seed(2))
    _, am, Qp, Dp, qmi = dense_maxsim_train(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), norm=3, kd=True)
    gq, gd = maxsim_backward(G.cuda(), Qp, Dp, am, qmi, norm=3, kd=True)
    assert torch.all(gd[0] == 0)  # fully masked doc
    for i in range(Nq):
        sl = slice(i * K, (i + 1) * K)
        _, am1, Qp1, Dp1, qm1 = dense_maxsim_train(Q[i:i + 1].cuda(), D[sl].cuda(), qm[i:i + 1].cuda(),
                                                   dm[sl].cuda(), norm=3, kd=False)
        assert torch.equal(am1.view(K, Lq), am.view(Nq, K, Lq)[i])
        gq1, gd1 = maxsim_backward(G[i:i + 1].cuda(), Qp1, Dp1, am1, qm1, norm=3, kd=False)
        assert torch.equal(gd1, gd[sl])


def _torch_ref(Q, D, qm, dm, normalize):
    """Plain fp32 autograd restatement of the forward (reference.py:26-98)."""
    if normalize:
        Q = torch.nn.functional.normalize(Q, dim=-1)
        D = torch.nn.functional.normalize(D, dim=-1)
    S = torch.einsum("isd,jtd->ijst", Q, D)
    S = S.masked_fill(~dm[None, :, None, :], float("-inf"))
    m = S.max(-1).values
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    m = m * qm[:, None, :]
    return m.sum(-1)


@pytest.mark.parametrize("normalize", [False, True])
def test_autograd_end_to_end(normalize):
    from late_interaction_kernels import maxsim

    _case(f"autograd e2e norm={normalize}")
    Q, D, qm, dm = _inputs(6, 9, 32, 40, 128, torch.float32, 3)
    Qc = Q.cuda().requires_grad_()
    Dc = D.cuda().requires_grad_()
    G = torch.randn(6, 9).cuda()
    s = maxsim(Qc, Dc, qm.cuda(), dm.cuda(), normalize=normalize)
    (s * G).sum().backward()
    Qr = Q.cuda().requires_grad_()
    Dr = D.cuda().requires_grad_()
    sr = _torch_ref(Qr, Dr, qm.cuda(), dm.cuda(), normalize)
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 1e-4
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < 1e-3
    assert torch.all(Qc.grad[~qm.cuda()] == 0)
    assert torch.all(Dc.grad[~dm.cuda()] == 0)


def test_backward_is_bitwise_deterministic():
    from late_interaction_kernels import maxsim

    _case("bwd determinism")
    Q, D, qm, dm = _inputs(16, 40, 32, 64, 128, torch.bfloat16, 5, masks=False)
    grads = []
    for _ in range(2):
        Qc = Q.cuda().requires_grad_()
        Dc = D.cuda().requires_grad_()
        maxsim(Qc, Dc, normalize=True).sum().backward()
        grads.append((Qc.grad.clone(), Dc.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


def test_pairs_kd_and_long_query_grads():
    from late_interaction_kernels import maxsim, maxsim_pairs

    _case("bwd pairs / kd 4-D / Lq > 512")
    g = torch.Generator().manual_seed(2)
    # pairs == KD with K = 1
    Q = torch.randn(4, 32, 64, generator=g).cuda().requires_grad_()
    D = torch.randn(4, 20, 64, generator=g).cuda().requires_grad_()
    maxsim_pairs(Q, D, normalize=True).sum().backward()
    Qr = Q.detach().clone().requires_grad_()
    Dr = D.detach().clone().requires_grad_()
    ref = torch.stack([_torch_ref(Qr[i : i + 1], Dr[i : i + 1], torch.ones(1, 32, dtype=torch.bool, device="cuda"),
                                  torch.ones(1, 20, dtype=torch.bool, device="cuda"), True)[0, 0] for i in range(4)])
    ref.sum().backward()
    assert rel_err(_np(Q.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(D.grad), _np(Dr.grad)) < 1e-3
    # 4-D KD
    Q = torch.randn(3, 16, 64, generator=g).cuda().requires_grad_()
    D = torch.randn(3, 5, 30, 64, generator=g).cuda().requires_grad_()
    maxsim(Q, D).sum().backward()
    Qr = Q.detach().clone().requires_grad_()
    Dr = D.detach().clone().requires_grad_()
    on_q = torch.ones(1, 16, dtype=torch.bool, device="cuda")
    on_d = torch.ones(5, 30, dtype=torch.bool, device="cuda")
    torch.stack([_torch_ref(Qr[i : i + 1], Dr[i], on_q, on_d, False)[0] for i in range(3)]).sum().backward()
    assert rel_err(_np(Q.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(D.grad), _np(Dr.grad)) < 1e-3
    # long query: the forward splits Lq into column-block chunks
    Q = torch.randn(2, 700, 64, generator=g).cuda().requires_grad_()
    D = torch.randn(3, 40, 64, generator=g).cuda().requires_grad_()
    maxsim(Q, D, normalize=True).sum().backward()
    Qr = Q.detach().clone().requires_grad_()
    Dr = D.detach().clone().requires_grad_()
    _torch_ref(Qr, Dr, torch.ones(2, 700, dtype=torch.bool, device="cuda"),
               torch.ones(3, 40, dtype=torch.bool, device="cuda"), True).sum().backward()
    assert rel_err(_np(Q.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(D.grad), _np(Dr.grad)) < 1e-3


def _varlen_ref(Qp, Dp, cu_q, cu_d):
    """fp32 autograd loop: scores[i, j] = sum_s max_t <Q_i[s], D_j[t]>, empty -> 0 (reference.py:213-245)."""
    Nq, Nd = len(cu_q) - 1, len(cu_d) - 1
    rows = []
    for i in range(Nq):
        Qi = Qp[cu_q[i] : cu_q[i + 1]]
        cols = []
        for j in range(Nd):
            Dj = Dp[cu_d[j] : cu_d[j + 1]]
            if Qi.shape[0] == 0 or Dj.shape[0] == 0:
                cols.append(Qp.sum() * 0)
            else:
                cols.append((Qi @ Dj.T).max(-1).values.sum())
        rows.append(torch.stack(cols))
    return torch.stack(rows)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
def test_varlen_grads(dtype, tol):
    from late_interaction_kernels import maxsim_varlen

    _case(f"varlen grads {dtype}")
    g = torch.Generator().manual_seed(9)
    # short docs (several per 32-row block), an empty doc, docs spanning blocks, an empty query
    ld = torch.tensor([3, 1, 0, 70, 5, 2, 33, 1, 64, 4, 9, 31])
    lq = torch.tensor([7, 0, 32, 19, 40])
    cu_d = torch.cat([torch.zeros(1, dtype=torch.long), ld.cumsum(0)]).to(torch.int32)
    cu_q = torch.cat([torch.zeros(1, dtype=torch.long), lq.cumsum(0)]).to(torch.int32)
    Q = torch.randn(int(lq.sum()), 96, generator=g).to(dtype)
    D = torch.randn(int(ld.sum()), 96, generator=g).to(dtype)
    G = torch.randn(len(lq), len(ld), generator=g)
    Qc = Q.cuda().requires_grad_()
    Dc = D.cuda().requires_grad_()
    s = maxsim_varlen(Qc, Dc, cu_q.cuda(), cu_d.cuda())
    (s * G.cuda()).sum().backward()
    Qr = Q.float().cuda().requires_grad_()
    Dr = D.float().cuda().requires_grad_()
    sr = _varlen_ref(Qr, Dr, cu_q.tolist(), cu_d.tolist())
    (sr * G.cuda()).sum().backward()
    assert Qc.grad.dtype == dtype and Dc.grad.dtype == dtype
    assert rel_err(_np(s), _np(sr)) < tol
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < tol
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < tol
    # inference path gives the same scores; a second backward is bitwise identical
    with torch.no_grad():
        s0 = maxsim_varlen(Q.cuda(), D.cuda(), cu_q.cuda(), cu_d.cuda())
    assert torch.equal(s.detach(), s0)
    g1 = (Qc.grad.clone(), Dc.grad.clone())
    Qc.grad = None
    Dc.grad = None
    (maxsim_varlen(Qc, Dc, cu_q.cuda(), cu_d.cuda(), max_seqlen_q=40, max_seqlen_d=70) * G.cuda()).sum().backward()
    assert torch.equal(Qc.grad, g1[0]) and torch.equal(Dc.grad, g1[1])


def test_padded_grads():
    from late_interaction_kernels import maxsim_padded

    _case("maxsim_padded grads")
    g = torch.Generator().manual_seed(12)
    B, C, Lq, Ld, d = 4, 3, 20, 30, 64
    Q = torch.randn(B, Lq, d, generator=g)
    D = torch.randn(B, C, Ld, d, generator=g)
    ql = torch.tensor([20, 5, 0, 13])
    dl = torch.randint(0, Ld + 1, (B, C), generator=g)
    dl[0, 0] = 0
    dl[1, 2] = Ld
    Qc = Q.cuda().requires_grad_()
    Dc = D.cuda().requires_grad_()
    s = maxsim_padded(Qc, Dc, ql.cuda(), dl.cuda())
    G = torch.randn(B, C, generator=g).cuda()
    (s * G).sum().backward()
    Qr = Q.cuda().requires_grad_()
    Dr = D.cuda().requires_grad_()
    ref = []
    for b in range(B):
        row = []
        for c in range(C):
            qi, dj = Qr[b, : ql[b]], Dr[b, c, : dl[b, c]]
            row.append((qi @ dj.T).max(-1).values.sum() if len(qi) and len(dj) else Qr.sum() * 0)
        ref.append(torch.stack(row))
    sr = torch.stack(ref)
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 1e-4
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < 1e-3


def test_score_pairs_grads():
    from late_interaction_kernels.score_pairs import score_pairs_packed

    _case("score_pairs grads")
    g = torch.Generator().manual_seed(21)
    lq = torch.tensor([12, 0, 30, 7, 25, 3])
    ld = torch.tensor([40, 2, 0, 17, 33, 5, 64, 1])
    cu_q = torch.cat([torch.zeros(1, dtype=torch.long), lq.cumsum(0)]).to(torch.int32)
    cu_d = torch.cat([torch.zeros(1, dtype=torch.long), ld.cumsum(0)]).to(torch.int32)
    # duplicates, a query in many pairs, a doc in many pairs, an out-of-range pair
    pq = torch.tensor([0, 2, 2, 3, 4, 4, 4, 5, 1, 2, 0, 3, 2, 4, 9])
    pd = torch.tensor([0, 3, 3, 6, 1, 6, 4, 7, 0, 2, 6, 6, 6, 5, 0])
    Q = torch.randn(int(lq.sum()), 64, generator=g)
    D = torch.randn(int(ld.sum()), 64, generator=g)
    G = torch.randn(len(pq), generator=g).cuda()
    Qc = Q.cuda().requires_grad_()
    Dc = D.cuda().requires_grad_()
    s = score_pairs_packed(Qc, Dc, cu_q.cuda(), cu_d.cuda(), pq.cuda(), pd.cuda())
    (s * G).sum().backward()
    Qr = Q.cuda().requires_grad_()
    Dr = D.cuda().requires_grad_()
    ref = []
    for a, b in zip(pq.tolist(), pd.tolist()):
        if a >= len(lq) or b >= len(ld) or lq[a] == 0 or ld[b] == 0:
            ref.append(Qr.sum() * 0)
            continue
        qi = Qr[cu_q[a] : cu_q[a + 1]]
        dj = Dr[cu_d[b] : cu_d[b + 1]]
        ref.append((qi @ dj.T).max(-1).values.sum())
    sr = torch.stack(ref)
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 1e-4
    assert rel_err(_np(Qc.grad), _np(Qr.grad)) < 1e-3
    assert rel_err(_np(Dc.grad), _np(Dr.grad)) < 1e-3
    g1 = (Qc.grad.clone(), Dc.grad.clone())
    Qc.grad = None
    Dc.grad = None
    (score_pairs_packed(Qc, Dc, cu_q.cuda(), cu_d.cuda(), pq.cuda(), pd.cuda()) * G).sum().backward()
    assert torch.equal(Qc.grad, g1[0]) and torch.equal(Dc.grad, g1[1])
