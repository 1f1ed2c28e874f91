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
