"""GPU parity of the Q gradients of the PLAID scorers and of maxsim_from_hidden.

* maxsim_residual / maxsim_residual_varlen with ``Q.requires_grad``: scores and
  grad_Q match torch autograd on a plain fp32 restatement over the oracle's
  decoded docs (oracle/lik_oracle.decode_residual_tokens, reference.py:124-139).
  Two input families keep every MaxSim winner unambiguous at bf16 precision,
  so a gradient row never depends on tie order:
  - ``exact``: integer centroids, quarter-step bucket weights, no normalise;
    every product is exact in fp32, grad_Q is exact up to the final bf16 round;
  - ``spread``: one-hot centroids and query tokens whose 16 live coordinates
    are a permutation of 1..16, so cosine gaps between distinct codes are
    >= 1/38 against bf16 errors of ~0.006 (exercises the normalise Jacobian).
  Tolerance: rel 1e-2 (bf16 gradient rows).
* maxsim_from_hidden: scores and the gradients of Q, H_d, W, b match torch
  autograd on ``maxsim(Q, normalize(F.linear(H_d, W, b)))`` (reference
  fused_head.py:262-332) at rel 1e-3 for fp32 inputs.
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


def _index(T, family, nbits, seed, d=128):
    g = torch.Generator().manual_seed(seed)
    nb = 2**nbits
    if family == "exact":
        cent = torch.randint(-8, 9, (64, d), generator=g).float()
        bw = (torch.arange(nb, dtype=torch.float32) - nb // 2) / 4.0
        codes = torch.randint(0, 64, (T,), generator=g, dtype=torch.int32)
    else:
        cent = torch.zeros(16, d)
        cent[torch.arange(16), torch.arange(16)] = 1.0
        bw = torch.linspace(-0.002, 0.002, nb)
        codes = torch.randint(0, 16, (T,), generator=g, dtype=torch.int32)
    bcodes = np.random.default_rng(seed).integers(0, nb, (T, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    return cent, bw, codes, res


def _queries(Nq, Lq, family, seed, d=128):
    g = torch.Generator().manual_seed(seed + 1)
    if family == "exact":
        return torch.randn(Nq, Lq, d, generator=g).to(torch.bfloat16)
    Q = torch.zeros(Nq, Lq, d)
    for i in range(Nq):
        for s in range(Lq):
            Q[i, s, :16] = (torch.randperm(16, generator=g) + 1).float()
    return Q.to(torch.bfloat16)


def _torch_scores(Q, emb, cu, normalize):
    """fp32 autograd MaxSim of Q [Nq, Lq, d] against ragged docs emb[cu[j]:cu[j+1]]."""
    if normalize:
        Q = torch.nn.functional.normalize(Q, dim=-1)
        emb = torch.nn.functional.normalize(emb, dim=-1)
    cols = []
    for j in range(len(cu) - 1):
        Dj = emb[cu[j] : cu[j + 1]]
        if Dj.shape[0] == 0:
            cols.append(torch.zeros(Q.shape[0], device=Q.device))
        else:
            cols.append(torch.einsum("isd,td->ist", Q, Dj).max(-1).values.sum(-1))
    return torch.stack(cols, 1)


@pytest.mark.parametrize("family,normalize", [("exact", False), ("spread", True), ("spread", False)])
@pytest.mark.parametrize("nbits", [2, 4])
def test_residual_varlen_q_grad(family, normalize, nbits):
    from late_interaction_kernels.plaid import maxsim_residual_varlen

    _case(f"residual varlen grad {family} norm={normalize} nbits={nbits}")
    g = torch.Generator().manual_seed(nbits)
    Nd = 13
    lens = torch.randint(1, 40, (Nd,), generator=g)
    lens[3] = 0
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    T = int(cu[-1])
    cent, bw, codes, res = _index(T, family, nbits, 10 + nbits)
    Q = _queries(5, 24, family, nbits)
    Qg = Q.cuda().requires_grad_()
    s = maxsim_residual_varlen(Qg, codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits,
                               normalize=normalize)
    G = torch.randn(5, Nd, generator=g).cuda()
    (s * G).sum().backward()
    emb = torch.from_numpy(O.decode_residual_tokens(codes.numpy(), res.numpy(), cent.numpy(), bw.numpy(), nbits))
    Qr = Q.float().cuda().requires_grad_()
    sr = _torch_scores(Qr, emb.float().cuda(), cu.tolist(), normalize)
    (sr * G).sum().backward()
    assert Qg.grad.dtype == torch.bfloat16 and Qg.grad.shape == Q.shape
    assert rel_err(_np(s), _np(sr)) < 1e-2
    assert rel_err(_np(Qg.grad), _np(Qr.grad)) < 1e-2
    # scores of the differentiable path equal the inference path's
    with torch.no_grad():
        s0 = maxsim_residual_varlen(Q.cuda(), codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits,
                                    normalize=normalize)
    assert rel_err(_np(s), _np(s0)) < 1e-5


def test_residual_padded_q_grad():
    from late_interaction_kernels.plaid import maxsim_residual

    _case("residual padded grad")
    g = torch.Generator().manual_seed(4)
    Nd, L, nbits = 9, 30, 2
    lens = torch.randint(1, L + 1, (Nd,), generator=g)
    lens[1] = 0
    lens[4] = L
    cent, bw, codes, res = _index(Nd * L, "spread", nbits, 5)
    Q = _queries(3, 16, "spread", 6)
    Qg = Q.float().cuda().requires_grad_()  # fp32 leaf: gradient comes back in fp32
    s = maxsim_residual(Qg, codes.view(Nd, L).cuda(), res.view(Nd, L, -1).cuda(), lens.cuda(), cent.cuda(),
                        bw.cuda(), nbits)
    G = torch.randn(3, Nd, generator=g).cuda()
    (s * G).sum().backward()
    emb = torch.from_numpy(O.decode_residual_tokens(codes.numpy(), res.numpy(), cent.numpy(), bw.numpy(), nbits))
    keep = torch.cat([torch.arange(j * L, j * L + int(lens[j])) for j in range(Nd)])
    cu = [0] + lens.cumsum(0).tolist()
    Qr = Q.float().cuda().requires_grad_()
    sr = _torch_scores(Qr, emb.float()[keep].cuda(), cu, True)
    (sr * G).sum().backward()
    assert Qg.grad.dtype == torch.float32
    assert rel_err(_np(s), _np(sr)) < 1e-2
    assert rel_err(_np(Qg.grad), _np(Qr.grad)) < 1e-2
    assert s[:, 1].abs().max().item() == 0.0


def _hidden_ref(Q, H, W, b, dm, normalize):
    D = torch.nn.functional.linear(H, W, b)
    if normalize:
        D = torch.nn.functional.normalize(D, dim=-1)
    S = torch.einsum("isd,jtd->ijst", Q, D)
    if dm is not None:
        S = S.masked_fill(~dm[None, :, None, :], float("-inf"))
    m = S.max(-1).values
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    return m.sum(-1)


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("bias", [True, False])
def test_maxsim_from_hidden_grads(normalize, bias):
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    _case(f"from_hidden norm={normalize} bias={bias}")
    g = torch.Generator().manual_seed(3 + normalize + 2 * bias)
    Nq, Lq, Nd, Ld, dm_, do = 4, 32, 7, 45, 256, 128
    Q = torch.nn.functional.normalize(torch.randn(Nq, Lq, do, generator=g), dim=-1)
    H = torch.randn(Nd, Ld, dm_, generator=g)
    W = torch.randn(do, dm_, generator=g) / 16
    b = torch.randn(do, generator=g) / 4 if bias else None
    dm = torch.arange(Ld)[None] < torch.randint(1, Ld + 1, (Nd,), generator=g)[:, None]
    dm[2] = False
    leaves = [t.cuda().requires_grad_() for t in (Q, H, W) + ((b,) if bias else ())]
    s = maxsim_from_hidden(leaves[0], leaves[1], leaves[2], leaves[3] if bias else None, dm.cuda(), normalize)
    G = torch.randn(Nq, Nd, generator=g).cuda()
    (s * G).sum().backward()
    refs = [t.cuda().requires_grad_() for t in (Q, H, W) + ((b,) if bias else ())]
    sr = _hidden_ref(refs[0], refs[1], refs[2], refs[3] if bias else None, dm.cuda(), normalize)
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 1e-4
    for a, r in zip(leaves, refs):
        assert rel_err(_np(a.grad), _np(r.grad)) < 1e-3
    assert s[:, 2].abs().max().item() == 0.0
    with torch.no_grad():  # inference path and 2-D Q
        s1 = maxsim_from_hidden(Q[0].cuda(), H.cuda(), W.cuda(), b.cuda() if bias else None, dm.cuda(), normalize)
    assert s1.shape == (Nd,)
    assert rel_err(_np(s1), _np(sr[0])) < 1e-4


def test_maxsim_from_hidden_validation():
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    _case("from_hidden validation")
    Q = torch.randn(2, 4, 8).cuda()
    H = torch.randn(3, 5, 16).cuda()
    with pytest.raises(ValueError, match="W must be"):
        maxsim_from_hidden(Q, H, torch.randn(8, 15).cuda())
    with pytest.raises(ValueError, match="b must be"):
        maxsim_from_hidden(Q, H, torch.randn(8, 16).cuda(), torch.randn(7).cuda())
    with pytest.raises(ValueError, match="H_d must be"):
        maxsim_from_hidden(Q, H[0], torch.randn(8, 16).cuda())
