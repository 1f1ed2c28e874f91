"""CPU checks of late_interaction_kernels.reference, the public eager-PyTorch
ground-truth module (reference __init__.py:65, reference.py:26-306).

Each function is compared in float64 with the exact-rational known answers
(tests/golden/known_answers.json) where they apply, and with the pinned CPU
oracle on seeded inputs, including masks, empty docs and queries, 2-D squeeze
rules, and the residual bit layout. No GPU and no HIP library are needed:
the module is plain PyTorch.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import lik_oracle as O
from late_interaction_kernels import reference as R

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


@pytest.mark.parametrize("case", GOLD["maxsim"], ids=lambda c: c["name"])
def test_maxsim_reference_known_answers(case):
    got = R.maxsim_reference(torch.tensor(case["Q"], dtype=torch.float64), torch.tensor(case["D"], dtype=torch.float64),
                             torch.tensor(case["q_mask"]), torch.tensor(case["d_mask"]), normalize=case["normalize"])
    np.testing.assert_allclose(got.numpy(), np.array(case["expected"]), rtol=0, atol=1e-12)


@pytest.mark.parametrize("normalize", [False, True])
def test_maxsim_reference_masks_and_squeeze(normalize):
    g = torch.Generator().manual_seed(1)
    Q = torch.randn(4, 6, 16, generator=g, dtype=torch.float64)
    D = torch.randn(5, 9, 16, generator=g, dtype=torch.float64)
    qm = torch.rand(4, 6, generator=g) > 0.3
    dm = torch.rand(5, 9, generator=g) > 0.3
    dm[2] = False
    got = R.maxsim_reference(Q, D, qm, dm, normalize=normalize)
    ref = O.maxsim(Q.numpy(), D.numpy(), qm.numpy(), dm.numpy(), normalize=normalize)
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-12, atol=1e-12)
    assert np.all(got.numpy()[:, 2] == 0)
    assert R.maxsim_reference(Q[0], D[0]).shape == ()
    assert R.maxsim_reference(Q[0], D).shape == (5,)
    assert R.maxsim_reference(Q, D[0]).shape == (4,)
    # bf16 inputs are widened to fp32
    assert R.maxsim_reference(Q.bfloat16(), D.bfloat16()).dtype == torch.float32


def test_varlen_scatter_padded_reference():
    g = torch.Generator().manual_seed(2)
    lq = [3, 0, 5]
    ld = [4, 1, 0, 6]
    Qp = torch.randn(sum(lq), 8, generator=g)
    Dp = torch.randn(sum(ld), 8, generator=g)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32)
    cu_d = torch.tensor(np.concatenate([[0], np.cumsum(ld)]), dtype=torch.int32)
    got = R.maxsim_reference_varlen(Qp, Dp, cu_q, cu_d)
    ref = O.maxsim_varlen(Qp.numpy(), Dp.numpy(), cu_q.numpy(), cu_d.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
    pq = torch.tensor([0, 2, 2, 1, 0])
    pd = torch.tensor([3, 0, 2, 1, 1])
    got = R.maxsim_reference_scatter(Qp, Dp, cu_q, cu_d, pq, pd)
    ref = O.maxsim_pairs(Qp.numpy(), Dp.numpy(), cu_q.numpy(), cu_d.numpy(), pq.numpy(), pd.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
    q = torch.randn(3, 5, 8, generator=g)
    docs = torch.randn(3, 2, 7, 8, generator=g)
    qlen = torch.tensor([5, 0, 2])
    dlen = torch.tensor([[7, 1], [3, 3], [0, 4]])
    got = R.maxsim_padded_reference(q, docs, qlen, dlen)
    ref = O.maxsim_padded(q.numpy(), docs.numpy(), qlen.numpy(), dlen.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_residual_references(nbits):
    g = torch.Generator().manual_seed(nbits)
    d, B, L, C = 16, 3, 6, 10
    cent = torch.randn(C, d, generator=g)
    codes = torch.randint(0, C, (B, L), generator=g)
    res = torch.randint(0, 256, (B, L, d * nbits // 8), generator=g, dtype=torch.uint8)
    bw = torch.linspace(-0.2, 0.2, 2**nbits)
    np.testing.assert_array_equal(R.unpack_residuals_reference(res, nbits, d).numpy(),
                                  O.unpack_residuals(res.numpy(), nbits, d))
    lens = torch.tensor([6, 0, 3])
    Q = torch.randn(2, 4, d, generator=g)
    for normalize in (False, True):
        got = R.maxsim_residual_reference(Q, codes, res, lens, cent, bw, nbits, normalize=normalize)
        ref = O.maxsim_residual(Q.numpy(), codes.numpy(), res.numpy(), lens.numpy(), cent.numpy(), bw.numpy(),
                                nbits, normalize=normalize)
        np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)


def test_approx_and_from_hidden_references():
    g = torch.Generator().manual_seed(3)
    qcs = torch.randn(20, 5, generator=g)
    codes = torch.randint(0, 20, (4, 7), generator=g)
    lens = torch.tensor([7, 0, 3, 1])
    got = R.plaid_approx_score_reference(qcs, codes, lens)
    np.testing.assert_allclose(got.numpy(), O.plaid_approx_score(qcs.numpy(), codes.numpy(), lens.numpy()),
                               rtol=1e-5, atol=1e-6)
    Q = torch.nn.functional.normalize(torch.randn(2, 4, 8, generator=g), dim=-1)
    H = torch.randn(3, 6, 12, generator=g)
    W = torch.randn(8, 12, generator=g)
    b = torch.randn(8, generator=g)
    dm = torch.rand(3, 6, generator=g) > 0.2
    got = R.maxsim_from_hidden_reference(Q, H, W, b, dm)
    Dp = np.einsum("jth,oh->jto", H.numpy().astype(np.float64), W.numpy()) + b.numpy()
    Dn = Dp / np.linalg.norm(Dp, axis=-1, keepdims=True)
    ref = O.maxsim(Q.numpy(), Dn, None, dm.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
