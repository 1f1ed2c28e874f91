"""GPU edge cases of the dense MaxSim path (reference tests/test_edge_cases.py):
single-token docs and queries, embedding dims that are not multiples of 16 (or
of 8), including one above 512, and a rerank-sized call checked on sampled docs.
Oracle: lik_oracle.maxsim (reference.py:26-98) in float64."""

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
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_single_token_doc(dtype):
    from late_interaction_kernels import maxsim

    _case(f"single-token doc {dtype}")
    g = torch.Generator().manual_seed(1)
    Q = torch.randn(2, 8, 128, generator=g).to(dtype)
    D = torch.randn(3, 1, 128, generator=g).to(dtype)
    got = maxsim(Q.cuda(), D.cuda())
    ref = O.maxsim(_np(Q), _np(D))
    assert np.abs(_np(got) - ref).max() < 1e-2 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_single_query_token(dtype):
    from late_interaction_kernels import maxsim

    _case(f"single query token {dtype}")
    g = torch.Generator().manual_seed(2)
    Q = torch.randn(2, 1, 128, generator=g).to(dtype)
    D = torch.randn(3, 64, 128, generator=g).to(dtype)
    got = maxsim(Q.cuda(), D.cuda())
    ref = O.maxsim(_np(Q), _np(D))
    assert np.abs(_np(got) - ref).max() < 1e-2 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("d", [16, 33, 37, 63, 96, 111, 250, 513])
@pytest.mark.parametrize("normalize", [False, True])
def test_odd_embedding_dims(d, normalize):
    from late_interaction_kernels import maxsim

    _case(f"odd dim d={d} normalize={normalize}")
    g = torch.Generator().manual_seed(d)
    Q = torch.randn(2, 16, d, generator=g).to(torch.float16)
    D = torch.randn(3, 32, d, generator=g).to(torch.float16)
    got = maxsim(Q.cuda(), D.cuda(), normalize=normalize)
    ref = O.maxsim(_np(Q), _np(D), normalize=normalize)
    assert np.abs(_np(got) - ref).max() / max(1.0, np.abs(ref).max()) < 5e-3


@pytest.mark.parametrize("d", [33, 513])
def test_odd_embedding_dims_masked_bf16(d):
    """Odd dims through the masked and normalised variant, bf16."""
    from late_interaction_kernels import maxsim

    _case(f"odd dim masked d={d}")
    g = torch.Generator().manual_seed(d + 7)
    Q = torch.randn(3, 20, d, generator=g).to(torch.bfloat16)
    D = torch.randn(5, 45, d, generator=g).to(torch.bfloat16)
    qm = torch.arange(20)[None] < torch.tensor([20, 5, 1])[:, None]
    dm = torch.rand(5, 45, generator=g) > 0.3
    got = maxsim(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), normalize=True)
    ref = O.maxsim(_np(Q), _np(D), qm.numpy(), dm.numpy(), normalize=True)
    assert rel_err(_np(got), ref) < 2e-2


def test_large_batch_many_docs():
    """A rerank-sized call (1 x 32 query tokens against 1000 docs of 300): all
    scores computed, ten sampled docs checked against the oracle."""
    from late_interaction_kernels import maxsim

    _case("large batch many docs")
    g = torch.Generator().manual_seed(3)
    Q = torch.randn(1, 32, 128, generator=g).to(torch.float16)
    D = torch.randn(1000, 300, 128, generator=g).to(torch.float16)
    got = maxsim(Q.cuda(), D.cuda())
    idx = torch.randperm(1000, generator=g)[:10]
    ref = O.maxsim(_np(Q), _np(D[idx]))
    err = np.abs(_np(got)[:, idx.numpy()] - ref).max()
    assert err < 5e-3 * max(1.0, np.abs(ref).max())
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("dtype,d", [(torch.float32, 300), (torch.float32, 260), (torch.bfloat16, 600)])
def test_wide_rows_masked(dtype, d):
    """Rows wider than the tile kernel's column blocks (fp32 > 256, bf16 > 512)
    take the one-wave-per-pair kernel: masks, normalisation, Lq > 32."""
    from late_interaction_kernels import maxsim

    _case(f"wide rows {dtype} d={d}")
    g = torch.Generator().manual_seed(d)
    Q = torch.randn(3, 40, d, generator=g).to(dtype)
    D = torch.randn(4, 70, d, generator=g).to(dtype)
    qm = torch.arange(40)[None] < torch.tensor([40, 33, 2])[:, None]
    dm = torch.rand(4, 70, generator=g) > 0.4
    dm[2] = False
    got = maxsim(Q.cuda(), D.cuda(), qm.cuda(), dm.cuda(), normalize=True)
    ref = O.maxsim(_np(Q), _np(D), qm.numpy(), dm.numpy(), normalize=True)
    assert rel_err(_np(got), ref) < (1e-4 if dtype == torch.float32 else 1e-2)
    assert _np(got)[:, 2].max() == 0.0


def test_wide_rows_kd_and_varlen():
    from late_interaction_kernels import maxsim, maxsim_varlen

    _case("wide rows kd + varlen")
    g = torch.Generator().manual_seed(9)
    d = 600
    Q = torch.randn(3, 24, d, generator=g).to(torch.bfloat16)
    Dkd = torch.randn(3, 5, 50, d, generator=g).to(torch.bfloat16)
    got = maxsim(Q.cuda(), Dkd.cuda())
    ref = np.stack([O.maxsim(_np(Q[i : i + 1]), _np(Dkd[i]))[0] for i in range(3)])
    assert rel_err(_np(got), ref) < 1e-2
    ql, dl = [24, 3, 17], [50, 1, 0, 33]
    Qp = torch.randn(sum(ql), d, generator=g).to(torch.bfloat16)
    Dp = torch.randn(sum(dl), d, generator=g).to(torch.bfloat16)
    cq = torch.tensor([0] + np.cumsum(ql).tolist(), dtype=torch.int32)
    cd = torch.tensor([0] + np.cumsum(dl).tolist(), dtype=torch.int32)
    got = maxsim_varlen(Qp.cuda(), Dp.cuda(), cq.cuda(), cd.cuda())
    ref = np.zeros((3, 4))
    for i in range(3):
        for k in range(4):
            if dl[k] and ql[i]:
                ref[i, k] = O.maxsim(_np(Qp[cq[i] : cq[i + 1]]), _np(Dp[cd[k] : cd[k + 1]]))
    assert rel_err(_np(got), ref) < 1e-2


@pytest.mark.parametrize("d", [48, 64, 300, 512])
@pytest.mark.parametrize("normalize", [False, True])
def test_bf16_narrow_and_wide_rows(d, normalize):
    """bf16 at d <= 64 and 256 < d <= 512 runs kernels with only the call's
    features compiled in (none; query-only or full normalise): one query
    (a corpus scan) and six, prefix doc masks (the extent path) and an
    empty doc, against the oracle."""
    from late_interaction_kernels import maxsim

    _case(f"bf16 d={d} normalize={normalize}")
    g = torch.Generator().manual_seed(d + int(normalize))
    D = torch.randn(40, 70, d, generator=g).to(torch.bfloat16)
    dm = torch.arange(70)[None] < torch.randint(1, 71, (40,), generator=g)[:, None]
    dm[7] = False
    for nq in (1, 6):
        Q = torch.randn(nq, 32, d, generator=g).to(torch.bfloat16)
        got = maxsim(Q.cuda(), D.cuda(), d_mask=dm.cuda(), normalize=normalize)
        ref = O.maxsim(_np(Q), _np(D), None, dm.numpy(), normalize=normalize)
        assert rel_err(_np(got).reshape(ref.shape), ref) < 1e-2, nq
        assert _np(got).reshape(ref.shape)[:, 7].max() == 0.0
