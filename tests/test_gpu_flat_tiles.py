"""GPU parity of the tile kernel's flat tiles.

In the two-workgroup DMA kernel (bf16 / fp16, d = 128, 4 waves x 4 column
blocks), a workgroup whose non-empty docs are all >= 32 tokens walks them as
32-row windows laid end to end: a doc ends inside a tile and the next doc
starts there. These cases put the boundary at every row of a tile (doc
lengths 32 + 7 k cover every residue mod 32), put a workgroup's last doc end
exactly on a tile end, mix workgroups that take flat tiles with workgroups
that hold a short doc (per-doc tiles), and put NaN / inf tokens on both sides
of a boundary (reference.py:83-85: a NaN row max scores the doc 0). Each is
compared with the oracle (oracle/lik_oracle.py) within the bf16 tolerance.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err
from late_interaction_kernels._lib import launch_options

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().double().cpu().numpy()


def _lengths(nd, short=()):
    lens = torch.tensor([32 + (7 * k) % 269 for k in range(nd)])
    for j in short:
        lens[j] = 5 + j % 20
    return lens


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("docs_per_wg", [1, 3, 8, 37, 64])
@pytest.mark.parametrize("short", [(), (17,), (0, 40, 41)])
def test_flat_tiles_padded(dtype, docs_per_wg, short):
    from late_interaction_kernels import maxsim

    Nq, Lq, Nd, Ld, d = 16, 32, 96, 300, 128
    _case(f"flat padded {dtype} R={docs_per_wg} short={short}")
    g = torch.Generator().manual_seed(docs_per_wg * 10 + len(short))
    Q = torch.randn(Nq, Lq, d, generator=g)
    D = torch.randn(Nd, Ld, d, generator=g)
    lens = _lengths(Nd, short)
    dm = torch.arange(Ld)[None] < lens[:, None]
    D[~dm] = NAN  # past each doc's prefix: never read
    Qd, Dd = Q.to(dtype), D.to(dtype)
    with launch_options(cfg=(4, 4), docs_per_wg=docs_per_wg):
        got = maxsim(Qd.cuda(), Dd.cuda(), None, dm.cuda(), normalize=False)
    ref = O.maxsim(_np(Qd), np.nan_to_num(_np(Dd)) * dm.numpy()[..., None], None, dm.numpy(), normalize=False)
    gn = _np(got)
    assert np.all(np.isfinite(gn))
    assert rel_err(gn, ref) < 1e-2


@pytest.mark.parametrize("docs_per_wg", [2, 5, 64])
def test_flat_tiles_varlen(docs_per_wg):
    from late_interaction_kernels import maxsim_varlen

    _case(f"flat varlen R={docs_per_wg}")
    g = torch.Generator().manual_seed(docs_per_wg)
    d, nq = 128, 16
    q_lens = torch.full((nq,), 32)
    d_lens = _lengths(80)
    cu_q = torch.zeros(nq + 1, dtype=torch.int32)
    cu_q[1:] = torch.cumsum(q_lens, 0)
    cu_d = torch.zeros(len(d_lens) + 1, dtype=torch.int32)
    cu_d[1:] = torch.cumsum(d_lens, 0)
    Qp = torch.randn(int(cu_q[-1]), d, generator=g).to(torch.bfloat16)
    Dp = torch.randn(int(cu_d[-1]), d, generator=g).to(torch.bfloat16)
    with launch_options(cfg=(4, 4), docs_per_wg=docs_per_wg):
        got = maxsim_varlen(Qp.cuda(), Dp.cuda(), cu_q.cuda(), cu_d.cuda())
    ref = O.maxsim_varlen(_np(Qp), _np(Dp), cu_q.numpy(), cu_d.numpy())
    assert rel_err(_np(got), ref) < 1e-2


@pytest.mark.parametrize("where", ["last_row", "first_row", "both"])
def test_flat_tiles_nonfinite_at_boundary(where):
    from late_interaction_kernels import maxsim

    _case(f"flat nonfinite {where}")
    Nq, Lq, Nd, Ld, d = 16, 32, 24, 200, 128
    g = torch.Generator().manual_seed(7)
    Q = torch.randn(Nq, Lq, d, generator=g)
    D = torch.randn(Nd, Ld, d, generator=g)
    lens = _lengths(Nd)
    dm = torch.arange(Ld)[None] < lens[:, None]
    poisoned = []
    for j in (3, 10, 11):
        if where in ("last_row", "both"):
            D[j, int(lens[j]) - 1, 2] = NAN  # last row of doc j, inside a tile shared with doc j + 1
            poisoned.append(j)
        if where in ("first_row", "both"):
            D[j + 1, 0, 5] = NAN  # first row of doc j + 1
            poisoned.append(j + 1)
    D[5, int(lens[5]) - 1, 0] = INF  # +inf similarity against some query tokens: they score 0
    D[~dm] = 0.0
    Qd, Dd = Q.to(torch.bfloat16), D.to(torch.bfloat16)
    with launch_options(cfg=(4, 4), docs_per_wg=Nd):
        got = maxsim(Qd.cuda(), Dd.cuda(), None, dm.cuda(), normalize=False)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.maxsim(_np(Qd), _np(Dd), None, dm.numpy(), normalize=False)
    gn = _np(got)
    assert np.all(np.isfinite(gn))
    for j in sorted(set(poisoned)):
        assert np.all(gn[:, j] == 0.0), j
    keep = [j for j in range(Nd) if j not in poisoned]
    assert rel_err(gn[:, keep], ref[:, keep]) < 1e-2
