"""GPU parity of the tile kernel's flat tiles.

In the two-workgroup DMA kernel (bf16 / fp16, d = 128, 4 waves x 4 column
blocks), a workgroup whose non-empty docs are all >= 32 tokens (packed docs:
>= 16, at most 1 in 16 under 32) walks them as 32-row windows laid end to
end: a doc ends inside a tile and the next doc starts there. These cases put
the boundary at every row of a tile (doc lengths 32 + 7 k cover every residue
mod 32), put a workgroup's last doc end exactly on a tile end, put two doc
ends in one tile (the second also exactly at its end), mix workgroups that
take flat tiles with workgroups that hold a short doc (per-doc tiles), and
put NaN / inf tokens on both sides of a boundary (reference.py:83-85: a NaN
row max scores the doc 0). Each is
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


def _rare_short_lengths(n):
    """Mostly 40..239 tokens, every 17th doc 16..31 (under 1 in 16, so packed
    ranges keep flat tiles): some tiles hold two doc ends, some of them with
    the second exactly at the tile's end (checked in the test)."""
    return [16 + (3 * k + 3) % 16 if k % 17 == 5 else 40 + (7 * k) % 200 for k in range(n)]


def _two_end_tiles(lens, r):
    """(two-end tiles, of them with the second end at row 32) over the ranges
    of r docs that take flat tiles (docs >= 16 tokens, at most 1 in 16 under 32)."""
    two = at32 = 0
    for w0 in range(0, len(lens), r):
        ls = lens[w0:w0 + r]
        if min(ls) < 16 or 16 * sum(x < 32 for x in ls) > len(ls):
            continue
        ends, pos = {}, 0
        for x in ls:
            pos += x
            ends.setdefault((pos - 1) // 32, []).append(pos - 32 * ((pos - 1) // 32))
        for bs in ends.values():
            if len(bs) >= 2:
                two += 1
                at32 += bs[1] == 32
    return two, at32


@pytest.mark.parametrize("docs_per_wg", [2, 5, 37, 64])
@pytest.mark.parametrize("short", [False, True])
def test_flat_tiles_varlen(docs_per_wg, short):
    """Packed docs take flat tiles down to 16 tokens: a doc of 16..31 tokens
    can sit entirely inside a tile, which then holds two doc ends."""
    from late_interaction_kernels import maxsim_varlen

    _case(f"flat varlen R={docs_per_wg} short={short}")
    g = torch.Generator().manual_seed(docs_per_wg + 100 * short)
    d, nq = 128, 16
    q_lens = torch.full((nq,), 32)
    if short:
        lens = _rare_short_lengths(200)
        if docs_per_wg in (37, 64):
            two, at32 = _two_end_tiles(lens, docs_per_wg)
            assert two > 0 and at32 > 0  # the cases this test is for
        d_lens = torch.tensor(lens)
    else:
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
