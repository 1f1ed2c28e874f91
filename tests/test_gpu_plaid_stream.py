"""GPU parity of the few-query PLAID path (lik_plaid_stream.hip).

lik_plaid_maxsim scores up to 4 queries of <= 32 tokens with one wavefront
per (query, doc range). Its exact variants (per-lane and LDS-gather decode;
launch_options(plaid_variant=2) forces the gather one where the layout allows it) use
the tile kernel's arithmetic (same decode, norm tree, rounding, MFMA order
and per-query summation order), so their scores are bitwise equal to the
tile kernel's (launch_options(plaid_variant=3) forces that one). The default for
centroids of the query's type is the split form (q.c + q.r on the stored
centroid chunks and bf16 / fp16 bucket weights, norm from ||c||^2 + 2 c.r +
||r||^2): within bf16 tolerance of both. Everything is checked against the
oracle (oracle/lik_oracle.maxsim_residual[_varlen], reference.py:142-179,
plaid.py:832-963). Cases: nbits 2 / 4 / 8, bf16 / fp16 / fp32 centroids,
d = 64 / 96 / 128, empty docs, packed and padded layouts, 1 and 3 queries.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err
from late_interaction_kernels._lib import launch_options

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _index(Nd, max_ld, d, nbits, seed, cdtype):
    g = torch.Generator().manual_seed(seed)
    cent = torch.nn.functional.normalize(torch.randn(300, d, generator=g), dim=-1).to(cdtype)
    bw = torch.linspace(-0.05, 0.05, 2**nbits)
    lens = torch.randint(1, max_ld + 1, (Nd,), generator=g)
    lens[0] = 0
    lens[Nd // 2] = 0
    lens[3] = max_ld
    T = int(lens.sum())
    codes = torch.randint(0, 300, (T,), generator=g, dtype=torch.int32)
    bcodes = np.random.default_rng(seed).integers(0, 2**nbits, (T, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    return cent, bw, codes, res, cu, lens


@pytest.mark.parametrize("nbits", [2, 4, 8])
@pytest.mark.parametrize("cdtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [128, 96, 64])
@pytest.mark.parametrize("nq", [1, 3])
def test_stream_varlen_matches_tile_kernel(nbits, cdtype, d, nq):
    from late_interaction_kernels.plaid import maxsim_residual_varlen

    _case(f"stream varlen nbits={nbits} {cdtype} d={d} nq={nq}")
    cent, bw, codes, res, cu, _ = _index(700, 90, d, nbits, nbits * 31 + d + nq, cdtype)
    g = torch.Generator().manual_seed(d + nq)
    qdt = torch.float16 if cdtype == torch.float16 else torch.bfloat16
    Q = torch.randn(nq, 32, d, generator=g).to(qdt).cuda()
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    stream = maxsim_residual_varlen(Q, *args)
    with launch_options(plaid_variant=2):
        exact = maxsim_residual_varlen(Q, *args)
    with launch_options(plaid_variant=3):
        tile = maxsim_residual_varlen(Q, *args)
    assert torch.equal(exact, tile)
    assert rel_err(stream.cpu().numpy(), tile.cpu().numpy()) < 1e-2
    for s in (stream, exact):
        assert s[:, 0].abs().max().item() == 0.0 and s[:, 350].abs().max().item() == 0.0
    ref = O.maxsim_residual_varlen(Q.float().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                   cent.float().numpy(), bw.numpy(), nbits)
    assert rel_err(stream.cpu().numpy(), ref) < 1e-2
    assert rel_err(exact.cpu().numpy(), ref) < 1e-2


@pytest.mark.parametrize("lq", [32, 20])
def test_stream_padded_and_short_queries(lq):
    from late_interaction_kernels.plaid import maxsim_residual

    _case(f"stream padded lq={lq}")
    Nd, L, d, nbits = 300, 64, 128, 2
    cent, bw, codes, res, cu, lens = _index(Nd, L, d, nbits, 5, torch.bfloat16)
    # padded layout [Nd, L]: copy each doc's tokens into its row
    pc = torch.zeros(Nd, L, dtype=torch.int32)
    pr = torch.zeros(Nd, L, res.shape[1], dtype=torch.uint8)
    for j in range(Nd):
        n = int(lens[j])
        pc[j, :n] = codes[cu[j] : cu[j] + n]
        pr[j, :n] = res[cu[j] : cu[j] + n]
    Q = torch.randn(2, lq, d).to(torch.bfloat16).cuda()
    args = (pc.cuda(), pr.cuda(), lens.to(torch.int32).cuda(), cent.cuda(), bw.cuda(), nbits)
    stream = maxsim_residual(Q, *args)
    with launch_options(plaid_variant=2):
        exact = maxsim_residual(Q, *args)
    with launch_options(plaid_variant=3):
        tile = maxsim_residual(Q, *args)
    assert torch.equal(exact, tile)
    assert rel_err(stream.cpu().numpy(), tile.cpu().numpy()) < 1e-2
    ref = O.maxsim_residual(Q.float().cpu().numpy(), pc.numpy(), pr.numpy(), lens.numpy(), cent.float().numpy(),
                            bw.numpy(), nbits)
    assert rel_err(stream.cpu().numpy(), ref) < 1e-2


@pytest.mark.parametrize("normalize", [True, False])
def test_split_form_large_index(normalize):
    """The split form at the benchmark's layout (d = 128, nbits = 2, bf16
    centroids over a 4096-row table, docs of 30..300 tokens), one query,
    against the exact gather variant and the oracle: the split form drops
    only the bf16 rounding of the normalised token (and rounds the bucket
    weights to bf16), so it stays within a few 1e-3 of both."""
    from late_interaction_kernels.plaid import maxsim_residual_varlen

    _case(f"split large normalize={normalize}")
    g = torch.Generator().manual_seed(77)
    Nd, d, nbits, nc = 1000, 128, 2, 4096
    cent = torch.nn.functional.normalize(torch.randn(nc, d, generator=g), dim=-1).to(torch.bfloat16)
    bw = torch.linspace(-0.1, 0.1, 4)
    lens = torch.randint(30, 301, (Nd,), generator=g)
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    T = int(cu[-1])
    codes = torch.randint(0, nc, (T,), generator=g, dtype=torch.int32)
    res = torch.randint(0, 256, (T, d * nbits // 8), generator=g, dtype=torch.uint8)
    Q = torch.nn.functional.normalize(torch.randn(1, 32, d, generator=g), dim=-1).to(torch.bfloat16).cuda()
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    split = maxsim_residual_varlen(Q, *args, normalize=normalize)
    with launch_options(plaid_variant=2):
        exact = maxsim_residual_varlen(Q, *args, normalize=normalize)
    e = rel_err(split.cpu().numpy(), exact.cpu().numpy())
    print(f"split vs exact rel err {e:.2e}")
    assert e < 5e-3
    ref = O.maxsim_residual_varlen(Q.float().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                   cent.float().numpy(), bw.numpy(), nbits, normalize=normalize)
    assert rel_err(split.cpu().numpy(), ref) < 5e-3
