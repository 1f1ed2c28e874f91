"""GPU parity at sizes where 32-bit offsets would overflow: a score matrix of
more than 2**31 entries and a packed token buffer larger than 4 GiB. The full
outputs are too large for the CPU oracle, so sampled documents (the last ones
among them, whose offsets are the largest) are checked against
lik_oracle.maxsim (reference.py:26-98), and every score must be finite.
Inputs are generated on the device."""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().float().cpu().numpy()


def _sample(n, g, k=48, tail=16):
    idx = torch.cat([torch.randint(0, n, (k,), generator=g), torch.arange(n - tail, n)])
    return torch.unique(idx)


def test_scores_beyond_2_pow_31_entries():
    """[64, 2**25 + 4096] scores (2.15e9 entries, 8.6 GB): output offsets past
    2**31 elements, docs of 4 tokens with random prefix masks."""
    from late_interaction_kernels import maxsim

    Nq, Lq, Nd, Ld, d = 64, 8, (1 << 25) + 4096, 4, 16
    _case(f"scores > 2^31: Nq={Nq} Nd={Nd} Ld={Ld} d={d}")
    assert Nq * Nd > 2**31
    gd = torch.Generator(device="cuda").manual_seed(11)
    Q = torch.randn(Nq, Lq, d, generator=gd, device="cuda", dtype=torch.bfloat16) * 0.25  # unit-scale rows
    D = torch.randn(Nd, Ld, d, generator=gd, device="cuda", dtype=torch.bfloat16)
    lens = torch.randint(1, Ld + 1, (Nd,), generator=gd, device="cuda")
    dm = torch.arange(Ld, device="cuda")[None] < lens[:, None]
    got = maxsim(Q, D, d_mask=dm)
    assert got.shape == (Nq, Nd)
    assert bool(torch.isfinite(got).all())
    idx = _sample(Nd, torch.Generator().manual_seed(12)).cuda()
    ref = O.maxsim(_np(Q), _np(D[idx]), d_mask=dm[idx].cpu().numpy())
    out = _np(got[:, idx])
    del got, D
    assert np.abs(out - ref).max() < 1e-2 * max(1.0, np.abs(ref).max())


def test_varlen_packed_buffer_beyond_4_gib():
    """maxsim_varlen over 17.3M packed bf16 tokens of d = 128 (4.4 GB): doc
    byte offsets past 2**32, lengths U[100, 300]."""
    from late_interaction_kernels import maxsim_varlen

    d, Lq, Nq = 128, 32, 4
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(100, 301, (86_000,), generator=g, dtype=torch.int32)
    cu_d = torch.zeros(lens.numel() + 1, dtype=torch.int32)
    cu_d[1:] = torch.cumsum(lens, 0)
    T = int(cu_d[-1])
    _case(f"varlen > 4 GiB: Nd={lens.numel()} T={T} d={d}")
    assert T * d * 2 > 2**32
    gd = torch.Generator(device="cuda").manual_seed(22)
    D = torch.randn(T, d, generator=gd, device="cuda", dtype=torch.bfloat16)
    Q = torch.randn(Nq * Lq, d, generator=gd, device="cuda", dtype=torch.bfloat16)
    cu_q = torch.arange(0, Nq * Lq + 1, Lq, dtype=torch.int32)
    got = maxsim_varlen(Q, D, cu_q.cuda(), cu_d.cuda(), max_seqlen_q=Lq, max_seqlen_d=300)
    assert got.shape == (Nq, lens.numel())
    assert bool(torch.isfinite(got).all())
    Qn = _np(Q).reshape(Nq, Lq, d)
    idx = _sample(lens.numel(), g, k=24, tail=8)
    out = _np(got)
    for j in idx.tolist():
        rows = _np(D[int(cu_d[j]) : int(cu_d[j + 1])])
        ref = O.maxsim(Qn, rows[None])[:, 0]
        assert np.abs(out[:, j] - ref).max() < 1e-2 * max(1.0, np.abs(ref).max()), j


@pytest.mark.parametrize("largest", [True, False])
def test_topk_select_very_wide_rows(largest):
    """One top-100 select over 2**28 + 17 scores per row (the tree select's
    many-level case), continuing a running list whose indices start past
    2**31 - 2**28 so the selected indices exceed 2**31. Scores are random
    floats (many exact ties: 2**28 draws of a 24-bit grid) with planted ties at the best value; expected: order by score, ties to
    the lower index (numpy over the full rows)."""
    from late_interaction_kernels.topk import topk_update

    R, n, k = 2, (1 << 28) + 17, 100
    base = (1 << 31) - (1 << 28) + 5
    _case(f"topk wide rows R={R} n={n} k={k} largest={largest}")
    gd = torch.Generator(device="cuda").manual_seed(31)
    s = torch.rand(R, n, generator=gd, device="cuda")
    # ties at the extreme: the same best value at a high and a low column
    best = 2.0 if largest else -1.0
    s[:, n - 3] = best
    s[:, 7] = best
    s[1, n - 1] = best
    run_s, run_i = topk_update(s, base, None, None, k, largest)
    sh = s.cpu().numpy()
    del s
    for r in range(R):
        row = sh[r] if largest else -sh[r]
        kth = np.partition(-row, k - 1)[k - 1]  # every column tied with the k-th best stays a candidate
        cand = np.nonzero(-row <= kth)[0]
        order = sorted(cand.tolist(), key=lambda c: (-row[c], c))[:k]
        assert run_i[r].cpu().numpy().tolist() == [base + c for c in order], r
        np.testing.assert_array_equal(run_s[r].cpu().numpy(), sh[r][order])
