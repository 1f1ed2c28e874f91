"""The doc-mask summary ahead of the tile kernels (doc_extent_kernel and its
dword-per-lane form doc_extent_w4_kernel in lik_maxsim.hip): per doc the
extent (last kept token + 1), whether the kept tokens have holes, and one
validity word per 32-token tile. A wrong summary scores the wrong tokens, so
each case compares the scores with the oracle (lik_oracle.maxsim,
reference.py:26-98) within the bf16 tolerance.

* Contiguous, 4-byte-aligned masks with L <= 1024 take the dword form: L
  around the dword, tile and 256-token chunk edges (1, 3, 31, 33, 255, 256,
  257, 301, 1024), holes in a row's last dword, prefix masks, a mask that keeps
  nothing, and a broadcast mask (row stride 0).
* A mask view whose base is not 4-byte aligned, a row stride that is not a
  multiple of 4, and L = 1025 take the byte-per-lane kernel.
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


def _score(Q, D, dm):
    from late_interaction_kernels import maxsim

    got = maxsim(Q.cuda(), D.cuda(), None, dm.cuda(), normalize=False)
    ref = O.maxsim(_np(Q), _np(D), None, dm.numpy(), normalize=False)
    gn = _np(got)
    assert np.all(np.isfinite(gn))
    assert rel_err(gn, ref) < 1e-2


def _mask(nd, L, g, kind):
    lens = torch.randint(0, L + 1, (nd,), generator=g)
    lens[0], lens[1] = L, min(L, 1)
    dm = torch.arange(L)[None] < lens[:, None]
    if kind == "holes":
        dm[::3, ::7] = False  # holes everywhere, including a row's last dword
        dm[1::3, L - 1] = True
        dm[2::5, max(L - 2, 0)] = False
    elif kind == "empty_row":
        dm[3] = False
    return dm


@pytest.mark.parametrize("L", [1, 3, 31, 33, 255, 256, 257, 301, 1024])
@pytest.mark.parametrize("kind", ["prefix", "holes", "empty_row"])
def test_mask_summary_dword_form(L, kind):
    _case(f"mask summary dword L={L} {kind}")
    g = torch.Generator().manual_seed(L * 7 + len(kind))
    nd = 40
    Q = torch.randn(3, 8, 64, generator=g).to(torch.bfloat16)
    D = torch.randn(nd, L, 64, generator=g).to(torch.bfloat16)
    _score(Q, D, _mask(nd, L, g, kind))


def test_mask_summary_broadcast():
    _case("mask summary broadcast row")
    g = torch.Generator().manual_seed(11)
    L = 77
    Q = torch.randn(2, 8, 64, generator=g).to(torch.bfloat16)
    D = torch.randn(30, L, 64, generator=g).to(torch.bfloat16)
    row = torch.rand(L, generator=g) > 0.3
    dm = row[None].expand(30, L)  # stride 0 over docs
    assert dm.stride(0) == 0
    _score(Q, D, dm)


@pytest.mark.parametrize("form", ["unaligned_base", "odd_row_stride", "long_rows"])
def test_mask_summary_byte_form(form):
    _case(f"mask summary byte form {form}")
    g = torch.Generator().manual_seed(len(form))
    nd = 24
    L = 1025 if form == "long_rows" else 90
    Q = torch.randn(2, 8, 64, generator=g).to(torch.bfloat16)
    D = torch.randn(nd, L, 64, generator=g).to(torch.bfloat16)
    base = _mask(nd, L + 1, g, "holes")
    if form == "unaligned_base":
        dm = base.cuda()[:, 1:]  # data pointer one byte past an aligned block
        assert dm.data_ptr() % 4 != 0
    elif form == "odd_row_stride":
        dm = base.cuda()[:, :L]  # row stride L + 1 = 91, not a multiple of 4
        assert dm.stride(0) % 4 != 0
    else:
        dm = base.cuda()[:, :L]
    from late_interaction_kernels import maxsim

    got = maxsim(Q.cuda(), D.cuda(), None, dm, normalize=False)
    ref = O.maxsim(_np(Q), _np(D), None, dm.cpu().numpy(), normalize=False)
    assert rel_err(_np(got), ref) < 1e-2
