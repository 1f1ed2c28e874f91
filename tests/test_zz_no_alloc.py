"""GPU test of lik_maxsim_noalloc, the allocation-free scoring entry point.

It is called through the C ABI (ctypes) and compared with lik_maxsim, the
entry point it mirrors, on two calls in a row that share the library's
per-device scratch array, the second with a smaller input: a masked batch
with holes (mask summaries in scratch) whose queries are longer than one
column block (query-chunk partial sums in scratch), then a smaller
normalised one. Without doc normalisation both entry points run the same
plan, so the scores are bitwise equal; with it lik_maxsim pre-normalises the
docs and may pick another column block, so the scores agree to fp32 rounding
of the per-query sums (1e-5 relative). A call whose scratch need exceeds the
fixed size is rejected on the host with LIK_ERR_WORKSPACE.
"""

import ctypes
import sys

import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _seqs(x, mask=None):
    from late_interaction_kernels import _lib

    m = None if mask is None else mask.view(torch.int8)
    return _lib.seqs(x, n=x.shape[0], length=x.shape[1], stride_n=x.stride(0), stride_l=x.stride(1), mask=m,
                     mask_strides=(m.stride(0), m.stride(1)) if m is not None else (0, 0))


def _both(Q, D, dm, flags):
    """(lik_maxsim scores, lik_maxsim_noalloc scores) for the same call."""
    from late_interaction_kernels import _lib

    lib = _lib.load()
    qs, ds = _seqs(Q), _seqs(D, dm)
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.empty(Q.shape[0], D.shape[0], device="cuda")
    nbytes = lib.lik_maxsim_workspace_size(ctypes.byref(qs), ctypes.byref(ds), flags)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    _lib.check(lib.lik_maxsim(ctypes.byref(qs), ctypes.byref(ds), flags, 1.0, ref.data_ptr(), ref.stride(0),
                              ref.stride(1), ws.data_ptr(), nbytes, stream), "lik_maxsim")
    got = torch.full_like(ref, float("nan"))
    _lib.check(lib.lik_maxsim_noalloc(ctypes.byref(qs), ctypes.byref(ds), flags, 1.0, got.data_ptr(), got.stride(0),
                                      got.stride(1), stream), "lik_maxsim_noalloc")
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_matches_lik_maxsim_twice():
    from late_interaction_kernels import _lib

    g = torch.Generator(device="cuda").manual_seed(41)
    # call 1: 40 queries of 700 tokens (two query chunks), 300 docs with a
    # prefix mask, some holes and an empty doc
    _case("noalloc call 1: Lq=700 masked")
    Q = torch.randn(40, 700, 128, generator=g, device="cuda").to(torch.bfloat16)
    D = torch.randn(300, 90, 128, generator=g, device="cuda").to(torch.bfloat16)
    dm = torch.arange(90, device="cuda")[None] < torch.randint(0, 91, (300,), generator=g, device="cuda")[:, None]
    dm[7, 3:9] = False
    dm[11] = False
    ref, got = _both(Q, D, dm, 0)
    assert torch.equal(got, ref)
    # call 2, smaller: normalised, fewer docs, no query chunks
    _case("noalloc call 2: smaller, normalize")
    Q2 = torch.randn(20, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    D2 = torch.randn(64, 50, 128, generator=g, device="cuda").to(torch.bfloat16)
    dm2 = torch.arange(50, device="cuda")[None] < torch.randint(1, 51, (64,), generator=g, device="cuda")[:, None]
    dm2[3, 0] = False
    ref2, got2 = _both(Q2, D2, dm2, _lib.LIK_NORMALIZE)
    assert rel_err(got2.cpu().numpy(), ref2.cpu().numpy()) < 1e-5
    # and the first call again after the second used the scratch
    _, again = _both(Q, D, dm, 0)
    assert torch.equal(again, ref)


def test_noalloc_rejects_oversize_scratch():
    """8M one-token docs with a mask need ~72 MB of mask summaries, more than
    the 64 MiB scratch: rejected before any launch, output untouched."""
    from late_interaction_kernels import _lib

    _case("noalloc oversize")
    lib = _lib.load()
    n = 8 << 20
    Q = torch.zeros(2, 8, 128, device="cuda", dtype=torch.bfloat16)
    D = torch.zeros(n, 1, 128, device="cuda", dtype=torch.bfloat16)
    dm = torch.ones(n, 1, device="cuda", dtype=torch.bool)
    qs, ds = _seqs(Q), _seqs(D, dm)
    out = torch.full((2, n), 7.0, device="cuda")
    rc = lib.lik_maxsim_noalloc(ctypes.byref(qs), ctypes.byref(ds), 0, 1.0, out.data_ptr(), out.stride(0),
                                out.stride(1), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.LIK_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
