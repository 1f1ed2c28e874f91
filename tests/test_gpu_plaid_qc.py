"""GPU parity of the prepared-corpus PLAID scan (plaid.ResidualIndex,
lik_plaid_token_records / lik_plaid_token_norms + lik_plaid_maxsim_qc).

* Token inverse norms equal 1 / max(||centroid + bucket weights||, 1e-12) of
  the oracle's float64 decode (oracle/lik_oracle.decode_residual_tokens,
  reference.py:142-179) to fp32 rounding (1e-6 relative).
* Scores match the oracle's decode + normalise + MaxSim within the bf16 bar
  (1e-2) and the exact LDS-gather decode route within 5e-3 (the query-centroid
  term is rounded to fp16, the bucket weights to the query type), with and
  without normalisation, for nbits 2 / 4 / 8, d = 64 / 128, bf16 and fp16,
  1 to 5 queries (two queries per wavefront, a partial last group) and
  empty docs (score 0).
* retrieve: indices equal a stable sort of the scan's own score row (ties
  to the lower index), scores equal the row at those indices.
* Calls the scan cannot take (Lq > 32, residual rows not a multiple of
  16 bytes) go to maxsim_residual_varlen and give its result exactly.
* Docs split inside the scan's 32-token tiles (short and empty docs, 1 to
  128 docs per wavefront): the same bits for every split.
* Token records (LIK_TOKEN_RECORDS): each record holds the token's code and
  bitwise lik_plaid_token_norms' value (also when written in two token
  ranges), and scores from the records equal
  bitwise the scores from the separate codes and norms, on the register scan
  (two queries per wavefront with records, one without: the same arithmetic
  per query) and the LDS-staged scan (plaid_variant 5, and the residual
  widths the register scan does not take),
  with and without normalisation; the C ABI rejects a missing or misaligned
  record pointer.
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


def _index(Nd, max_ld, d, nbits, seed, cdtype, ncent=300):
    g = torch.Generator().manual_seed(seed)
    cent = torch.nn.functional.normalize(torch.randn(ncent, d, generator=g), dim=-1).to(cdtype)
    bw = torch.linspace(-0.1, 0.1, 2**nbits)
    lens = torch.randint(1, max_ld + 1, (Nd,), generator=g)
    lens[0] = 0
    lens[Nd // 2] = 0
    lens[3] = max_ld
    T = int(lens.sum())
    codes = torch.randint(0, ncent, (T,), generator=g, dtype=torch.int32)
    bcodes = np.random.default_rng(seed).integers(0, 2**nbits, (T, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    return cent, bw, codes, res, cu


@pytest.mark.parametrize("nbits,d", [(2, 128), (4, 128), (8, 128), (2, 64), (4, 64)])
@pytest.mark.parametrize("cdtype", [torch.bfloat16, torch.float16])
def test_token_norms_and_scores(nbits, d, cdtype):
    from late_interaction_kernels.plaid import ResidualIndex, maxsim_residual_varlen

    _case(f"qc nbits={nbits} d={d} {cdtype}")
    cent, bw, codes, res, cu = _index(400, 90, d, nbits, nbits * 7 + d, cdtype)
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    idx = ResidualIndex(*args)
    emb = O.decode_residual_tokens(codes.numpy(), res.numpy(), cent.double().numpy(), bw.numpy(), nbits)
    inv_ref = 1.0 / np.maximum(np.linalg.norm(emb, axis=-1), 1e-12)
    assert rel_err(idx.token_inv.cpu().numpy(), inv_ref) < 1e-6
    g = torch.Generator().manual_seed(d + nbits)
    for nq, lq in ((1, 32), (2, 32), (5, 20)):
        Q = torch.randn(nq, lq, d, generator=g).to(cdtype).cuda()
        for normalize in (True, False):
            got = idx.score(Q, normalize=normalize)
            with launch_options(plaid_variant=2):
                exact = maxsim_residual_varlen(Q, *args, normalize=normalize)
            # the split form against the exact decode route: fp16 q.c and bf16
            # bucket weights (measured below 2e-3 on these inputs)
            assert rel_err(got.cpu().numpy(), exact.cpu().numpy()) < 3e-3, (nq, normalize)
            ref = O.maxsim_residual_varlen(Q.double().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                           cent.double().numpy(), bw.numpy(), nbits, normalize=normalize)
            assert rel_err(got.cpu().numpy(), ref) < 1e-2, (nq, normalize)
            assert got[:, 0].abs().max().item() == 0.0 and got[:, 200].abs().max().item() == 0.0


def test_retrieve_and_large_table():
    """A 65,536-centroid table (the benchmark's size: 4 MB of fp16 scores per
    query), 3,000 docs of 30..300 tokens, one and two queries: top-100
    against a stable sort of the scan's own scores."""
    from late_interaction_kernels.plaid import ResidualIndex, retrieve_residual_varlen

    _case("qc retrieve 65536 centroids")
    g = torch.Generator(device="cuda").manual_seed(5)
    Nd, d, nbits, nc = 3000, 128, 2, 65536
    lens = torch.randint(30, 301, (Nd,), generator=g, device="cuda")
    cu = torch.zeros(Nd + 1, dtype=torch.int32, device="cuda")
    cu[1:] = lens.cumsum(0).to(torch.int32)
    T = int(cu[-1])
    cent = torch.nn.functional.normalize(torch.randn(nc, d, generator=g, device="cuda"), dim=-1).to(torch.bfloat16)
    codes = torch.randint(0, nc, (T,), generator=g, device="cuda", dtype=torch.int32)
    res = torch.randint(0, 256, (T, 32), generator=g, device="cuda", dtype=torch.uint8)
    bw = torch.linspace(-0.1, 0.1, 4, device="cuda")
    idx = ResidualIndex(codes, res, cu, cent, bw, nbits)
    for nq in (1, 2):
        Q = torch.nn.functional.normalize(torch.randn(nq, 32, d, generator=g, device="cuda"), dim=-1).to(torch.bfloat16)
        s, i = idx.retrieve(Q, 100)
        full = idx.score(Q)
        order = torch.sort(full, dim=1, descending=True, stable=True).indices[:, :100]
        assert torch.equal(i, order)
        assert torch.equal(s, torch.gather(full, 1, i))
        rs, ri = retrieve_residual_varlen(Q, codes, res, cu, cent, bw, nbits, 100, chunk=None)
        assert rel_err(s.cpu().numpy(), rs.cpu().numpy()) < 5e-3
        # both routes select nearly the same documents (near-ties may swap at the margin)
        for r in range(nq):
            assert len(set(i[r].tolist()) & set(ri[r].tolist())) >= 95
        dj = torch.tensor([0, 1, 1500, Nd - 1])
        spans = [(int(cu[j]), int(cu[j + 1])) for j in dj.tolist()]
        tok = torch.cat([torch.arange(a, b) for a, b in spans]).cuda()
        cs = np.concatenate([[0], np.cumsum([b - a for a, b in spans])])
        ref = O.maxsim_residual_varlen(Q.double().cpu().numpy(), codes[tok].cpu().numpy(), res[tok].cpu().numpy(), cs,
                                       cent.double().cpu().numpy(), bw.cpu().numpy(), nbits)
        assert rel_err(full[:, dj.cuda()].cpu().numpy(), ref) < 1e-2


def test_fallbacks_equal_varlen_route():
    from late_interaction_kernels.plaid import ResidualIndex, maxsim_residual_varlen

    _case("qc fallbacks")
    cent, bw, codes, res, cu = _index(50, 40, 96, 2, 3, torch.bfloat16)  # 24-byte residual rows
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    idx = ResidualIndex(*args)
    Q = torch.randn(2, 32, 96).to(torch.bfloat16).cuda()
    assert torch.equal(idx.score(Q), maxsim_residual_varlen(Q, *args))
    cent, bw, codes, res, cu = _index(50, 40, 128, 2, 4, torch.bfloat16)
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    idx = ResidualIndex(*args)
    Q = torch.randn(2, 40, 128).to(torch.bfloat16).cuda()  # Lq > 32
    assert torch.equal(idx.score(Q), maxsim_residual_varlen(Q, *args))


@pytest.mark.parametrize("nq", [1, 3])
def test_docs_split_inside_tiles(nq):
    """The scan walks each wavefront's docs as one token stream in 32-token
    tiles, so a tile can hold the end of one doc, whole short docs and the
    start of the next. Many short docs (0..40 tokens, runs of empty docs, a
    leading and a trailing empty doc) scored with 1, 3, 37 and 128 docs per
    wavefront: a doc's score is a max per column (exact in any order) summed
    in a fixed order, so every split gives the same bits; and the scores match
    the exact decode route within the split form's 5e-3."""
    from late_interaction_kernels.plaid import ResidualIndex, maxsim_residual_varlen

    _case(f"qc short docs nq={nq}")
    g = torch.Generator().manual_seed(11 + nq)
    Nd, d, nbits, ncent = 700, 128, 2, 500
    lens = torch.randint(0, 41, (Nd,), generator=g)
    lens[:3] = 0
    lens[100:140] = 0
    lens[-2:] = 0
    lens[200:260] = torch.randint(1, 4, (60,), generator=g)
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    T = int(cu[-1])
    cent = torch.nn.functional.normalize(torch.randn(ncent, d, generator=g), dim=-1).to(torch.bfloat16)
    codes = torch.randint(0, ncent, (T,), generator=g, dtype=torch.int32)
    res = torch.randint(0, 256, (T, 32), generator=g, dtype=torch.uint8)
    bw = torch.linspace(-0.1, 0.1, 4)
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    idx = ResidualIndex(*args)
    Q = torch.randn(nq, 32, d, generator=g).to(torch.bfloat16).cuda()
    for normalize in (True, False):
        with launch_options(plaid_variant=2):
            exact = maxsim_residual_varlen(Q, *args, normalize=normalize)
        empty = (lens == 0).nonzero().flatten().cuda()
        # the register-direct scan (automatic) and the LDS-staged one (variant 5)
        for variant in (0, 5):
            with launch_options(plaid_variant=variant):
                base = idx.score(Q, normalize=normalize)
            for r in (3, 37, 128):
                with launch_options(docs_per_wg=r, plaid_variant=variant):
                    got = idx.score(Q, normalize=normalize)
                assert torch.equal(got, base), (r, normalize, variant)
            assert rel_err(base.cpu().numpy(), exact.cpu().numpy()) < 5e-3, (normalize, variant)
            assert base[:, empty].abs().max().item() == 0.0


def test_table_range_falls_back():
    """Query / centroid norms whose products could leave fp16's range (the q.c
    table) take the exact route: the scores equal maxsim_residual_varlen's bits
    and the oracle's, where the scan's fp16 table would hold inf."""
    from late_interaction_kernels.plaid import ResidualIndex, maxsim_residual_varlen

    _case("qc fp16 table range")
    cent, bw, codes, res, cu = _index(60, 50, 128, 2, 9, torch.bfloat16)
    cent = (cent.float() * 300.0).to(torch.bfloat16)  # |c| = 300
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    idx = ResidualIndex(*args)
    Q = (torch.nn.functional.normalize(torch.randn(1, 32, 128), dim=-1) * 400.0).to(torch.bfloat16).cuda()
    got = idx.score(Q, normalize=False)  # |q.c| up to 1.2e5 > 65504
    assert torch.equal(got, maxsim_residual_varlen(Q, *args, normalize=False))
    ref = O.maxsim_residual_varlen(Q.double().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                   cent.double().numpy(), bw.numpy(), 2, normalize=False)
    assert np.all(np.isfinite(got.cpu().numpy())) and rel_err(got.cpu().numpy(), ref) < 1e-2
    # normalised queries keep |q.c| <= 300: the scan runs, within its bound
    got_n = idx.score(Q, normalize=True)
    ref_n = O.maxsim_residual_varlen(Q.double().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                     cent.double().numpy(), bw.numpy(), 2, normalize=True)
    assert rel_err(got_n.cpu().numpy(), ref_n) < 1e-2


def test_c_abi_empty_query_tokens():
    """lik_plaid_maxsim_qc with Q->len == 0 writes zero scores (no scan launch)."""
    import ctypes

    from late_interaction_kernels import _lib
    from late_interaction_kernels.plaid import ResidualIndex

    _case("qc C ABI Lq = 0")
    cent, bw, codes, res, cu = _index(20, 30, 128, 2, 13, torch.bfloat16)
    idx = ResidualIndex(codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    Q = torch.zeros(2, 0, 128, device="cuda", dtype=torch.bfloat16)
    out = torch.full((2, 20), 7.0, device="cuda")
    qs = _lib.seqs(Q, n=2, length=0, stride_n=128, stride_l=128)
    docs = idx._docs()
    lib = _lib.load()
    rc = lib.lik_plaid_maxsim_qc(ctypes.byref(qs), ctypes.byref(docs), idx.token_rec.data_ptr(),
                                 _lib.LIK_NORMALIZE | _lib.LIK_TOKEN_RECORDS, out.data_ptr(), out.stride(0),
                                 out.stride(1), None, 0, None, _lib.stream_of(out))
    assert rc == _lib.LIK_OK
    assert out.abs().max().item() == 0.0


def _qc_call(idx, Q, token_ptr, flags, opts=None):
    """lik_plaid_maxsim_qc through the C ABI: (return code, [Nq, Nd] scores)."""
    import ctypes

    from late_interaction_kernels import _lib

    nq, lq, _ = Q.shape
    out = torch.full((nq, idx.n_docs), float("nan"), device="cuda")
    qs = _lib.seqs(Q, n=nq, length=lq, stride_n=Q.stride(0), stride_l=Q.stride(1))
    docs = idx._docs()
    lib = _lib.load()
    nbytes = lib.lik_plaid_maxsim_qc_workspace_size(ctypes.byref(qs), ctypes.byref(docs))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    with launch_options(**(opts or {})):
        rc = lib.lik_plaid_maxsim_qc(ctypes.byref(qs), ctypes.byref(docs), token_ptr, flags, out.data_ptr(),
                                     out.stride(0), out.stride(1), ws.data_ptr(), nbytes, _lib.call_opts(),
                                     _lib.stream_of(out))
    torch.cuda.synchronize()
    return rc, out


@pytest.mark.parametrize("nbits,d", [(2, 128), (4, 64), (8, 128), (2, 64)])
def test_token_records_equal_norms_route(nbits, d):
    import ctypes

    from late_interaction_kernels import _lib
    from late_interaction_kernels.plaid import ResidualIndex

    _case(f"qc records nbits={nbits} d={d}")
    cent, bw, codes, res, cu = _index(500, 70, d, nbits, 31 + nbits + d, torch.bfloat16)
    codes[::97] = -3  # out-of-range codes decode as centroid 0 on every route
    codes[5::89] = 100000
    idx = ResidualIndex(codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), nbits)
    T = codes.numel()
    inv = torch.empty(T, device="cuda")
    lib = _lib.load()
    docs = idx._docs()
    assert lib.lik_plaid_token_norms(ctypes.byref(docs), 0, T, inv.data_ptr(), _lib.stream_of(inv)) == _lib.LIK_OK
    torch.cuda.synchronize()
    assert torch.equal(idx.token_rec[:, 0].cpu(), codes)
    assert torch.equal(idx.token_rec[:, 1].cpu(), inv.view(torch.int32).cpu())
    # records of two token ranges, written at their absolute indices, equal one call
    rec2 = torch.full_like(idx.token_rec, -7)
    half = T // 2 + 3
    for a, b in ((half, T), (0, half)):
        assert lib.lik_plaid_token_records(ctypes.byref(docs), a, b, rec2.data_ptr(), _lib.stream_of(rec2)) == 0
    torch.cuda.synchronize()
    assert torch.equal(rec2, idx.token_rec)
    g = torch.Generator().manual_seed(d * nbits)
    for nq, lq, opts in ((1, 32, {}), (1, 32, {"plaid_variant": 5}), (3, 24, {}), (3, 24, {"plaid_variant": 5}),
                         (2, 32, {"docs_per_wg": 3})):
        Q = torch.randn(nq, lq, d, generator=g).to(torch.bfloat16).cuda()
        for normalize in (True, False):
            f = _lib.LIK_NORMALIZE if normalize else 0
            rc0, base = _qc_call(idx, Q, inv.data_ptr(), f, opts)
            rc1, got = _qc_call(idx, Q, idx.token_rec.data_ptr(), f | _lib.LIK_TOKEN_RECORDS, opts)
            assert rc0 == _lib.LIK_OK and rc1 == _lib.LIK_OK
            assert torch.equal(got, base), (nq, opts, normalize)
    # the records are required with the flag, and 8-byte aligned
    Q = torch.randn(1, 32, d, generator=g).to(torch.bfloat16).cuda()
    assert _qc_call(idx, Q, None, _lib.LIK_TOKEN_RECORDS)[0] == _lib.LIK_ERR_INVALID
    assert _qc_call(idx, Q, idx.token_rec.data_ptr() + 4, _lib.LIK_TOKEN_RECORDS)[0] == _lib.LIK_ERR_UNSUPPORTED
