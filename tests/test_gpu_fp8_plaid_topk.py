"""GPU parity: fp8 MaxSim, PLAID decode+MaxSim, fused top-k merge, approx score.

fp8 tolerance 3e-2 against the fp32 oracle on the original (unquantised)
inputs and 2e-3 against the oracle on the exact dequantised values the kernel
sees; PLAID 1e-2 (bf16 compute); top-k indices bit-exact against a stable
sort (score, then lower index) of the GPU's own scores.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err
from late_interaction_kernels._lib import launch_options

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("Nq,Lq,Nd,Ld", [(4, 24, 16, 1030), (3, 32, 10, 77), (1, 32, 5, 64)])
def test_fp8_per_tensor(Nq, Lq, Nd, Ld):
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_tensor

    _case(f"fp8 {Nq},{Lq},{Nd},{Ld}")
    g = torch.Generator().manual_seed(Ld)
    Q = torch.nn.functional.normalize(torch.randn(Nq, Lq, 128, generator=g), dim=-1)
    D = torch.nn.functional.normalize(torch.randn(Nd, Ld, 128, generator=g), dim=-1)
    Qf, sq = quantize_fp8_per_tensor(Q.cuda())
    Df, sd = quantize_fp8_per_tensor(D.cuda())
    got = _np(maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd))
    ref = O.maxsim(Q.numpy(), D.numpy())
    assert rel_err(got, ref) < 3e-2
    deq = O.maxsim(_np(Qf) * sq.item(), _np(Df) * sd.item())
    assert rel_err(got, deq) < 2e-3


@pytest.mark.parametrize("d,Lq", [(128, 24), (128, 32), (64, 30), (128, 1000)])
def test_fp8_wide_column_groups(d, Lq):
    """Calls that fill a 768-column group run the fp8 4 x 6 configuration (two
    workgroups per CU); prefix masks, masks with holes (the second, masked
    launch) and empty docs, checked against the dequantised oracle and, bit
    for bit, against the 4 x 4 configuration (launch_options forces it; the per-query
    column sums are in the same order)."""
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_tensor

    _case(f"fp8 4x6 d={d} Lq={Lq}")
    g = torch.Generator().manual_seed(d + Lq)
    Nq, Nd, Ld = 70, 40, 100
    Q = torch.nn.functional.normalize(torch.randn(Nq, Lq, d, generator=g), dim=-1)
    D = torch.nn.functional.normalize(torch.randn(Nd, Ld, d, generator=g), dim=-1)
    dm = torch.arange(Ld)[None] < torch.randint(0, Ld + 1, (Nd,), generator=g)[:, None]
    dm[3, 10:20] = False  # holes: this doc goes through the masked launch
    dm[5] = False
    Qf, sq = quantize_fp8_per_tensor(Q.cuda())
    Df, sd = quantize_fp8_per_tensor(D.cuda())
    got = maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd, d_mask=dm.cuda())
    deq = O.maxsim(_np(Qf) * sq.item(), _np(Df) * sd.item(), None, dm.numpy())
    assert rel_err(_np(got), deq) < 2e-3
    assert _np(got)[:, 5].max() == 0.0
    with launch_options(cfg=(4, 6)):
        forced = maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd, d_mask=dm.cuda())
    assert torch.equal(forced, got)
    with launch_options(cfg=(4, 4)):
        narrow = maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd, d_mask=dm.cuda())
    assert rel_err(_np(narrow), _np(got)) < 1e-5


def test_fp8_per_token_and_masks():
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_token

    _case("fp8 per-token")
    g = torch.Generator().manual_seed(8)
    Q = torch.randn(3, 32, 128, generator=g)
    D = torch.randn(7, 90, 128, generator=g)
    qm = torch.rand(3, 32, generator=g) > 0.2
    dm = torch.rand(7, 90, generator=g) > 0.2
    Qf, sq = quantize_fp8_per_token(Q.cuda())
    Df, sd = quantize_fp8_per_token(D.cuda())
    got = _np(maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd, q_mask=qm.cuda(), d_mask=dm.cuda()))
    Qd = _np(Qf) * sq.cpu().numpy()[..., None]
    Dd = _np(Df) * sd.cpu().numpy()[..., None]
    assert rel_err(got, O.maxsim(Qd, Dd, qm.numpy(), dm.numpy())) < 2e-3
    assert rel_err(got, O.maxsim(Q.numpy(), D.numpy(), qm.numpy(), dm.numpy())) < 3e-2


@pytest.mark.parametrize("q_tok,d_tok", [(True, False), (False, True)])
def test_fp8_mixed_scales(q_tok, d_tok):
    """One side per-token, the other per-tensor (a 0-d device scale read by
    the kernel): against the oracle on the dequantised values."""
    from late_interaction_kernels.fp8 import (maxsim_inference_fp8, quantize_fp8_per_tensor,
                                              quantize_fp8_per_token)

    _case(f"fp8 mixed q_tok={q_tok} d_tok={d_tok}")
    g = torch.Generator().manual_seed(12)
    Q = torch.randn(5, 24, 128, generator=g)
    D = torch.randn(9, 70, 128, generator=g)
    Qf, sq = (quantize_fp8_per_token if q_tok else quantize_fp8_per_tensor)(Q.cuda())
    Df, sd = (quantize_fp8_per_token if d_tok else quantize_fp8_per_tensor)(D.cuda())
    got = _np(maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd))
    Qd = _np(Qf) * (sq.cpu().numpy()[..., None] if q_tok else sq.item())
    Dd = _np(Df) * (sd.cpu().numpy()[..., None] if d_tok else sd.item())
    assert rel_err(got, O.maxsim(Qd, Dd)) < 2e-3


def test_fp8_graph_capture_replay():
    """Per-tensor scales are read on the device, so an fp8 call can be
    captured: every replay equals the eager result, also after the scale
    tensors change in place (the graph reads them at replay time)."""
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_tensor

    _case("fp8 graph")
    g = torch.Generator().manual_seed(13)
    Qf, sq = quantize_fp8_per_tensor(torch.randn(8, 32, 128, generator=g).cuda())
    Df, sd = quantize_fp8_per_tensor(torch.randn(64, 100, 128, generator=g).cuda())
    eager = maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd)  # warm the allocator
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = maxsim_inference_fp8(Qf[:2], Df[:5], scale_Q=sq, scale_D=sd)  # eager work between replays
        torch.cuda.synchronize()
    sd.mul_(2.0)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd))
    assert rel_err(_np(out), 2 * _np(eager)) < 1e-6


def test_fp8_per_token_after_other_kernels():
    """Regression: the per-row-scale epilogue must not read stale LDS on its
    first iteration. Interleave other MaxSim launches (which leave negative
    values in LDS) with one-doc-per-workgroup per-token fp8 calls."""
    from late_interaction_kernels import maxsim
    from late_interaction_kernels.fp8 import maxsim_inference_fp8, quantize_fp8_per_token

    _case("fp8 per-token interleaved")
    g = torch.Generator().manual_seed(9)
    Q = torch.randn(2, 32, 128, generator=g)
    D = torch.randn(5, 40, 128, generator=g)
    Qf, sq = quantize_fp8_per_token(Q.cuda())
    Df, sd = quantize_fp8_per_token(D.cuda())
    ref = O.maxsim(_np(Qf) * sq.cpu().numpy()[..., None], _np(Df) * sd.cpu().numpy()[..., None])
    other_q = -torch.rand(64, 32, 128, device="cuda").to(torch.bfloat16)
    other_d = torch.rand(300, 64, 128, device="cuda").to(torch.bfloat16)
    for _ in range(4):
        maxsim(other_q, other_d, normalize=True)
        got = _np(maxsim_inference_fp8(Qf, Df, scale_Q=sq, scale_D=sd))
        assert rel_err(got, ref) < 2e-3


def _index(Nd, max_Ld, d, n_cent, nbits, seed, cdtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    cent = (torch.randn(n_cent, d, generator=g) * 0.3)
    bw = torch.linspace(-0.1, 0.1, 2**nbits)
    lens = torch.randint(max_Ld // 2, max_Ld + 1, (Nd,), generator=g)
    lens[0] = 0
    codes = torch.randint(0, n_cent, (Nd, max_Ld), generator=g)
    bcodes = np.random.default_rng(seed).integers(0, 2**nbits, (Nd, max_Ld, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    return cent.to(cdtype), bw, lens, codes, res


@pytest.mark.parametrize("nbits", [2, 4, 8])
@pytest.mark.parametrize("cdtype", [torch.float32, torch.bfloat16, torch.float16])
def test_plaid_padded(nbits, cdtype):
    from late_interaction_kernels.plaid import maxsim_residual

    _case(f"plaid padded {nbits} {cdtype}")
    cent, bw, lens, codes, res = _index(12, 70, 128, 64, nbits, nbits, cdtype)
    g = torch.Generator().manual_seed(1)
    Q = torch.randn(5, 32, 128, generator=g).to(torch.bfloat16)
    got = maxsim_residual(Q.cuda(), codes.cuda(), res.cuda(), lens.cuda(), cent.cuda(), bw.cuda(), nbits)
    ref = O.maxsim_residual(_np(Q), codes.numpy(), res.numpy(), lens.numpy(), _np(cent), bw.numpy(), nbits)
    gn = _np(got)
    assert np.all(gn[:, 0] == 0)
    assert rel_err(gn, ref) < 1e-2


@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("Nq,Lq", [(1, 32), (40, 32), (2, 600)])
def test_plaid_varlen(nbits, Nq, Lq):
    from late_interaction_kernels.plaid import maxsim_residual, maxsim_residual_varlen

    _case(f"plaid varlen {nbits} {Nq} {Lq}")
    cent, bw, lens, codes, res = _index(30, 90, 128, 256, nbits, 100 + nbits)
    keep = torch.arange(90)[None] < lens[:, None]
    codes_flat = codes[keep]
    res_flat = res[keep]
    cu = torch.zeros(31, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    g = torch.Generator().manual_seed(Nq)
    Q = torch.randn(Nq, Lq, 128, generator=g).to(torch.bfloat16)
    got = maxsim_residual_varlen(Q.cuda(), codes_flat.cuda(), res_flat.cuda(), cu.cuda(), cent.cuda(), bw.cuda(),
                                 nbits)
    ref = O.maxsim_residual_varlen(_np(Q), codes_flat.numpy(), res_flat.numpy(), cu.numpy(), _np(cent),
                                   bw.numpy(), nbits)
    assert rel_err(_np(got), ref) < 1e-2
    pad = maxsim_residual(Q.cuda(), codes.cuda(), res.cuda(), lens.cuda(), cent.cuda(), bw.cuda(), nbits)
    assert torch.allclose(got, pad, atol=1e-4)


def test_plaid_identity_buckets_equals_dense():
    from late_interaction_kernels import maxsim
    from late_interaction_kernels.plaid import maxsim_residual

    _case("plaid identity")
    g = torch.Generator().manual_seed(3)
    cent = torch.randn(16, 64, generator=g).to(torch.bfloat16)
    codes = torch.randint(0, 16, (3, 10), generator=g)
    res = torch.zeros(3, 10, 64, dtype=torch.uint8)
    Q = torch.randn(2, 6, 64, generator=g).to(torch.bfloat16)
    args = (Q.cuda(), codes.cuda(), res.cuda(), torch.full((3,), 10).cuda(), cent.cuda(), torch.zeros(256).cuda(), 8)
    # no normalisation: decoded tokens are exactly the bf16 centroids -> same products
    got = maxsim_residual(*args, normalize=False)
    dense = maxsim(Q.cuda(), cent[codes].cuda(), normalize=False)
    assert torch.allclose(got, dense, atol=1e-5)
    # normalised: PLAID rounds the fp32-normalised token to bf16, the dense path
    # scales the dot product instead -> equal to bf16 accuracy
    got = maxsim_residual(*args, normalize=True)
    dense = maxsim(Q.cuda(), cent[codes].cuda(), normalize=True)
    assert rel_err(_np(got), _np(dense)) < 1e-2


def test_plaid_empty_corpus():
    from late_interaction_kernels.plaid import maxsim_residual_varlen

    _case("plaid empty")
    Q = torch.randn(2, 8, 128, device="cuda", dtype=torch.bfloat16)
    out = maxsim_residual_varlen(Q, torch.zeros(0, dtype=torch.int32, device="cuda"),
                                 torch.zeros(0, 32, dtype=torch.uint8, device="cuda"),
                                 torch.zeros(1, dtype=torch.int32, device="cuda"),
                                 torch.randn(4, 128, device="cuda"), torch.zeros(4, device="cuda"), 2)
    assert out.shape == (2, 0)


@pytest.mark.parametrize("largest", [True, False])
@pytest.mark.parametrize("n,k,chunk", [(100, 10, None), (5000, 100, 4096), (9000, 1000, 2048), (37, 37, 5),
                                       (300, 7, 1), (300000, 100, None), (70000, 1000, None), (20001, 1, None),
                                       (50000, 64, 20000), (4097, 4097 - 4096, 4096),
                                       # large-capacity class (1024 < k <= 8192) and the k > 8192 sort
                                       (20000, 3000, 4096), (30000, 1025, 10000), (100000, 8192, None),
                                       (12000, 5000, 6000), (9000, 9000, None)])
def test_topk_merge_bit_exact(largest, n, k, chunk):
    from late_interaction_kernels.topk import topk_update

    _case(f"topk {largest} {n} {k} {chunk}")
    g = torch.Generator().manual_seed(n + k)
    s = (torch.randint(0, 50, (6, n), generator=g).float() / 7.0)  # heavy ties
    s[0, 3] = float("inf")
    s[1, :] = 0.0
    sc = s.cuda()
    run_s = run_i = None
    cs = n if chunk is None else chunk
    for st in range(0, n, cs):
        run_s, run_i = topk_update(sc[:, st:st + cs], st, run_s, run_i, k, largest)
    ws, wi = O.topk_stable(s.numpy(), k, largest=largest)
    np.testing.assert_array_equal(run_i.cpu().numpy(), wi)
    np.testing.assert_array_equal(run_s.cpu().numpy(), ws)


@pytest.mark.parametrize("largest", [True, False])
@pytest.mark.parametrize("n,k,chunk", [(5000, 100, 512), (3000, 7, 1), (9000, 1000, 2048), (4100, 64, 4096)])
def test_topk_merge_chunks_in_reverse(largest, n, k, chunk):
    """Chunks merged last-first: once the running list holds k entries, a
    chunk's scores that tie the list's worst one carry lower doc indices and
    must win the tie (the merge keeps only chunk keys above the list's worst
    key); the result is still the stable top-k of the whole row."""
    from late_interaction_kernels.topk import topk_update

    _case(f"topk reverse {largest} {n} {k} {chunk}")
    g = torch.Generator().manual_seed(n * 3 + k)
    s = (torch.randint(0, 20, (5, n), generator=g).float() / 3.0)  # heavy ties
    s[2, :] = 1.0
    sc = s.cuda()
    run_s = run_i = None
    for st in reversed(range(0, n, chunk)):
        run_s, run_i = topk_update(sc[:, st:st + chunk], st, run_s, run_i, k, largest)
    ws, wi = O.topk_stable(s.numpy(), k, largest=largest)
    np.testing.assert_array_equal(run_i.cpu().numpy(), wi)
    np.testing.assert_array_equal(run_s.cpu().numpy(), ws)


def test_topk_merge_entry_point():
    """lik_topk_merge keeps its one-workgroup-per-row contract (n <= 4096)."""
    from late_interaction_kernels import _lib

    _case("topk merge entry point")
    lib = _lib.load()
    g = torch.Generator().manual_seed(5)
    prev = torch.sort(torch.randint(0, 20, (3, 50), generator=g).float(), dim=-1, descending=True).values
    prev_i = torch.arange(10000, 10050).expand(3, 50).contiguous()
    s = torch.randint(0, 20, (3, 4096), generator=g).float()
    out_s = torch.empty(3, 80, device="cuda")
    out_i = torch.empty(3, 80, device="cuda", dtype=torch.int64)
    ps, pi, sc = prev.cuda(), prev_i.cuda(), s.cuda()
    rc = lib.lik_topk_merge(sc.data_ptr(), 3, 4096, 4096, 0, ps.data_ptr(), pi.data_ptr(), 50, 50, 80, 1,
                            out_s.data_ptr(), out_i.data_ptr(), 80, _lib.stream_of(out_s))
    assert rc == _lib.LIK_OK
    rc = lib.lik_topk_merge(sc.data_ptr(), 3, 4097, 4096, 0, None, None, 0, 0, 80, 1,
                            out_s.data_ptr(), out_i.data_ptr(), 80, _lib.stream_of(out_s))
    assert rc == _lib.LIK_ERR_UNSUPPORTED
    torch.cuda.synchronize()
    all_s = torch.cat([prev, s], -1).numpy()
    all_i = torch.cat([prev_i, torch.arange(4096).expand(3, 4096)], -1).numpy()
    # stable order on (score desc, index asc)
    for r in range(3):
        order = np.lexsort((all_i[r], -all_s[r]))[:80]
        np.testing.assert_array_equal(out_i[r].cpu().numpy(), all_i[r][order])
        np.testing.assert_array_equal(out_s[r].cpu().numpy(), all_s[r][order])


@pytest.mark.parametrize("largest", [1, 0])
def test_topk_merge_full_unsorted_list_aliased(largest):
    """lik_topk_merge with a full running list (prev_k == k) given in no
    particular order and aliased to the output: the merge keeps only chunk
    scores that beat the list's worst entry (its minimum key, wherever it
    sits), and writes over the list it read. Heavy ties between the list and
    the chunk; list indices lie both below and above the chunk's."""
    from late_interaction_kernels import _lib

    _case(f"topk merge full unsorted aliased largest={largest}")
    lib = _lib.load()
    g = torch.Generator().manual_seed(17 + largest)
    k, n = 80, 4096
    prev = torch.randint(0, 12, (4, k), generator=g).float()
    # list indices below and above the chunk's 1000..5095, never inside it
    pool = torch.cat([torch.arange(0, 1000), torch.arange(6000, 30000)])
    prev_i = pool[torch.randperm(pool.numel(), generator=g)[: 4 * k]].reshape(4, k).to(torch.int64)
    s = torch.randint(0, 12, (4, n), generator=g).float()
    s[3] = 5.0  # a row of one value
    base = 1000  # chunk indices 1000..5095 overlap the list's range
    ps, pi, sc = prev.cuda(), prev_i.cuda(), s.cuda()
    all_s = torch.cat([prev, s], -1).numpy()
    all_i = torch.cat([prev_i, torch.arange(base, base + n).expand(4, n)], -1).numpy()
    rc = lib.lik_topk_merge(sc.data_ptr(), 4, n, n, base, ps.data_ptr(), pi.data_ptr(), k, k, k, largest,
                            ps.data_ptr(), pi.data_ptr(), k, _lib.stream_of(ps))
    assert rc == _lib.LIK_OK
    torch.cuda.synchronize()
    sign = -1 if largest else 1
    for r in range(4):
        rs, ri = all_s[r], all_i[r]
        order = np.lexsort((ri, sign * rs))[:k]
        np.testing.assert_array_equal(pi[r].cpu().numpy(), ri[order])
        np.testing.assert_array_equal(ps[r].cpu().numpy(), rs[order])


def test_retrieve_matches_oracle_on_gpu_scores():
    from late_interaction_kernels import maxsim, retrieve

    _case("retrieve")
    g = torch.Generator().manual_seed(12)
    Q = torch.randn(7, 32, 128, generator=g).to(torch.bfloat16).cuda()
    D = torch.randn(900, 40, 128, generator=g).to(torch.bfloat16).cuda()
    full = maxsim(Q, D, normalize=True)
    ws, wi = O.topk_stable(full.cpu().numpy(), 50)
    for chunk in (None, 128, 899, 4096):
        s, i = retrieve(Q, D, top_k=50, chunk=chunk)
        np.testing.assert_array_equal(i.cpu().numpy(), wi)
        np.testing.assert_array_equal(s.cpu().numpy(), ws)


def test_plaid_retrieve():
    from late_interaction_kernels.plaid import maxsim_residual_varlen, retrieve_residual_varlen

    _case("plaid retrieve")
    cent, bw, lens, codes, res = _index(700, 40, 128, 128, 2, 77)
    keep = torch.arange(40)[None] < lens[:, None]
    cu = torch.zeros(701, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    args = (codes[keep].cuda(), res[keep].cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    Q = torch.randn(3, 32, 128).to(torch.bfloat16).cuda()
    full = maxsim_residual_varlen(Q, *args)
    ws, wi = O.topk_stable(full.cpu().numpy(), 100)
    s, i = retrieve_residual_varlen(Q, *args, 100, chunk=256)
    np.testing.assert_array_equal(i.cpu().numpy(), wi)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


@pytest.mark.parametrize("chunk", [1, 7, 256, 1000])
@pytest.mark.parametrize("piece_tokens", [0, 300])
def test_plaid_retrieve_decode_route(chunk, piece_tokens, monkeypatch):
    """The decode-once route (forced): each chunk is decoded in pieces of at
    most _DECODE_TOKENS tokens into one reused buffer, scored by the tile
    kernel, and merged into the running top-k. Chunks of 1, 7, 256 docs and
    one chunk for the whole corpus; piece_tokens = 300 splits chunks into
    several decode pieces (a doc longer than that is a piece of its own);
    docs 0 and 20..27 are empty, so one 7-doc chunk holds no token. The
    result equals a stable top-k of the full score matrix bit for bit."""
    from late_interaction_kernels import plaid
    from late_interaction_kernels.plaid import maxsim_residual_varlen, retrieve_residual_varlen

    _case(f"plaid retrieve decode route chunk={chunk} piece_tokens={piece_tokens}")
    if piece_tokens:
        monkeypatch.setattr(plaid, "_DECODE_TOKENS", piece_tokens)
    cent, bw, lens, codes, res = _index(700, 40, 128, 128, 2, 78)
    lens[20:28] = 0
    keep = torch.arange(40)[None] < lens[:, None]
    cu = torch.zeros(701, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    args = (codes[keep].cuda(), res[keep].cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    g = torch.Generator().manual_seed(9)
    Q = torch.randn(5, 32, 128, generator=g).to(torch.bfloat16).cuda()
    with launch_options(plaid_route="decode"):
        full = maxsim_residual_varlen(Q, *args)
        s, i = retrieve_residual_varlen(Q, *args, 100, chunk=chunk)
    ws, wi = O.topk_stable(full.cpu().numpy(), 100)
    np.testing.assert_array_equal(i.cpu().numpy(), wi)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


def test_plaid_approx_score_gpu():
    from late_interaction_kernels.plaid import plaid_approx_score

    _case("approx")
    g = torch.Generator().manual_seed(6)
    qcs = torch.randn(64, 32, generator=g)
    codes = torch.randint(-3, 70, (20, 50), generator=g)
    lens = torch.randint(0, 51, (20,), generator=g)
    lens[3] = 0
    got = plaid_approx_score(qcs.cuda(), codes.cuda(), lens.cuda())
    ref = O.plaid_approx_score(qcs.numpy(), codes.numpy(), lens.numpy())
    assert got[3].item() == 0.0
    np.testing.assert_allclose(_np(got), ref, rtol=1e-6, atol=1e-5)
