"""GPU parity: dense / KD / pairs / padded / varlen MaxSim vs the CPU oracle.

Every test calls the public API, which goes through the C ABI of
liblik_hip.so. Tolerances (rel_err = max|a-b| / max|ref|): fp32 inputs 1e-4,
bf16 and fp16 1e-2.
"""

import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2, torch.float16: 1e-2}
GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _rand(shape, dtype, gen, normalize=False):
    x = torch.randn(*shape, generator=gen)
    if normalize:
        x = torch.nn.functional.normalize(x, dim=-1)
    return x.to(dtype).cuda()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(
    "Nq,Lq,Nd,Ld,d",
    [
        (1, 32, 1, 32, 128),
        (2, 32, 3, 300, 128),
        (4, 24, 9, 77, 128),
        (17, 32, 40, 180, 128),
        (3, 7, 5, 33, 64),
        (2, 40, 6, 65, 96),
        (5, 32, 8, 100, 256),
        (2, 16, 3, 20, 48),
        (40, 32, 70, 64, 128),  # > 512 query tokens: several column groups
    ],
)
def test_dense_parity(dtype, Nq, Lq, Nd, Ld, d):
    from late_interaction_kernels import maxsim

    _case(f"dense {dtype} {Nq},{Lq},{Nd},{Ld},{d}")
    g = torch.Generator().manual_seed(Nq * 1000 + Ld)
    Q = _rand((Nq, Lq, d), dtype, g)
    D = _rand((Nd, Ld, d), dtype, g)
    got = maxsim(Q, D, normalize=True)
    torch.cuda.synchronize()
    ref = O.maxsim(_np(Q), _np(D), normalize=True)
    assert rel_err(_np(got), ref) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("normalize", [False, True])
def test_dense_masks(dtype, normalize):
    from late_interaction_kernels import maxsim

    _case(f"masks {dtype} norm={normalize}")
    g = torch.Generator().manual_seed(11)
    Nq, Lq, Nd, Ld, d = 6, 32, 10, 150, 128
    Q = _rand((Nq, Lq, d), dtype, g)
    D = _rand((Nd, Ld, d), dtype, g)
    qm = torch.rand(Nq, Lq, generator=g) > 0.3
    dm = torch.rand(Nd, Ld, generator=g) > 0.3
    dm[2] = False  # fully masked doc
    qm[1] = False  # fully masked query
    dm[4, 40:] = False  # prefix mask (extent 40)
    got = maxsim(Q, D, qm.cuda(), dm.cuda(), normalize=normalize)
    ref = O.maxsim(_np(Q), _np(D), qm.numpy(), dm.numpy(), normalize=normalize)
    g_np = _np(got)
    assert np.all(g_np[:, 2] == 0) and np.all(g_np[1] == 0)
    assert rel_err(g_np, ref) < TOL[dtype]


@pytest.mark.parametrize("case", GOLD["maxsim"], ids=lambda c: c["name"])
def test_known_answers_gpu(case):
    from late_interaction_kernels import maxsim

    _case(f"known {case['name']}")
    Q = torch.tensor(case["Q"], dtype=torch.float32).cuda()
    D = torch.tensor(case["D"], dtype=torch.float32).cuda()
    got = maxsim(Q, D, torch.tensor(case["q_mask"]).bool().cuda(), torch.tensor(case["d_mask"]).bool().cuda(),
                 normalize=case["normalize"])
    assert rel_err(_np(got), np.array(case["expected"])) < 1e-4


def test_squeeze_rules():
    from late_interaction_kernels import maxsim

    _case("squeeze")
    q = torch.randn(5, 64).cuda()
    d = torch.randn(7, 64).cuda()
    s = maxsim(q, d, normalize=True)
    assert s.shape == ()
    assert maxsim(q, d[None], normalize=True).shape == (1,)
    assert maxsim(q[None], d, normalize=True).shape == (1,)
    assert abs(s.item() - float(O.maxsim(_np(q), _np(d), normalize=True))) < 1e-3


@pytest.mark.parametrize("Lq", [513, 700, 1030])
def test_long_query_chunking(Lq):
    from late_interaction_kernels import maxsim

    _case(f"longq {Lq}")
    g = torch.Generator().manual_seed(Lq)
    Q = _rand((3, Lq, 128), torch.bfloat16, g)
    D = _rand((5, 90, 128), torch.bfloat16, g)
    qm = (torch.rand(3, Lq, generator=g) > 0.2)
    got = maxsim(Q, D, qm.cuda(), normalize=True)
    ref = O.maxsim(_np(Q), _np(D), qm.numpy(), normalize=True)
    assert rel_err(_np(got), ref) < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Lq,K", [(32, 8), (24, 3), (200, 2), (600, 2)])
def test_kd_layout(dtype, Lq, K):
    from late_interaction_kernels import maxsim

    _case(f"kd {dtype} Lq={Lq} K={K}")
    g = torch.Generator().manual_seed(K * 7 + Lq)
    Nq, Ld, d = 5, 75, 128
    Q = _rand((Nq, Lq, d), dtype, g)
    D = _rand((Nq, K, Ld, d), dtype, g)
    qm = torch.rand(Nq, Lq, generator=g) > 0.2
    dm = torch.rand(Nq, K, Ld, generator=g) > 0.25
    got = maxsim(Q, D, qm.cuda(), dm.cuda(), normalize=True)
    ref = O.maxsim_kd(_np(Q), _np(D), qm.numpy(), dm.numpy(), normalize=True)
    assert got.shape == (Nq, K)
    assert rel_err(_np(got), ref) < TOL[dtype]


def test_maxsim_pairs():
    from late_interaction_kernels import maxsim_pairs

    _case("pairs")
    g = torch.Generator().manual_seed(3)
    Q = _rand((6, 32, 128), torch.bfloat16, g)
    D = _rand((6, 50, 128), torch.bfloat16, g)
    got = maxsim_pairs(Q, D, normalize=True)
    ref = np.array([O.maxsim(_np(Q[i]), _np(D[i]), normalize=True) for i in range(6)])
    assert got.shape == (6,)
    assert rel_err(_np(got), ref) < 1e-2


def _pack(lens, d, dtype, g):
    data = _rand((sum(lens), d), dtype, g, normalize=True)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.tensor(lens, dtype=torch.int32).cumsum(0)
    return data, cu.cuda()


@pytest.mark.parametrize(
    "q_lens,d_lens,d",
    [
        ([32, 32], [64, 128, 32, 200], 128),
        ([5, 10, 1], [50, 60, 1], 128),
        ([32], [300] * 4, 128),
        ([16, 48, 32, 8], [128, 256, 512, 32, 200], 256),
        ([5, 0, 3], [8, 0, 16], 128),  # empty query and empty doc
        ([32] * 20, [16, 2048, 33, 700, 1, 64], 128),
    ],
)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_varlen(q_lens, d_lens, d, dtype):
    from late_interaction_kernels import maxsim_varlen

    _case(f"varlen {dtype} {q_lens[:3]} {d_lens[:3]} {d}")
    g = torch.Generator().manual_seed(len(q_lens) * 100 + len(d_lens))
    Qp, cu_q = _pack(q_lens, d, dtype, g)
    Dp, cu_d = _pack(d_lens, d, dtype, g)
    got = maxsim_varlen(Qp, Dp, cu_q, cu_d)
    ref = O.maxsim_varlen(_np(Qp), _np(Dp), cu_q.cpu().numpy(), cu_d.cpu().numpy())
    assert rel_err(_np(got), ref) < 1e-2
    gn = _np(got)
    for i, L in enumerate(q_lens):
        if L == 0:
            assert np.all(gn[i] == 0)
    for j, L in enumerate(d_lens):
        if L == 0:
            assert np.all(gn[:, j] == 0)


def test_varlen_matches_padded():
    from late_interaction_kernels import maxsim, maxsim_varlen

    _case("varlen==padded")
    Nq, Nd, Lq, Ld, d = 4, 8, 32, 256, 128
    Q = torch.randn(Nq, Lq, d, device="cuda", dtype=torch.float16)
    D = torch.randn(Nd, Ld, d, device="cuda", dtype=torch.float16)
    cu_q = torch.arange(0, (Nq + 1) * Lq, Lq, device="cuda", dtype=torch.int32)
    cu_d = torch.arange(0, (Nd + 1) * Ld, Ld, device="cuda", dtype=torch.int32)
    a = maxsim_varlen(Q.reshape(-1, d), D.reshape(-1, d), cu_q, cu_d)
    b = maxsim(Q, D, normalize=False)
    assert torch.allclose(a, b, atol=1e-3)


def test_maxsim_padded_and_pack():
    from late_interaction_kernels import maxsim_padded
    from late_interaction_kernels.padded import pack_padded
    from late_interaction_kernels.score_pairs import score_pairs_packed

    _case("padded")
    g = torch.Generator().manual_seed(5)
    B, C, Lq, Ld, d = 4, 5, 32, 64, 128
    Q = _rand((B, Lq, d), torch.bfloat16, g, normalize=True)
    D = _rand((B, C, Ld, d), torch.bfloat16, g, normalize=True)
    ql = torch.randint(1, Lq + 1, (B,), generator=g)
    dl = torch.randint(1, Ld + 1, (B, C), generator=g)
    dl[1, 2] = 0  # empty candidate
    got = maxsim_padded(Q, D, ql.cuda(), dl.cuda())
    ref = O.maxsim_padded(_np(Q), _np(D), ql.numpy(), dl.numpy())
    assert rel_err(_np(got), ref) < 1e-2
    dl[1, 2] = 3
    pb = pack_padded(Q, D, ql.cuda(), dl.cuda())
    flat = score_pairs_packed(pb.Q_packed, pb.D_packed, pb.cu_seqlens_q, pb.cu_seqlens_d, pb.pair_q_idx,
                              pb.pair_d_idx, max_seqlen_q=pb.max_seqlen_q, max_seqlen_d=pb.max_seqlen_d)
    ref2 = O.maxsim_padded(_np(Q), _np(D), ql.numpy(), dl.numpy())
    assert rel_err(_np(flat.view(B, C)), ref2) < 1e-2


def test_score_pairs_arbitrary():
    from late_interaction_kernels.score_pairs import score_pairs_packed

    _case("pairs-arbitrary")
    g = torch.Generator().manual_seed(9)
    q_lens, d_lens = [7, 32, 0, 19], [40, 3, 100, 0, 65]
    Qp, cu_q = _pack(q_lens, 128, torch.bfloat16, g)
    Dp, cu_d = _pack(d_lens, 128, torch.bfloat16, g)
    pq = torch.tensor([0, 1, 1, 2, 3, 3, 0], dtype=torch.int32)
    pd = torch.tensor([4, 0, 2, 1, 3, 1, 2], dtype=torch.int32)
    got = score_pairs_packed(Qp, Dp, cu_q, cu_d, pq.cuda(), pd.cuda())
    ref = O.maxsim_pairs(_np(Qp), _np(Dp), cu_q.cpu().numpy(), cu_d.cpu().numpy(), pq.numpy(), pd.numpy())
    assert rel_err(_np(got), ref) < 1e-2


def test_determinism_bitwise():
    from late_interaction_kernels import maxsim

    _case("determinism")
    g = torch.Generator().manual_seed(21)
    Q = _rand((64, 32, 128), torch.bfloat16, g)
    D = _rand((300, 120, 128), torch.bfloat16, g)
    dm = (torch.rand(300, 120, generator=g) > 0.1).cuda()
    a = maxsim(Q, D, d_mask=dm, normalize=True)
    b = maxsim(Q, D, d_mask=dm, normalize=True)
    assert torch.equal(a, b)


def test_non_contiguous_inputs():
    from late_interaction_kernels import maxsim

    _case("noncontig")
    g = torch.Generator().manual_seed(2)
    Qb = _rand((3, 32, 256), torch.bfloat16, g)
    Db = _rand((40, 5, 128), torch.bfloat16, g)
    Q = Qb[:, :, ::2]  # stride-2 last dim
    D = Db.transpose(0, 1)  # [5, 40, 128] non-contiguous
    got = maxsim(Q, D, normalize=True)
    ref = O.maxsim(_np(Q), _np(D), normalize=True)
    assert rel_err(_np(got), ref) < 1e-2


@pytest.mark.parametrize("form", ["dense_normalize", "mask_with_holes", "kd_mask", "varlen"])
def test_cuda_graph_capture_replay(form):
    """Captured calls replay to the eager result, with eager work (other
    shapes) between replays: the dense call, a doc mask with holes (mask
    summary pre-pass, then the mask-free and the masked launch), the KD
    layout with a mask (streaming kernel) and packed docs (with
    max_seqlen_q / max_seqlen_d given: without them the call reads the longest
    sequence back to the host, as the reference does)."""
    from late_interaction_kernels import maxsim, maxsim_varlen

    _case(f"graph {form}")
    g = torch.Generator().manual_seed(4)
    if form == "varlen":
        cu_q = torch.tensor([0, 32, 64, 96], dtype=torch.int32).cuda()
        lens = torch.randint(1, 200, (50,), generator=g)
        cu_d = torch.zeros(51, dtype=torch.int32)
        cu_d[1:] = torch.cumsum(lens, 0)
        cu_d = cu_d.cuda()
        Qp = _rand((96, 128), torch.bfloat16, g)
        Dp = _rand((int(cu_d[-1]), 128), torch.bfloat16, g)
        # with the bounds given there is no host sync (the cover check is an async assert)
        call = lambda: maxsim_varlen(Qp, Dp, cu_q, cu_d, max_seqlen_q=32, max_seqlen_d=200)
    elif form == "kd_mask":
        Q = _rand((8, 32, 128), torch.bfloat16, g)
        D = _rand((8, 12, 90, 128), torch.bfloat16, g)
        dm = (torch.arange(90)[None, None] < torch.randint(1, 91, (8, 12), generator=g)[..., None]).cuda()
        call = lambda: maxsim(Q, D, d_mask=dm)
    else:
        Q = _rand((8, 32, 128), torch.bfloat16, g)
        D = _rand((64, 100, 128), torch.bfloat16, g)
        if form == "mask_with_holes":
            dm = (torch.arange(100)[None] < torch.randint(1, 101, (64,), generator=g)[:, None])
            dm[::5, 3] = False
            dm = dm.cuda()
            call = lambda: maxsim(Q, D, d_mask=dm)
        else:
            call = lambda: maxsim(Q, D, normalize=True)
    eager = call()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()  # warm the allocator
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = maxsim(_rand((2, 16, 128), torch.bfloat16, g), _rand((5, 40, 128), torch.bfloat16, g))
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_doc_prenormalise_matches_in_kernel(dtype):
    """Several query groups (20 queries) normalise the docs once ahead of the
    tile kernel; one group (16 queries) normalises them inside it. Same
    rounding, same MFMA order, same per-query summation order (a query's
    place in its group is the same): the first 16 rows are bitwise equal."""
    from late_interaction_kernels import maxsim

    _case(f"prenorm {dtype}")
    g = torch.Generator().manual_seed(31)
    Q = (torch.randn(20, 32, 128, generator=g) * 3).to(dtype).cuda()
    D = (torch.randn(37, 75, 128, generator=g) * 0.2).to(dtype).cuda()
    dm = (torch.arange(75)[None] < torch.randint(1, 76, (37,), generator=g)[:, None]).cuda()
    allq = maxsim(Q, D, d_mask=dm, normalize=True)
    first = maxsim(Q[:16], D, d_mask=dm, normalize=True)
    assert torch.equal(allq[:16], first)
    ref = O.maxsim(_np(Q), _np(D), None, dm.cpu().numpy(), normalize=True)
    assert rel_err(_np(allq), ref) < TOL[dtype]
