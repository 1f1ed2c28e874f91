"""GPU parity of the fused projection head (lik_maxsim_from_hidden, lik_head.hip)
behind maxsim_from_hidden (reference fused_head.py:262-332) on 16-bit inputs.

Reference of the same op in plain torch fp32: D = H @ W^T + b in fp32, rows
normalised (x / max(||x||, 1e-12)) and rounded to the input dtype (the
reference's fused kernel rounds the normalised tile before its MaxSim dot,
fused_head.py:150-162), scores in fp64 over those rounded rows.

* Scores within rel 2e-3 (the projection's fp32 accumulation order differs,
  which moves a few rounded elements by one 16-bit ulp).
* The saved argmax equals the reference's (lowest index among the maxima)
  wherever the best and second-best scores differ by more than 2e-2.
* maxsim_from_hidden without grad runs the fused kernel (same bits); its
  training route (projection GEMM + argmax forward + winner-row backward)
  gives gradients of Q, H, W, b matching fp32 autograd at that route's
  winners (rel 2e-2, bf16 inputs and gradients).
* Shapes around the kernel's edges: d_model 768 / 384 / 200 (a partial 64-dim
  unit) / 8; d_out 128 / 96 / 64 / 40 / 32; docs of 1, 255, 256, 257, 300
  tokens (the 256-token workgroup chunks), masks with holes, an all-masked
  doc (score 0, argmax -1), 1..256 query tokens; f16 as well as bf16.
* Bitwise equal on a second run (fixed reduction order).
* Outside the kernel's shapes (more than 256 query tokens, fp32) the call
  projects first and gives the reference's scores.
"""

import ctypes
import sys

import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _np(t):
    return t.detach().double().cpu().numpy()


def _inputs(Nq, Lq, Nd, Ld, dmod, dout, dtype, seed, bias=True, holes=True):
    g = torch.Generator().manual_seed(seed)
    Q = torch.nn.functional.normalize(torch.randn(Nq, Lq, dout, generator=g), dim=-1).to(dtype)
    H = torch.randn(Nd, Ld, dmod, generator=g).to(dtype)
    W = (torch.randn(dout, dmod, generator=g) * dmod**-0.5).to(dtype)
    b = (torch.randn(dout, generator=g) / 4).to(dtype) if bias else None
    lens = torch.randint(1, Ld + 1, (Nd,), generator=g)
    lens[0] = Ld
    dm = torch.arange(Ld)[None] < lens[:, None]
    if holes:
        dm &= torch.rand(Nd, Ld, generator=g) > 0.2
    if Nd > 2:
        dm[2] = False  # all masked
    return Q, H, W, b, dm


def _proj_ref(H, W, b, normalize, dtype):
    D = H.float() @ W.float().t()
    if b is not None:
        D = D + b.float()
    if normalize:
        D = D / D.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    return D.to(dtype)


def _ref(Q, H, W, b, dm, normalize):
    """fp64 scores, argmax and the best-minus-second gap over the rounded rows."""
    D = _proj_ref(H, W, b, normalize, Q.dtype).double()
    S = torch.einsum("isd,jtd->ijst", Q.double(), D)
    S = S.masked_fill(~dm[None, :, None, :], float("-inf"))
    top = S.topk(min(2, S.shape[-1]), dim=-1)
    m = top.values[..., 0]
    am = torch.where(torch.isfinite(m), top.indices[..., 0], torch.full_like(top.indices[..., 0], -1))
    gap = (top.values[..., 0] - top.values[..., 1]) if S.shape[-1] > 1 else torch.full_like(m, float("inf"))
    m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    return m.sum(-1), am, gap


CASES = [
    # Nq, Lq, Nd, Ld, d_model, d_out
    (1, 32, 12, 300, 768, 128),
    (4, 32, 9, 257, 384, 96),
    (2, 16, 7, 256, 200, 64),
    (3, 5, 6, 255, 8, 40),
    (8, 32, 5, 65, 128, 32),
    (1, 1, 4, 1, 64, 128),
    # more (doc, 256-token chunk) items than CUs: the persistent kernel's
    # workgroups take several items each (its load pipeline runs across items;
    # d_model 64 is one unit per item, so it runs two items ahead)
    (1, 32, 300, 600, 384, 128),
    (2, 16, 700, 100, 64, 64),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("normalize", [True, False])
def test_fused_forward_and_argmax(case, dtype, normalize):
    from late_interaction_kernels._core import from_hidden_forward

    Nq, Lq, Nd, Ld, dmod, dout = case
    _case(f"fused head fwd {case} {dtype} norm={normalize}")
    Q, H, W, b, dm = _inputs(Nq, Lq, Nd, Ld, dmod, dout, dtype, sum(case) + normalize)
    got = from_hidden_forward(Q.cuda(), H.cuda(), W.cuda(), b.cuda(), dm.cuda(), normalize=normalize, want_argmax=True)
    assert got is not None, "the fused kernel must take this shape"
    s, am = got
    rs, ram, gap = _ref(Q, H, W, b, dm, normalize)
    assert rel_err(_np(s), rs.numpy()) < 2e-3
    am = am.view(Nq, Nd, Lq).cpu()
    sep = (gap > 2e-2) | (ram < 0)
    assert torch.equal(am[sep], ram[sep])
    if Nd > 2:
        assert s[:, 2].abs().max().item() == 0.0 and bool((am[:, 2] == -1).all())
    again = from_hidden_forward(Q.cuda(), H.cuda(), W.cuda(), b.cuda(), dm.cuda(), normalize=normalize,
                                want_argmax=True)
    assert torch.equal(again[0], got[0]) and torch.equal(again[1], got[1])


@pytest.mark.parametrize("case", CASES)
def test_fused_forward_without_mask(case):
    """No doc mask and no lengths: the persistent kernel computes the token
    validity words from the padded length itself (no validity pre-pass), so
    every token before Ld counts, including a last 256-token chunk that is
    only partly inside the docs (Ld 300, 257, 255, 65, 1, 600, 100)."""
    from late_interaction_kernels._core import from_hidden_forward

    Nq, Lq, Nd, Ld, dmod, dout = case
    _case(f"fused head fwd no mask {case}")
    Q, H, W, b, _ = _inputs(Nq, Lq, Nd, Ld, dmod, dout, torch.bfloat16, sum(case) + 7, holes=False)
    got = from_hidden_forward(Q.cuda(), H.cuda(), W.cuda(), b.cuda(), None, normalize=True, want_argmax=True)
    assert got is not None, "the fused kernel must take this shape"
    s, am = got
    rs, ram, gap = _ref(Q, H, W, b, torch.ones(Nd, Ld, dtype=torch.bool), True)
    assert rel_err(_np(s), rs.numpy()) < 2e-3
    am = am.view(Nq, Nd, Lq).cpu()
    sep = (gap > 2e-2) | (ram < 0)
    assert torch.equal(am[sep], ram[sep])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 32, 12, 300, 768, 128), (3, 20, 9, 130, 384, 96)])
def test_bias_in_input_dtype(shape, dtype):
    """A bias in the inputs' 16-bit dtype goes to the kernel as is
    (LIK_BIAS_16, widened in the kernel); an fp32 bias goes as fp32. The fp32
    copy of a 16-bit bias holds the same values, so both calls give the same
    bits. Unknown flag bits are still rejected."""
    from late_interaction_kernels import _lib
    from late_interaction_kernels._core import from_hidden_forward

    Nq, Lq, Nd, Ld, dmod, dout = shape
    _case(f"fused head bias dtype {shape} {dtype}")
    Q, H, W, b, dm = _inputs(Nq, Lq, Nd, Ld, dmod, dout, dtype, sum(shape) + 3)
    args = (Q.cuda(), H.cuda(), W.cuda())
    s16, a16 = from_hidden_forward(*args, b.cuda(), dm.cuda(), normalize=True, want_argmax=True)
    s32, a32 = from_hidden_forward(*args, b.float().cuda(), dm.cuda(), normalize=True, want_argmax=True)
    assert torch.equal(s16, s32) and torch.equal(a16, a32)
    rs, _, _ = _ref(Q, H, W, b, dm, True)
    assert rel_err(_np(s16), rs.numpy()) < 2e-3
    assert _lib.LIK_BIAS_16 == 16


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("shape", [(2, 32, 10, 300, 768, 128), (1, 32, 40, 70, 384, 96)])
def test_public_routes(shape, bias):
    """maxsim_from_hidden without grad is the fused kernel (the same bits as
    the entry point; 2-D Q squeezed); with grad (the training route: projection
    GEMM, argmax forward, winner-row backward) scores and gradients of Q, H, W,
    b match fp32 autograd taken at that route's winners, rel 5e-3 / 2e-2."""
    from late_interaction_kernels._core import dense_maxsim_train, from_hidden_forward
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    Nq, Lq, Nd, Ld, dmod, dout = shape
    _case(f"fused head routes {shape} bias={bias}")
    Q, H, W, b, dm = _inputs(Nq, Lq, Nd, Ld, dmod, dout, torch.bfloat16, 11 + bias, bias=bias)
    Qc, Hc, Wc, dmc = Q.cuda(), H.cuda(), W.cuda(), dm.cuda()
    bc = b.cuda() if bias else None
    with torch.no_grad():
        s_inf = maxsim_from_hidden(Qc, Hc, Wc, bc, dmc, True)
        s_one = maxsim_from_hidden(Qc[0], Hc, Wc, bc, dmc, True)
    assert torch.equal(s_inf, from_hidden_forward(Qc, Hc, Wc, bc, dmc, normalize=True, want_argmax=False)[0])
    assert s_one.shape == (Nd,) and torch.equal(s_one, s_inf[0])

    leaves = [t.cuda().requires_grad_() for t in (Q, H, W) + ((b,) if bias else ())]
    s = maxsim_from_hidden(leaves[0], leaves[1], leaves[2], leaves[3] if bias else None, dmc, True)
    G = torch.randn(Nq, Nd, generator=torch.Generator().manual_seed(1)).cuda()
    (s * G).sum().backward()
    # the training route's winners: the argmax forward on the projected docs
    D = torch.nn.functional.linear(Hc, Wc, bc)
    am = dense_maxsim_train(Qc, D, None, dmc, norm=2, kd=False)[1].view(Nq, Nd, Lq).long()
    refs = [t.float().cuda().requires_grad_() for t in (Q, H, W) + ((b,) if bias else ())]
    Df = torch.nn.functional.normalize(torch.nn.functional.linear(refs[1], refs[2], refs[3] if bias else None), dim=-1)
    jj = torch.arange(Nd, device="cuda").view(1, Nd, 1).expand(Nq, Nd, Lq)
    Dw = Df[jj, am.clamp_min(0)]  # [Nq, Nd, Lq, d_out]
    sr = ((refs[0][:, None] * Dw).sum(-1) * (am >= 0)).sum(-1)
    (sr * G).sum().backward()
    assert rel_err(_np(s), _np(sr)) < 5e-3
    assert rel_err(_np(s_inf), _np(sr)) < 5e-3
    # training (bf16 projection, then normalise) against inference (fp32
    # projection, bias and normalise, one rounding): the rounding of the
    # projection is the only difference
    assert rel_err(_np(s), _np(s_inf)) < 1e-2
    for a, r in zip(leaves, refs):
        assert a.grad.dtype == a.dtype
        assert rel_err(_np(a.grad), _np(r.grad)) < 2e-2
    assert s[:, 2].abs().max().item() == 0.0


def test_permuted_hidden_states_grad():
    """H_d dense but permuted (a transposed view) requiring grad: grad_H has
    H_d's shape and matches the contiguous input's gradient (within bf16: the
    projection GEMM accumulates in another order on the permuted layout, so a
    near-tied winner may move: all but a few rows agree)."""
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    _case("fused head permuted H grad")
    Q, H, W, b, dm = _inputs(2, 32, 6, 40, 128, 64, torch.bfloat16, 31)
    Hp = H.permute(1, 0, 2).contiguous().permute(1, 0, 2)  # same values, [Ld, Nd, d_model] storage
    assert not Hp.is_contiguous()
    grads = []
    for Hx in (H, Hp):
        h = Hx.cuda().requires_grad_()
        s = maxsim_from_hidden(Q.cuda(), h, W.cuda(), b.cuda(), dm.cuda(), True)
        s.sum().backward()
        grads.append(h.grad)
    assert grads[1].shape == H.shape
    a, r = _np(grads[1]).reshape(-1, H.shape[-1]), _np(grads[0]).reshape(-1, H.shape[-1])
    row_ok = np.abs(a - r).max(axis=1) <= 2e-2 * np.abs(r).max()
    assert row_ok.mean() > 0.97


def test_outside_the_kernel_projects_first():
    from late_interaction_kernels._core import from_hidden_forward
    from late_interaction_kernels.fused_head import maxsim_from_hidden

    _case("fused head unsupported shapes")
    Q, H, W, b, dm = _inputs(9, 32, 5, 40, 128, 128, torch.bfloat16, 21)  # 288 query tokens
    Qc, Hc, Wc, bc, dmc = Q.cuda(), H.cuda(), W.cuda(), b.cuda(), dm.cuda()
    assert from_hidden_forward(Qc, Hc, Wc, bc, dmc, normalize=True, want_argmax=False) is None
    with torch.no_grad():
        s = maxsim_from_hidden(Qc, Hc, Wc, bc, dmc, True)
    rs, _, _ = _ref(Q, H, W, b, dm, True)
    assert rel_err(_np(s), rs.numpy()) < 1e-2
    assert from_hidden_forward(Qc.float(), Hc.float(), Wc.float(), bc, dmc, normalize=True, want_argmax=False) is None


def test_c_abi_checks():
    """Through the C ABI: unsupported shapes are refused before any launch,
    a missing workspace is reported, and an empty query batch succeeds."""
    from late_interaction_kernels import _lib

    _case("fused head C ABI")
    lib = _lib.load()
    Q = torch.zeros(1, 32, 160, device="cuda", dtype=torch.bfloat16)
    H = torch.zeros(2, 10, 64, device="cuda", dtype=torch.bfloat16)
    W = torch.zeros(160, 64, device="cuda", dtype=torch.bfloat16)
    out = torch.zeros(1, 2, device="cuda")
    qs = _lib.seqs(Q, n=1, length=32, stride_n=Q.stride(0), stride_l=Q.stride(1))
    hs = _lib.seqs(H, n=2, length=10, stride_n=H.stride(0), stride_l=H.stride(1))
    rc = lib.lik_maxsim_from_hidden(ctypes.byref(qs), ctypes.byref(hs), W.data_ptr(), 64, None, 0, out.data_ptr(), 2, 1,
                                    None, None, 0, _lib.stream_of(out))
    assert rc == _lib.LIK_ERR_UNSUPPORTED  # d_out 160 > 128
    Q2 = torch.zeros(1, 32, 128, device="cuda", dtype=torch.bfloat16)
    W2 = torch.zeros(128, 64, device="cuda", dtype=torch.bfloat16)
    qs2 = _lib.seqs(Q2, n=1, length=32, stride_n=Q2.stride(0), stride_l=Q2.stride(1))
    assert lib.lik_maxsim_from_hidden_workspace_size(ctypes.byref(qs2), ctypes.byref(hs)) > 0
    rc = lib.lik_maxsim_from_hidden(ctypes.byref(qs2), ctypes.byref(hs), W2.data_ptr(), 64, None, 0, out.data_ptr(), 2,
                                    1, None, None, 0, _lib.stream_of(out))
    assert rc == _lib.LIK_ERR_WORKSPACE
    rc = lib.lik_maxsim_from_hidden(ctypes.byref(qs2), ctypes.byref(hs), W2.data_ptr(), 64, None, 4, out.data_ptr(), 2,
                                    1, None, None, 0, _lib.stream_of(out))
    assert rc == _lib.LIK_ERR_INVALID  # only LIK_NORMALIZE_D and LIK_BIAS_16
    qs0 = _lib.seqs(Q2, n=0, length=32, stride_n=Q2.stride(0), stride_l=Q2.stride(1))
    rc = lib.lik_maxsim_from_hidden(ctypes.byref(qs0), ctypes.byref(hs), W2.data_ptr(), 64, None, 0, out.data_ptr(), 2,
                                    1, None, None, 0, _lib.stream_of(out))
    assert rc == _lib.LIK_OK
