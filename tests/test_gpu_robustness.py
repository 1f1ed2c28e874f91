"""GPU robustness and scorer contract (reference tests/test_robustness.py:84-280,
tests/test_retrieve.py:15-225): inference / no-grad modes, error paths, int64
cu_seqlens, tiny magnitudes, MaxSimScorer forwarding, retrieve vs an explicit
stable top-k, chunked == unchunked, per-call backward names, the one-shot
normalisation warning. Oracle: lik_oracle (reference.py)."""

import sys
import warnings

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
    return t.detach().float().cpu().numpy()


def _randn(*shape, dtype=torch.float16, seed=0, **kw):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda().requires_grad_(kw.get("grad", False))


def test_inference_mode_returns_correct_scores():
    from late_interaction_kernels import maxsim

    _case("inference_mode")
    Q, D = _randn(2, 16, 128, seed=1), _randn(4, 64, 128, seed=2)
    with torch.inference_mode():
        s = maxsim(Q, D)
    ref = O.maxsim(_np(Q), _np(D))
    assert np.abs(_np(s) - ref).max() / max(1.0, np.abs(ref).max()) < 5e-3


def test_no_grad_output_has_no_grad_fn():
    from late_interaction_kernels import maxsim

    _case("no_grad")
    Q, D = _randn(2, 8, 128, seed=3, grad=True), _randn(3, 16, 128, seed=4, grad=True)
    with torch.no_grad():
        s = maxsim(Q, D)
    assert s.grad_fn is None and not s.requires_grad


def test_error_paths():
    from late_interaction_kernels import maxsim

    _case("error paths")
    Q = _randn(2, 16, 128, seed=5)
    with pytest.raises(ValueError):
        maxsim(Q, _randn(4, 64, 256, seed=6))
    with pytest.raises(ValueError, match="same device"):
        maxsim(Q, torch.randn(4, 64, 128, dtype=torch.float16))
    with pytest.raises(ValueError, match="backward"):
        maxsim(Q, _randn(4, 8, 128, seed=7), normalize=True, backward="nope")


def test_varlen_accepts_int64_cu_seqlens():
    from late_interaction_kernels import maxsim_varlen

    _case("varlen int64 cu")
    Qp, Dp = _randn(16, 128, seed=8), _randn(100, 128, seed=9)
    cq = torch.tensor([0, 8, 16], device="cuda", dtype=torch.int64)
    cd = torch.tensor([0, 50, 100], device="cuda", dtype=torch.int64)
    out = maxsim_varlen(Qp, Dp, cq, cd)
    assert out.shape == (2, 2)
    ref = np.array([[O.maxsim(_np(Qp[a:b]), _np(Dp[c:e])) for c, e in ((0, 50), (50, 100))]
                    for a, b in ((0, 8), (8, 16))])
    assert rel_err(_np(out), ref) < 1e-2


def test_very_small_magnitudes_dont_underflow():
    from late_interaction_kernels import maxsim

    _case("small magnitudes")
    Q = torch.nn.functional.normalize(_randn(2, 16, 128, seed=10).float(), dim=-1).half()
    D = torch.nn.functional.normalize(_randn(4, 64, 128, seed=11).float(), dim=-1).half()
    fast = maxsim(Q, D)
    ref = O.maxsim(_np(Q), _np(D))
    assert np.abs(_np(fast) - ref).max() / max(1.0, np.abs(ref).max()) < 5e-3
    assert (np.abs(_np(fast)) > 0).all()


def test_scorer_forwards_bytewise_and_backward():
    from late_interaction_kernels import MaxSimScorer, maxsim

    _case("scorer forwarding")
    Q, D = _randn(3, 24, 128, seed=12), _randn(7, 96, 128, seed=13)
    assert torch.equal(MaxSimScorer(normalize=True, backward="unified")(Q, D),
                       maxsim(Q, D, normalize=True, backward="unified"))
    Qg = _randn(2, 8, 128, dtype=torch.float32, seed=14, grad=True)
    Dg = _randn(4, 16, 128, dtype=torch.float32, seed=15, grad=True)
    q_ids = torch.ones(2, 8, device="cuda", dtype=torch.long)
    q_ids[:, -2:] = 0
    d_ids = torch.ones(4, 16, device="cuda", dtype=torch.long)
    d_ids[:, -4:] = 0
    s = MaxSimScorer(normalize=True, mask_pad_token=0).forward_with_ids(Qg, Dg, q_ids, d_ids)
    assert s.shape == (2, 4)
    s.sum().backward()
    assert Qg.grad is not None and Dg.grad is not None
    assert (Dg.grad[:, -4:] == 0).all()  # pad tokens never win a max


@pytest.mark.parametrize("backward", ["auto", "unified", "lowmem"])
def test_per_call_backward_names(backward):
    from late_interaction_kernels import maxsim

    _case(f"backward={backward}")
    Q = _randn(2, 16, 64, dtype=torch.float32, seed=16, grad=True)
    D = _randn(4, 32, 64, dtype=torch.float32, seed=17, grad=True)
    maxsim(Q, D, normalize=True, backward=backward).sum().backward()
    assert Q.grad is not None and D.grad is not None


def test_retrieve_matches_stable_topk_and_chunking():
    from late_interaction_kernels import MaxSimScorer, maxsim, retrieve

    _case("retrieve vs topk")
    Q, D = _randn(4, 16, 128, seed=18), _randn(64, 32, 128, seed=19)
    s, i = retrieve(Q, D, top_k=10, normalize=True)
    ws, wi = O.topk_stable(_np(maxsim(Q, D, normalize=True)), 10)
    np.testing.assert_array_equal(i.cpu().numpy(), wi)
    np.testing.assert_array_equal(_np(s), ws)
    Q2, D2 = _randn(2, 16, 128, seed=20), _randn(100, 32, 128, seed=21)
    fs, fi = retrieve(Q2, D2, top_k=5, normalize=True)
    cs, ci = retrieve(Q2, D2, top_k=5, normalize=True, chunk=17)
    assert torch.equal(fs, cs) and torch.equal(fi, ci)
    s1, i1 = MaxSimScorer(normalize=True).retrieve(Q2, D2, top_k=5)
    assert torch.equal(s1, fs) and torch.equal(i1, fi)


def test_unnormalized_input_warns_once(monkeypatch):
    from late_interaction_kernels import autograd as ag
    from late_interaction_kernels import maxsim

    _case("norm warning")
    monkeypatch.delenv("LIK_SUPPRESS_NORM_WARN", raising=False)
    monkeypatch.setattr(ag, "_NORM_CHECKED", False)
    Q = _randn(2, 16, 64, dtype=torch.float32, seed=22) * 10.0
    D = _randn(4, 32, 64, dtype=torch.float32, seed=23)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        maxsim(Q, D, normalize=False)
        maxsim(Q, D, normalize=False)
    msgs = [str(x.message) for x in w if "late-interaction-kernels" in str(x.message)]
    assert len(msgs) == 1 and "normalize=True" in msgs[0]
