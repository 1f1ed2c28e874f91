"""Freeze the public signatures downstreams call by keyword (reference
tests/test_public_api.py and the kwarg lists of autograd.py:356-501,
varlen.py:452-459, padded.py:216-223, retrieve.py:103-205, plaid.py:619-628,
832-843, fp8.py:35-59,234-242). CPU only: importing the package loads no GPU
code."""

import inspect

import late_interaction_kernels as lik
from late_interaction_kernels import fp8, plaid


def _params(fn):
    return list(inspect.signature(fn).parameters)


def test_maxsim_and_pairs_keyword_contract():
    for fn in (lik.maxsim, lik.maxsim_pairs):
        p = inspect.signature(fn).parameters
        assert _params(fn)[:4] == ["Q", "D", "q_mask", "d_mask"]
        assert p["normalize"].kind is inspect.Parameter.KEYWORD_ONLY and p["normalize"].default is False
        assert p["backward"].kind is inspect.Parameter.KEYWORD_ONLY and p["backward"].default is None


def test_varlen_padded_retrieve_signatures():
    assert _params(lik.maxsim_varlen) == ["Q_packed", "D_packed", "cu_seqlens_q", "cu_seqlens_d", "max_seqlen_q",
                                          "max_seqlen_d"]
    assert _params(lik.maxsim_padded) == ["queries", "documents", "query_lengths", "doc_lengths", "validate"]
    p = inspect.signature(lik.retrieve).parameters
    assert list(p)[:5] == ["Q", "D", "top_k", "q_mask", "d_mask"]
    assert p["normalize"].default is True and p["chunk"].default is None
    assert p["largest"].default is True and p["sorted"].default is True


def test_scorer_surface():
    s = lik.MaxSimScorer()
    assert s.normalize is True and s.backward == "auto" and s.mask_pad_token is None
    for m in ("forward", "score", "retrieve", "forward_with_ids"):
        assert callable(getattr(s, m))
    assert _params(s.forward) == ["Q", "D", "q_mask", "d_mask"]


def test_plaid_and_fp8_signatures():
    p = inspect.signature(plaid.maxsim_residual_varlen).parameters
    assert list(p)[:7] == ["Q", "codes_flat", "residuals_flat", "cu_seqlens_d", "centroids", "bucket_weights", "nbits"]
    assert p["max_seqlen_d"].default is None and p["normalize"].default is True
    p = inspect.signature(fp8.maxsim_inference_fp8).parameters
    assert list(p)[:2] == ["Q", "D"]
    for k in ("scale_Q", "scale_D", "q_mask", "d_mask"):
        assert p[k].kind is inspect.Parameter.KEYWORD_ONLY
    assert callable(fp8.quantize_fp8_per_tensor) and callable(fp8.quantize_fp8_per_token)
    assert isinstance(lik.__version__, str)
