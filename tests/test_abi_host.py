"""CPU-side checks of the boundary: the C-ABI library loads and exports every
symbol include/lik.h declares (no compute calls, so no GPU is needed), the
ctypes binding mirrors the header's structs, and the Python layer validates
arguments the way the reference does (ValueError before any launch) and
refuses CPU tensors instead of falling back to a CPU path."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lik.h"


def _declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w \*]*?\b(lik_\w+)\s*\(", text, flags=re.M))


def _library():
    from late_interaction_kernels import _lib

    if not _lib.library_path().exists():
        pytest.skip("liblik_hip.so is not built (run python __graft_entry__.py build)")
    return _lib, ctypes.CDLL(str(_lib.library_path()))


def test_header_declares_the_documented_entry_points():
    decl = _declared_functions()
    assert {"lik_maxsim", "lik_maxsim_workspace_size", "lik_maxsim_pairs", "lik_plaid_maxsim",
            "lik_plaid_approx_score", "lik_topk_merge", "lik_version"} <= decl


def test_library_exports_every_declared_symbol():
    _lib, lib = _library()
    decl = _declared_functions()
    missing = sorted(s for s in decl if not hasattr(lib, s))
    assert not missing, f"declared in include/lik.h but not exported: {missing}"
    assert set(_lib.EXPORTED_SYMBOLS) == decl


def test_version_string_names_the_target():
    _lib, _ = _library()
    assert "gfx950" in _lib.version()


def test_ctypes_structs_match_header_field_order():
    from late_interaction_kernels import _lib

    text = HEADER.read_text()
    for struct, cls in (("lik_seqs_t", _lib.LikSeqs), ("lik_plaid_docs_t", _lib.LikPlaidDocs)):
        body = re.search(r"typedef struct \{([^{}]*)\}\s*" + struct, text).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = re.findall(r"(\w+)\s*;", body)
        assert [f[0] for f in cls._fields_] == names, struct


def test_invalid_arguments_are_rejected_without_a_gpu():
    # The library validates before it launches: bad descriptors come back as
    # LIK_ERR_INVALID, and an empty problem is a no-op, neither touching a device.
    _lib, lib = _library()
    _lib.load()
    bad = _lib.LikSeqs()
    bad.dim = 0
    ok = _lib.LikSeqs()
    ok.dim, ok.dtype, ok.n, ok.len = 128, _lib.LIK_BF16, 0, 0
    rc = lib.lik_maxsim(ctypes.byref(bad), ctypes.byref(ok), 0, ctypes.c_float(1.0), None, 0, 0, None, 0, None)
    assert rc == _lib.LIK_ERR_INVALID
    rc = lib.lik_maxsim(ctypes.byref(ok), ctypes.byref(ok), 0, ctypes.c_float(1.0), None, 0, 0, None, 0, None)
    assert rc == _lib.LIK_OK
    assert lib.lik_topk_merge(None, 4, 8, 8, 0, None, None, 0, 0, 2048, 1, None, None, 0, None) != _lib.LIK_OK
    # tree select: no workspace up to 4096 scores a row, two ping-pong key
    # buffers of rows * ceil(n / 4096) * k keys above
    L = _lib.load()
    assert L.lik_topk_select_workspace_size(8, 4096, 100) == 0
    assert L.lik_topk_select_workspace_size(2, 4097, 100) == 2 * 2 * 2 * 100 * 8
    assert L.lik_topk_select_workspace_size(1, 1 << 20, 100) == 2 * 256 * 100 * 8
    rc = L.lik_topk_select(1, 1, 1 << 20, 1 << 20, 0, None, None, 0, 0, 100, 1, 1, 1, 100, None, 0, None)
    assert rc == _lib.LIK_ERR_WORKSPACE
    # large-capacity class (1024 < k <= 8192): 8192-score slices
    assert L.lik_topk_select_workspace_size(2, 8192, 2000) == 0
    assert L.lik_topk_select_workspace_size(2, 100000, 2000) == 2 * 2 * 13 * 2000 * 8
    assert L.lik_topk_select_workspace_size(2, 100000, 1024) == 2 * 2 * 25 * 1024 * 8
    # k beyond the largest class, or a running list wider than k's class, is
    # rejected before any launch (dummy pointers are never dereferenced)
    rc = L.lik_topk_select(1, 1, 10000, 10000, 0, None, None, 0, 0, 8193, 1, 1, 1, 8193, None, 0, None)
    assert rc == _lib.LIK_ERR_UNSUPPORTED
    rc = L.lik_topk_select(1, 1, 100, 100, 0, 1, 1, 2000, 2000, 1000, 1, 1, 1, 1000, None, 0, None)
    assert rc == _lib.LIK_ERR_UNSUPPORTED
    rc = L.lik_topk_merge(1, 1, 8193, 8193, 0, None, None, 0, 0, 2000, 1, 1, 1, 2000, None)
    assert rc == _lib.LIK_ERR_UNSUPPORTED
    # token records: a null descriptor or an inverted range is invalid, an empty
    # range a no-op; a misaligned record array is refused before any launch
    assert L.lik_plaid_token_records(None, 0, 1, None, None) == _lib.LIK_ERR_INVALID
    docs = _lib.LikPlaidDocs()
    docs.nbits, docs.dim, docs.n_buckets, docs.bucket_weights, docs.res_stride_tok = 2, 128, 4, 8, 32
    assert L.lik_plaid_token_records(ctypes.byref(docs), 5, 4, None, None) == _lib.LIK_ERR_INVALID
    assert L.lik_plaid_token_records(ctypes.byref(docs), 4, 4, None, None) == _lib.LIK_OK
    docs.codes, docs.residuals, docs.centroids, docs.n_centroids = 16, 16, 16, 1
    assert L.lik_plaid_token_records(ctypes.byref(docs), 0, 4, 4, None) == _lib.LIK_ERR_UNSUPPORTED


def test_value_errors_match_the_reference_contract():
    from late_interaction_kernels import maxsim, maxsim_pairs

    Q = torch.randn(2, 4, 16)
    with pytest.raises(ValueError, match="embedding dim"):
        maxsim(Q, torch.randn(3, 5, 8))
    with pytest.raises(ValueError, match="backward="):
        maxsim(Q, torch.randn(3, 5, 16), backward="bogus")
    with pytest.raises(ValueError, match="D.shape\\[0\\] == Q.shape\\[0\\]"):
        maxsim(Q, torch.randn(3, 2, 5, 16))
    with pytest.raises(ValueError, match="Q.shape\\[0\\] == D.shape\\[0\\]"):
        maxsim_pairs(Q, torch.randn(3, 5, 16))


def test_cpu_tensors_are_refused_not_computed():
    from late_interaction_kernels import maxsim, maxsim_varlen

    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        maxsim(torch.randn(2, 4, 16), torch.randn(3, 5, 16))
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        maxsim_varlen(torch.randn(4, 16), torch.randn(4, 16), cu, cu)
