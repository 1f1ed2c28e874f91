"""ctypes binding of liblik_hip.so, the gfx950 HIP kernels behind every op.

The C ABI is declared in ``include/lik.h``. This module only marshals torch
tensors (device memory, strides) and the current HIP stream into those
calls; it never computes a result itself. If the library is missing or the
tensors are not on a ROCm GPU, the ops raise — there is no CPU fallback.
"""

from __future__ import annotations

import contextlib
import contextvars
import ctypes
import os
from pathlib import Path

import torch

_LIB_PATH = Path(os.environ.get("LIK_LIBRARY") or Path(__file__).resolve().parent / "_lib" / "liblik_hip.so")

LIK_OK = 0
LIK_ERR_INVALID = -1
LIK_ERR_UNSUPPORTED = -2
LIK_ERR_WORKSPACE = -3
LIK_ERR_LAUNCH = -4

LIK_BF16, LIK_F16, LIK_F32, LIK_FP8_E4M3 = 0, 1, 2, 3
LIK_NORMALIZE = 1
LIK_KD_LAYOUT = 2
LIK_NORMALIZE_Q = 4
LIK_NORMALIZE_D = 8
LIK_BIAS_16 = 16
LIK_TOKEN_RECORDS = 32


def norm_flags(norm: int) -> int:
    """API flag for a normalise bitmask (1: query tokens, 2: doc tokens)."""
    return {0: 0, 1: LIK_NORMALIZE_Q, 2: LIK_NORMALIZE_D, 3: LIK_NORMALIZE}[norm]

_ERRORS = {
    LIK_ERR_INVALID: "invalid argument",
    LIK_ERR_UNSUPPORTED: "unsupported shape/dtype",
    LIK_ERR_WORKSPACE: "workspace too small",
    LIK_ERR_LAUNCH: "kernel launch failed",
}

# Every symbol include/lik.h declares; tests check the library exports them all.
EXPORTED_SYMBOLS = (
    "lik_maxsim",
    "lik_maxsim_workspace_size",
    "lik_maxsim_argmax",
    "lik_maxsim_from_hidden",
    "lik_maxsim_from_hidden_workspace_size",
    "lik_maxsim_backward",
    "lik_maxsim_backward_workspace_size",
    "lik_maxsim_pairs",
    "lik_maxsim_pairs_argmax",
    "lik_maxsim_pairs_backward",
    "lik_maxsim_pairs_backward_workspace_size",
    "lik_plaid_maxsim",
    "lik_plaid_decode",
    "lik_plaid_approx_score",
    "lik_residual_reverse_bits",
    "lik_topk_merge",
    "lik_topk_select",
    "lik_topk_select_workspace_size",
    "lik_version",
    "lik_maxsim_ex",
    "lik_maxsim_workspace_size_ex",
    "lik_plaid_maxsim_ex",
    "lik_maxsim_noalloc",
    "lik_plaid_token_norms",
    "lik_plaid_token_records",
    "lik_plaid_maxsim_qc",
    "lik_plaid_maxsim_qc_workspace_size",
)

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class LikSeqs(ctypes.Structure):
    """Mirror of ``lik_seqs_t``."""

    _fields_ = [
        ("data", _p),
        ("dtype", _i32),
        ("dim", _i32),
        ("n", _i64),
        ("len", _i64),
        ("stride_n", _i64),
        ("stride_l", _i64),
        ("cu_seqlens", _p),
        ("lengths", _p),
        ("mask", _p),
        ("mask_stride_n", _i64),
        ("mask_stride_l", _i64),
        ("token_scale", _p),
        ("scale_stride_n", _i64),
        ("scale_stride_l", _i64),
    ]


class LikPlaidDocs(ctypes.Structure):
    """Mirror of ``lik_plaid_docs_t``."""

    _fields_ = [
        ("codes", _p),
        ("residuals", _p),
        ("cu_seqlens", _p),
        ("lengths", _p),
        ("n", _i64),
        ("max_len", _i64),
        ("codes_stride_n", _i64),
        ("res_stride_tok", _i64),
        ("centroids", _p),
        ("centroid_dtype", _i32),
        ("dim", _i32),
        ("n_centroids", _i64),
        ("cent_stride", _i64),
        ("bucket_weights", _p),
        ("n_buckets", _i32),
        ("nbits", _i32),
    ]


class LikLaunchOpts(ctypes.Structure):
    """Mirror of ``lik_launch_opts_t``."""

    _fields_ = [
        ("col_waves", _i32),
        ("col_blocks", _i32),
        ("docs_per_wg", _i32),
        ("plaid_variant", _i32),
        ("timing_start", _p),
        ("timing_stop", _p),
    ]


_lib = None


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load liblik_hip.so once; raise with build instructions if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(
            f"late_interaction_kernels: native library {_LIB_PATH} is missing. "
            "Build it with `python late-interaction-kernels_amd/build_lib.py` "
            "(hipcc, --offload-arch=gfx950)."
        )
    lib = ctypes.CDLL(str(_LIB_PATH))
    P = ctypes.POINTER
    lib.lik_maxsim.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32, ctypes.c_float, _p, _i64, _i64, _p,
                               ctypes.c_size_t, _p]
    lib.lik_maxsim.restype = ctypes.c_int
    lib.lik_maxsim_workspace_size.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32]
    lib.lik_maxsim_workspace_size.restype = ctypes.c_size_t
    lib.lik_maxsim_argmax.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32, _p, _i64, _i64, _p, _p,
                                      ctypes.c_size_t, _p]
    lib.lik_maxsim_argmax.restype = ctypes.c_int
    lib.lik_maxsim_from_hidden.argtypes = [P(LikSeqs), P(LikSeqs), _p, _i64, _p, ctypes.c_uint32, _p, _i64, _i64,
                                           _p, _p, ctypes.c_size_t, _p]
    lib.lik_maxsim_from_hidden.restype = ctypes.c_int
    lib.lik_maxsim_from_hidden_workspace_size.argtypes = [P(LikSeqs), P(LikSeqs)]
    lib.lik_maxsim_from_hidden_workspace_size.restype = ctypes.c_size_t
    lib.lik_maxsim_backward.argtypes = [_p, _i64, P(LikSeqs), P(LikSeqs), _p, ctypes.c_uint32, _p, _p, _p,
                                        ctypes.c_size_t, _p]
    lib.lik_maxsim_backward.restype = ctypes.c_int
    lib.lik_maxsim_backward_workspace_size.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32]
    lib.lik_maxsim_backward_workspace_size.restype = ctypes.c_size_t
    lib.lik_maxsim_pairs.argtypes = [P(LikSeqs), P(LikSeqs), _p, _p, _i64, ctypes.c_uint32, _p, _p]
    lib.lik_maxsim_pairs.restype = ctypes.c_int
    lib.lik_maxsim_pairs_argmax.argtypes = [P(LikSeqs), P(LikSeqs), _p, _p, _i64, ctypes.c_uint32, _p, _p, _p]
    lib.lik_maxsim_pairs_argmax.restype = ctypes.c_int
    lib.lik_maxsim_pairs_backward.argtypes = [_p, P(LikSeqs), P(LikSeqs), _p, _p, _i64, _p, ctypes.c_uint32, _p, _p,
                                              _p, ctypes.c_size_t, _p]
    lib.lik_maxsim_pairs_backward.restype = ctypes.c_int
    lib.lik_maxsim_pairs_backward_workspace_size.argtypes = [P(LikSeqs), P(LikSeqs), _i64]
    lib.lik_maxsim_pairs_backward_workspace_size.restype = ctypes.c_size_t
    lib.lik_plaid_maxsim.argtypes = [P(LikSeqs), P(LikPlaidDocs), ctypes.c_uint32, _p, _i64, _i64, _p]
    lib.lik_plaid_maxsim.restype = ctypes.c_int
    lib.lik_plaid_decode.argtypes = [P(LikPlaidDocs), _i64, _i64, ctypes.c_uint32, _i32, _p, _i64, _p]
    lib.lik_plaid_decode.restype = ctypes.c_int
    lib.lik_residual_reverse_bits.argtypes = [_p, _p, _i64, _p]
    lib.lik_residual_reverse_bits.restype = ctypes.c_int
    lib.lik_plaid_approx_score.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _p]
    lib.lik_plaid_approx_score.restype = ctypes.c_int
    lib.lik_topk_merge.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, ctypes.c_int, _p, _p,
                                   _i64, _p]
    lib.lik_topk_merge.restype = ctypes.c_int
    lib.lik_topk_select.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, ctypes.c_int, _p, _p,
                                    _i64, _p, ctypes.c_size_t, _p]
    lib.lik_topk_select.restype = ctypes.c_int
    lib.lik_topk_select_workspace_size.argtypes = [_i64, _i64, _i64]
    lib.lik_topk_select_workspace_size.restype = ctypes.c_size_t
    lib.lik_version.argtypes = []
    lib.lik_version.restype = ctypes.c_char_p
    lib.lik_maxsim_ex.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32, ctypes.c_float, _p, _i64, _i64, _p,
                                  ctypes.c_size_t, P(LikLaunchOpts), _p]
    lib.lik_maxsim_ex.restype = ctypes.c_int
    lib.lik_maxsim_workspace_size_ex.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32, P(LikLaunchOpts)]
    lib.lik_maxsim_workspace_size_ex.restype = ctypes.c_size_t
    lib.lik_plaid_maxsim_ex.argtypes = [P(LikSeqs), P(LikPlaidDocs), ctypes.c_uint32, _p, _i64, _i64,
                                        P(LikLaunchOpts), _p]
    lib.lik_plaid_maxsim_ex.restype = ctypes.c_int
    lib.lik_maxsim_noalloc.argtypes = [P(LikSeqs), P(LikSeqs), ctypes.c_uint32, ctypes.c_float, _p, _i64, _i64, _p]
    lib.lik_maxsim_noalloc.restype = ctypes.c_int
    lib.lik_plaid_token_norms.argtypes = [P(LikPlaidDocs), _i64, _i64, _p, _p]
    lib.lik_plaid_token_norms.restype = ctypes.c_int
    lib.lik_plaid_token_records.argtypes = [P(LikPlaidDocs), _i64, _i64, _p, _p]
    lib.lik_plaid_token_records.restype = ctypes.c_int
    lib.lik_plaid_maxsim_qc_workspace_size.argtypes = [P(LikSeqs), P(LikPlaidDocs)]
    lib.lik_plaid_maxsim_qc_workspace_size.restype = ctypes.c_size_t
    lib.lik_plaid_maxsim_qc.argtypes = [P(LikSeqs), P(LikPlaidDocs), _p, ctypes.c_uint32, _p, _i64, _i64, _p,
                                        ctypes.c_size_t, P(LikLaunchOpts), _p]
    lib.lik_plaid_maxsim_qc.restype = ctypes.c_int
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != LIK_OK:
        raise RuntimeError(f"{what}: {_ERRORS.get(rc, 'error')} (code {rc})")


def require_gpu(*tensors: torch.Tensor | None) -> None:
    """The engine runs on ROCm GPUs only; no CPU fallback exists."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "late_interaction_kernels (MI355X build) runs on ROCm GPU tensors only; "
                f"got a tensor on {t.device}. Move inputs to the GPU (device='cuda')."
            )
    if getattr(torch.version, "hip", None) is None:
        raise RuntimeError("late_interaction_kernels (MI355X build) needs a ROCm build of PyTorch")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


DTYPE_CODE = {
    torch.bfloat16: LIK_BF16,
    torch.float16: LIK_F16,
    torch.float32: LIK_F32,
}
if hasattr(torch, "float8_e4m3fn"):
    DTYPE_CODE[torch.float8_e4m3fn] = LIK_FP8_E4M3


def seqs(
    data: torch.Tensor,
    *,
    n: int,
    length: int,
    stride_n: int = 0,
    stride_l: int,
    cu: torch.Tensor | None = None,
    lengths: torch.Tensor | None = None,
    mask: torch.Tensor | None = None,
    mask_strides: tuple[int, int] = (0, 0),
    token_scale: torch.Tensor | None = None,
    scale_strides: tuple[int, int] = (0, 0),
) -> LikSeqs:
    s = LikSeqs()
    s.data = data.data_ptr()
    s.dtype = DTYPE_CODE[data.dtype]
    s.dim = data.shape[-1]
    s.n = n
    s.len = length
    s.stride_n = stride_n
    s.stride_l = stride_l
    s.cu_seqlens = ptr(cu)
    s.lengths = ptr(lengths)
    s.mask = ptr(mask)
    s.mask_stride_n, s.mask_stride_l = mask_strides
    s.token_scale = ptr(token_scale)
    s.scale_stride_n, s.scale_stride_l = scale_strides
    return s


def version() -> str:
    return load().lik_version().decode()


# Launch options of the scoring calls made in the current context (thread /
# asyncio task): a forced column block, docs per workgroup, the PLAID kernel
# variant, and a launch timer. The C library itself keeps no state between
# calls; these are handed to it per call as a lik_launch_opts_t.
_OPTS: contextvars.ContextVar[dict | None] = contextvars.ContextVar("lik_launch_opts", default=None)


_HIP = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime that torch already loaded (libamdhip64), for event calls."""
    global _HIP
    if _HIP is None:
        for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
            try:
                h = ctypes.CDLL(name)
                break
            except OSError:
                continue
        else:
            raise RuntimeError("libamdhip64 not found (HIP runtime)")
        h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _HIP = h
    return _HIP


class LaunchTimer:
    """Collects a pair of HIP events for the MaxSim scoring launches of every
    call made while it is active (see :func:`launch_options`). The events are
    created with hipEventCreate (a host call: nothing is queued on the
    stream); the library records them with the launches themselves."""

    def __init__(self) -> None:
        self.pairs: list[tuple[int, int]] = []

    def new_pair(self) -> tuple[int, int]:
        hip = _hip_runtime()
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        if hip.hipEventCreate(ctypes.byref(a)) != 0 or hip.hipEventCreate(ctypes.byref(b)) != 0:
            raise RuntimeError("hipEventCreate failed")
        self.pairs.append((a.value, b.value))
        return a.value, b.value

    def total_ms(self) -> tuple[float, int]:
        """Wait for the recorded launches; return (summed ms, launch count)."""
        hip = _hip_runtime()
        tot = 0.0
        ms = ctypes.c_float()
        for a, b in self.pairs:
            if hip.hipEventSynchronize(b) != 0 or hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
                raise RuntimeError("timing events were not recorded")
            tot += ms.value
        n = len(self.pairs)
        for a, b in self.pairs:
            hip.hipEventDestroy(a)
            hip.hipEventDestroy(b)
        self.pairs = []
        return tot, n


@contextlib.contextmanager
def launch_options(*, cfg: tuple[int, int] | None = None, docs_per_wg: int = 0, plaid_variant: int = 0,
                   plaid_route: str = "auto", timer: LaunchTimer | None = None):
    """Tuning / measurement options for the scoring calls inside the block.
    ``plaid_route``: "fused" or "decode" forces the PLAID route of large
    query batches (default: by query-token count)."""
    tok = _OPTS.set({"cfg": cfg, "docs_per_wg": docs_per_wg, "plaid_variant": plaid_variant,
                     "plaid_route": plaid_route, "timer": timer})
    try:
        yield
    finally:
        _OPTS.reset(tok)


def plaid_route() -> str:
    o = _OPTS.get()
    return "auto" if o is None else o["plaid_route"]


def call_opts():
    """ctypes pointer to this call's ``lik_launch_opts_t``, or None (defaults)."""
    o = _OPTS.get()
    if o is None:
        return None
    s = LikLaunchOpts()
    if o["cfg"]:
        s.col_waves, s.col_blocks = o["cfg"]
    s.docs_per_wg = o["docs_per_wg"]
    s.plaid_variant = o["plaid_variant"]
    if o["timer"] is not None:
        s.timing_start, s.timing_stop = o["timer"].new_pair()
    return ctypes.pointer(s)


def _elem_align(dtype: torch.dtype) -> int:
    """Elements per 16-byte chunk: the kernels need rows of whole chunks."""
    return 16 // torch.empty((), dtype=dtype).element_size()


def prepare_tokens(x: torch.Tensor) -> torch.Tensor:
    """Return ``x`` with a contiguous last dim padded (with zeros) to a multiple
    of 16 bytes, rows 16-byte aligned. Zero padding changes no dot product and
    no norm, so results are unaffected."""
    align = _elem_align(x.dtype)
    d = x.shape[-1]
    pad = (-d) % align
    if pad:
        if x.element_size() == 1:  # fp8: pad the raw bytes (0x00 == +0.0)
            x = torch.nn.functional.pad(x.contiguous().view(torch.uint8), (0, pad)).view(x.dtype)
        else:
            x = torch.nn.functional.pad(x, (0, pad))
    if x.stride(-1) != 1:
        x = x.contiguous()
    ok = x.data_ptr() % 16 == 0 and all((s * x.element_size()) % 16 == 0 for s in x.stride()[:-1])
    if not ok:
        x = x.contiguous()
        if x.data_ptr() % 16 != 0:
            y = torch.empty_like(x)
            y.copy_(x)
            x = y
    return x


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)

