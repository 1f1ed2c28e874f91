"""Load a fast-plaid / ColBERTv2 on-disk PLAID index for the PLAID kernels.

Reads the files fast-plaid serialises (the reference's loader,
benchmarks/plaid/bench_fastplaid_e2e.py:75-140, reads the same ones):

* ``metadata.json`` (``nbits``, ``num_chunks``),
* ``centroids.npy`` ``[n_centroids, d]``, ``bucket_weights.npy`` ``[2**nbits]``,
* ``doclens.{i}.json`` per chunk (document lengths, concatenated in order),
* ``merged_codes.npy`` / ``merged_residuals.npy`` (flat over all tokens), or
  the per-chunk ``codes.{i}.npy`` / ``residuals.{i}.npy`` when fast-plaid
  skipped the merge.

``.npy`` files are memory-mapped with ``numpy.load`` (no pickle), clipped to
``sum(doclens)`` tokens and copied to the GPU. fast-plaid stores each code's
bits least-significant first and packs the stream most-significant-bit first
(``numpy.packbits``), which is the bit-reverse of every byte of the
little-endian layout the kernels read (``reference.py:124-139``).

``bit_order`` chooses what the kernels see:

* ``"colbert"`` (default): the residuals are converted once on the device
  with ``lik_residual_reverse_bits``, so every token decodes to the ColBERTv2
  embedding the index was built from and the scores equal ``reference.py``'s
  on those embeddings.
* ``"raw"``: the bytes are used as stored. This is what the reference's own
  end-to-end harness does (``bench_fastplaid_e2e.py:75-140`` feeds fast-plaid's
  bytes to its kernel unconverted; ``bench_decompress_maxsim.py:144-149`` notes
  the reversed layout), so scores equal that harness's, bit for bit in decode.
"""

from __future__ import annotations

import glob
import json
import os

import numpy as np
import torch

from . import _lib


def reverse_residual_bits(residuals: torch.Tensor) -> torch.Tensor:
    """Bit-reverse every byte of a uint8 GPU tensor (returns a new tensor)."""
    _lib.require_gpu(residuals)
    if residuals.dtype != torch.uint8:
        raise ValueError("residuals must be uint8")
    src = residuals.contiguous()
    out = torch.empty_like(src)
    lib = _lib.load()
    with torch.cuda.device(src.device):
        rc = lib.lik_residual_reverse_bits(src.data_ptr(), out.data_ptr(), src.numel(), _lib.stream_of(out))
    _lib.check(rc, "lik_residual_reverse_bits")
    return out


def _npy(path: str) -> np.ndarray:
    return np.load(path, mmap_mode="r", allow_pickle=False)


def load_fastplaid_index(
    index_path: str,
    *,
    device: str | torch.device = "cuda",
    centroid_dtype: torch.dtype = torch.float16,
    d: int | None = None,
    bit_order: str = "colbert",
) -> dict:
    """Read a fast-plaid index directory into the tensors
    :func:`~late_interaction_kernels.plaid.maxsim_residual_varlen` and
    :func:`~late_interaction_kernels.plaid.retrieve_residual_varlen` take.

    Returns a dict with the reference loader's keys: ``nbits``, ``centroids``,
    ``bucket_weights``, ``codes_flat`` (int32 here), ``residuals_flat`` (uint8;
    converted to the kernels' bit order unless ``bit_order="raw"``),
    ``doc_lengths``, ``cu_seqlens_d``, ``n_docs``, ``total_tokens``, ``d``.
    """
    if bit_order not in ("colbert", "raw"):
        raise ValueError(f"bit_order must be 'colbert' or 'raw'; got {bit_order!r}")
    with open(os.path.join(index_path, "metadata.json")) as f:
        metadata = json.load(f)
    nbits = int(metadata["nbits"])
    if nbits not in (2, 4, 8):
        raise ValueError(f"nbits must be 2, 4 or 8; got {nbits}")
    num_chunks = int(metadata["num_chunks"])
    centroids_np = _npy(os.path.join(index_path, "centroids.npy"))
    d = int(d or centroids_np.shape[1])
    packed_dim = (d * nbits + 7) // 8
    centroids = torch.from_numpy(np.array(centroids_np, copy=True)).to(device=device, dtype=centroid_dtype)
    bucket_weights = torch.from_numpy(np.array(_npy(os.path.join(index_path, "bucket_weights.npy")), copy=True))
    bucket_weights = bucket_weights.to(device=device, dtype=torch.float32)

    doc_lens: list[int] = []
    for i in range(num_chunks):
        with open(os.path.join(index_path, f"doclens.{i}.json")) as f:
            doc_lens.extend(int(x) for x in json.load(f))
    total = int(sum(doc_lens))

    merged_codes = os.path.join(index_path, "merged_codes.npy")
    merged_res = os.path.join(index_path, "merged_residuals.npy")
    if os.path.exists(merged_codes) and os.path.exists(merged_res):
        codes_np = [_npy(merged_codes).reshape(-1)]
        res_np = [_npy(merged_res).reshape(-1, packed_dim)]
    else:
        def _chunk_key(p: str) -> int:
            return int(os.path.basename(p).split(".")[1])

        codes_np = [_npy(p).reshape(-1) for p in sorted(glob.glob(os.path.join(index_path, "codes.*.npy")),
                                                       key=_chunk_key)]
        res_np = [_npy(p).reshape(-1, packed_dim) for p in sorted(glob.glob(os.path.join(index_path, "residuals.*.npy")),
                                                                  key=_chunk_key)]
    codes_all = np.concatenate(codes_np) if len(codes_np) > 1 else codes_np[0]
    res_all = np.concatenate(res_np) if len(res_np) > 1 else res_np[0]
    if codes_all.shape[0] < total or res_all.shape[0] < total:
        raise ValueError(f"index holds {codes_all.shape[0]} codes / {res_all.shape[0]} residual rows "
                         f"for {total} document tokens")
    codes_flat = torch.from_numpy(np.ascontiguousarray(codes_all[:total]).astype(np.int32, copy=False)).to(device)
    res_raw = torch.from_numpy(np.array(res_all[:total], dtype=np.uint8, copy=True)).to(device)
    residuals_flat = (reverse_residual_bits(res_raw) if bit_order == "colbert" else res_raw).view(total, packed_dim)

    doc_lengths = torch.tensor(doc_lens, device=device, dtype=torch.int64)
    cu = torch.zeros(len(doc_lens) + 1, dtype=torch.int32, device=device)
    cu[1:] = doc_lengths.to(torch.int32).cumsum(0)
    return {
        "nbits": nbits,
        "centroids": centroids,
        "bucket_weights": bucket_weights,
        "codes_flat": codes_flat,
        "residuals_flat": residuals_flat,
        "doc_lengths": doc_lengths,
        "cu_seqlens_d": cu,
        "n_docs": len(doc_lens),
        "total_tokens": total,
        "d": d,
    }


__all__ = ["load_fastplaid_index", "reverse_residual_bits"]
