"""GPU parity of the PLAID decode kernel and the decode-once scoring route.

* lik_plaid_decode without normalisation is compared bit for bit with the
  oracle's decode (oracle/lik_oracle.decode_residual_tokens, reference.py:
  124-139,158-167) on inputs whose decoded values are exactly representable
  in the output type (integer centroids, quarter-step bucket weights), which
  pins the bit order, the field width and the bucket lookup exactly.
* With normalisation the rows match the oracle to bf16 rounding (2^-8).
* The decode-once route and the fused decode+MaxSim kernel produce bitwise
  identical scores (same decoded rows, same MFMA order), for both
  maxsim_residual_varlen (incl. multi-chunk decode) and retrieve.
"""

import sys

import numpy as np
import pytest
import torch

import lik_oracle as O
from conftest import rel_err

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _exact_index(T, d, n_cent, nbits, seed, cdtype):
    g = torch.Generator().manual_seed(seed)
    cent = torch.randint(-8, 9, (n_cent, d), generator=g).to(cdtype)
    nb = 2**nbits
    bw = (torch.arange(nb, dtype=torch.float32) - nb // 2) / 4.0  # exact quarter steps
    codes = torch.randint(0, n_cent, (T,), generator=g, dtype=torch.int32)
    bcodes = np.random.default_rng(seed).integers(0, nb, (T, d))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    return cent, bw, codes, res


@pytest.mark.parametrize("nbits", [2, 4, 8])
@pytest.mark.parametrize("cdtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 96])
def test_decode_bit_exact(nbits, cdtype, d):
    from late_interaction_kernels.plaid import decode_residual_tokens

    _case(f"decode exact nbits={nbits} {cdtype} d={d}")
    cent, bw, codes, res = _exact_index(1000, d, 50, nbits, nbits * 7 + d, cdtype)
    got = decode_residual_tokens(codes.cuda(), res.cuda(), cent.cuda(), bw.cuda(), nbits, normalize=False)
    ref = O.decode_residual_tokens(codes.numpy(), res.numpy(), cent.float().numpy(), bw.numpy(), nbits)
    assert got.dtype == torch.bfloat16 and got.shape == (1000, d)
    np.testing.assert_array_equal(got.float().cpu().numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_decode_normalised(out_dtype):
    from late_interaction_kernels.plaid import decode_residual_tokens

    _case(f"decode normalised {out_dtype}")
    g = torch.Generator().manual_seed(5)
    cent = torch.randn(300, 128, generator=g)
    bw = torch.linspace(-0.1, 0.1, 4)
    codes = torch.randint(0, 300, (4000,), generator=g, dtype=torch.int32)
    res = torch.randint(0, 256, (4000, 32), generator=g, dtype=torch.uint8)
    got = decode_residual_tokens(codes.cuda(), res.cuda(), cent.cuda(), bw.cuda(), 2, dtype=out_dtype)
    ref = O.decode_residual_tokens(codes.numpy(), res.numpy(), cent.numpy(), bw.numpy(), 2)
    ref = ref / np.linalg.norm(ref, axis=-1, keepdims=True)
    err = np.abs(got.float().cpu().numpy() - ref).max()
    assert err < (2**-8 if out_dtype == torch.bfloat16 else 2**-11)


def _varlen_index(Nd, max_Ld, nbits, seed):
    g = torch.Generator().manual_seed(seed)
    cent = torch.randn(256, 128, generator=g) * 0.3
    bw = torch.linspace(-0.1, 0.1, 2**nbits)
    lens = torch.randint(1, max_Ld + 1, (Nd,), generator=g)
    lens[2] = 0
    lens[5] = max_Ld
    codes = torch.randint(0, 256, (int(lens.sum()),), generator=g, dtype=torch.int32)
    bcodes = np.random.default_rng(seed).integers(0, 2**nbits, (int(lens.sum()), 128))
    res = torch.from_numpy(O.pack_residuals(bcodes, nbits))
    cu = torch.zeros(Nd + 1, dtype=torch.int32)
    cu[1:] = lens.cumsum(0).to(torch.int32)
    return cent, bw, codes, res, cu


@pytest.mark.parametrize("budget", [1 << 20, 150])
def test_decode_route_matches_fused_bitwise(monkeypatch, budget):
    from late_interaction_kernels import plaid

    _case(f"routes budget={budget}")
    cent, bw, codes, res, cu = _varlen_index(60, 200, 2, 11)
    g = torch.Generator().manual_seed(2)
    Q = torch.randn(9, 32, 128, generator=g).to(torch.bfloat16).cuda()
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    monkeypatch.setattr(plaid, "_DECODE_ROUTE_MIN_QTOK", 1 << 30)
    fused = plaid.maxsim_residual_varlen(Q, *args)
    monkeypatch.setattr(plaid, "_DECODE_ROUTE_MIN_QTOK", 1)
    monkeypatch.setattr(plaid, "_DECODE_TOKENS", budget)
    routed = plaid.maxsim_residual_varlen(Q, *args)
    assert torch.equal(fused, routed)
    assert fused[:, 2].abs().max().item() == 0.0  # empty doc
    ref = O.maxsim_residual_varlen(Q.float().cpu().numpy(), codes.numpy(), res.numpy(), cu.numpy(),
                                   cent.numpy(), bw.numpy(), 2)
    assert rel_err(routed.cpu().numpy(), ref) < 1e-2


@pytest.mark.parametrize("budget,chunk", [(1 << 20, 256), (300, 256), (700, None)])
def test_retrieve_decode_route(monkeypatch, budget, chunk):
    from late_interaction_kernels import plaid

    _case(f"retrieve decode route budget={budget} chunk={chunk}")
    cent, bw, codes, res, cu = _varlen_index(900, 60, 2, 21)
    Q = torch.randn(70, 32, 128).to(torch.bfloat16).cuda()  # 2240 query tokens: decode route
    args = (codes.cuda(), res.cuda(), cu.cuda(), cent.cuda(), bw.cuda(), 2)
    assert plaid._use_decode_route(70, 32)
    monkeypatch.setattr(plaid, "_DECODE_TOKENS", budget)
    s, i = plaid.retrieve_residual_varlen(Q, *args, 50, chunk=chunk)
    monkeypatch.setattr(plaid, "_DECODE_ROUTE_MIN_QTOK", 1 << 30)
    full = plaid.maxsim_residual_varlen(Q, *args)  # fused route
    ws, wi = O.topk_stable(full.cpu().numpy(), 50)
    np.testing.assert_array_equal(i.cpu().numpy(), wi)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


def _write_fastplaid_index(path, nbits, merged, seed=3, exact=False):
    """A small index directory in fast-plaid's on-disk format (ColBERTv2 bit
    packing). exact: centroids and bucket weights on a 1/16 grid, so every
    decoded value c + w is exact in bf16."""
    import json
    import os

    rng = np.random.default_rng(seed)
    d, n_cent = 128, 40
    doclens = [rng.integers(1, 30, 25).tolist(), rng.integers(1, 30, 17).tolist()]
    cent = rng.standard_normal((n_cent, d)).astype(np.float32)
    bw = np.linspace(-0.2, 0.2, 2**nbits).astype(np.float32)
    if exact:
        cent = (rng.integers(-16, 16, (n_cent, d)) / 16).astype(np.float32)
        bw = ((np.arange(2**nbits) - 2 ** (nbits - 1)) / 16).astype(np.float32)
    codes = [rng.integers(0, n_cent, sum(dl)).astype(np.int64) for dl in doclens]
    bcodes = [rng.integers(0, 2**nbits, (sum(dl), d)) for dl in doclens]
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "metadata.json"), "w") as f:
        json.dump({"nbits": nbits, "num_chunks": 2}, f)
    np.save(os.path.join(path, "centroids.npy"), cent)
    np.save(os.path.join(path, "bucket_weights.npy"), bw)
    for i, dl in enumerate(doclens):
        with open(os.path.join(path, f"doclens.{i}.json"), "w") as f:
            json.dump(dl, f)
    packed = [O.pack_residuals_colbert(b, nbits) for b in bcodes]
    if merged:
        np.save(os.path.join(path, "merged_codes.npy"), np.concatenate(codes + [np.zeros(3, np.int64)]))
        np.save(os.path.join(path, "merged_residuals.npy"), np.concatenate(packed + [np.zeros((3, d * nbits // 8), np.uint8)]))
    else:
        for i in range(2):
            np.save(os.path.join(path, f"codes.{i}.npy"), codes[i])
            np.save(os.path.join(path, f"residuals.{i}.npy"), packed[i])
    return sum(doclens, []), cent, bw, np.concatenate(codes), np.concatenate(bcodes)


@pytest.mark.parametrize("nbits", [2, 4])
@pytest.mark.parametrize("merged", [False, True])
def test_fastplaid_index_loader(tmp_path, nbits, merged):
    from late_interaction_kernels.plaid import maxsim_residual_varlen
    from late_interaction_kernels.plaid_index import load_fastplaid_index

    _case(f"fast-plaid loader nbits={nbits} merged={merged}")
    doclens, cent, bw, codes, bcodes = _write_fastplaid_index(str(tmp_path), nbits, merged)
    idx = load_fastplaid_index(str(tmp_path), centroid_dtype=torch.float32)
    T = sum(doclens)
    assert idx["n_docs"] == len(doclens) and idx["total_tokens"] == T and idx["nbits"] == nbits
    np.testing.assert_array_equal(idx["codes_flat"].cpu().numpy(), codes)
    # residuals converted to the kernels' little-endian field layout, bit for bit
    np.testing.assert_array_equal(idx["residuals_flat"].cpu().numpy(), O.pack_residuals(bcodes, nbits))
    np.testing.assert_array_equal(idx["cu_seqlens_d"].cpu().numpy(), np.concatenate([[0], np.cumsum(doclens)]))
    Q = torch.randn(3, 32, 128).to(torch.bfloat16).cuda()
    got = maxsim_residual_varlen(Q, idx["codes_flat"], idx["residuals_flat"], idx["cu_seqlens_d"], idx["centroids"],
                                 idx["bucket_weights"], nbits)
    ref = O.maxsim_residual_varlen(Q.float().cpu().numpy(), codes, O.pack_residuals(bcodes, nbits),
                                   idx["cu_seqlens_d"].cpu().numpy(), cent, bw, nbits)
    assert rel_err(got.cpu().numpy(), ref) < 1e-2


@pytest.mark.parametrize("nbits", [2, 4])
def test_fastplaid_index_loader_raw_bits(tmp_path, nbits):
    """bit_order="raw" keeps fast-plaid's bytes as stored, as the reference's
    end-to-end harness does (bench_fastplaid_e2e.py:75-140): decode is bit-exact
    against the oracle's little-endian unpack of the unconverted bytes, and the
    scores equal the oracle on those bytes (the harness's result)."""
    from late_interaction_kernels.plaid import decode_residual_tokens, maxsim_residual_varlen
    from late_interaction_kernels.plaid_index import load_fastplaid_index

    _case(f"fast-plaid loader raw nbits={nbits}")
    doclens, cent, bw, codes, bcodes = _write_fastplaid_index(str(tmp_path), nbits, True, exact=True)
    raw = load_fastplaid_index(str(tmp_path), centroid_dtype=torch.float32, bit_order="raw")
    stored = O.pack_residuals_colbert(bcodes, nbits)  # the bytes on disk
    np.testing.assert_array_equal(raw["residuals_flat"].cpu().numpy(), stored)
    dec = decode_residual_tokens(raw["codes_flat"], raw["residuals_flat"], raw["centroids"], raw["bucket_weights"],
                                 nbits, normalize=False)
    want = O.decode_residual_tokens(codes, stored, cent, bw, nbits)
    np.testing.assert_array_equal(dec.float().cpu().numpy(), want.astype(np.float32))
    # and the converted ("colbert") load decodes the ColBERTv2 fields
    conv = load_fastplaid_index(str(tmp_path), centroid_dtype=torch.float32)
    dec_c = decode_residual_tokens(conv["codes_flat"], conv["residuals_flat"], conv["centroids"],
                                   conv["bucket_weights"], nbits, normalize=False)
    want_c = O.decode_residual_tokens(codes, O.pack_residuals(bcodes, nbits), cent, bw, nbits)
    np.testing.assert_array_equal(dec_c.float().cpu().numpy(), want_c.astype(np.float32))
    Q = torch.randn(3, 32, 128).to(torch.bfloat16).cuda()
    got = maxsim_residual_varlen(Q, raw["codes_flat"], raw["residuals_flat"], raw["cu_seqlens_d"], raw["centroids"],
                                 raw["bucket_weights"], nbits)
    ref = O.maxsim_residual_varlen(Q.float().cpu().numpy(), codes, stored, raw["cu_seqlens_d"].cpu().numpy(), cent, bw,
                                   nbits)
    assert rel_err(got.cpu().numpy(), ref) < 1e-2
    with pytest.raises(ValueError):
        load_fastplaid_index(str(tmp_path), bit_order="msb")
