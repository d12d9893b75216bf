"""The nearest-codebook search on the MI355X (ldx_vq_nearest4, ldx_vq_squared_norms4) against
the oracle, bit for bit: indices, norms and straight-through values are integer or
exactly-rounded results, so nothing but equality is accepted. Cases restate the reference's
own tests (tests/test_vq_optimized.py:27-94): strided batches of a 2,048-entry codebook,
first-index ties at midpoints and duplicate entries, NaN distances from fp16 norm overflow,
and a one-entry codebook; plus a config-sized search (51,200 latent vectors x 8,192 codes)
checked on sampled rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import vq as ovq

pytestmark = pytest.mark.gpu

DTYPES = {"float16": (torch.float16, np.float16), "float32": (torch.float32, np.float32)}


def _bits(a: np.ndarray) -> np.ndarray:
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def _search(pkg, dev, flat: np.ndarray, codebook: np.ndarray, tt):
    z = torch.from_numpy(flat).to(dev).to(tt).contiguous()
    cb = torch.from_numpy(codebook).to(dev).to(tt).contiguous()
    norms = pkg.ops.squared_norms4(cb)
    q = torch.empty_like(z)
    idx = pkg.ops.nearest_codebook4(z, cb, norms, quantized=q)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), q.cpu().numpy(), norms.cpu().numpy()


@pytest.mark.parametrize("dtype", list(DTYPES))
@pytest.mark.parametrize(("positions", "entries"), [(1, 2048), (2, 33), (3, 1), (31, 2), (32, 32), (33, 31)])
def test_nearest_codebook_first_index_at_ties(pkg, dev, dtype, positions, entries) -> None:
    """Duplicate entries, midpoints between neighbours and the entries themselves (and a
    zero vector) as latents: the indices, norms and straight-through values equal the
    oracle's bit for bit (tests/test_vq_optimized.py:54-94)."""
    tt, nt = DTYPES[dtype]
    rng = np.random.default_rng(317)
    cb = rng.normal(size=(entries, 4)).astype(np.float32)
    if entries > 3:
        cb[-1] = cb[0]
        cb[3] = -cb[2]
    pts = np.concatenate([(cb[:-1] + cb[1:]) / 2, cb, np.zeros((1, 4))]).astype(np.float32)
    pts = np.tile(pts, (positions // len(pts) + 1, 1))[:positions]
    cbt, ptt = cb.astype(nt), pts.astype(nt)
    idx, q, norms = _search(pkg, dev, ptt, cbt, tt)
    want_idx, want_q = ovq.quantize4(ptt, cbt, nt)
    np.testing.assert_array_equal(_bits(norms), _bits(ovq.squared_norms4(cbt, nt)))
    np.testing.assert_array_equal(idx, want_idx)
    np.testing.assert_array_equal(_bits(q), _bits(want_q))
    # fp16 squared norms overflow on finite values: NaN distances keep first-index priority
    special = np.array([[np.nan, 0, 0, 0], [300, 1, -2, 3]], np.float32).astype(nt)
    idx, _, _ = _search(pkg, dev, special, cbt, tt)
    np.testing.assert_array_equal(idx, ovq.nearest_codebook4(special, cbt, nt))


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_quantize_strided_batches(pkg, dev, dtype) -> None:
    """A strided (2, 4, 9, 8, 7) latent against 2,048 codes through VqDecoder.quantize: the
    straight-through values equal the oracle's bit for bit (tests/test_vq_optimized.py:27-51)."""
    tt, nt = DTYPES[dtype]
    rng = np.random.default_rng(2701)
    cb = rng.normal(size=(2048, 4)).astype(np.float32).astype(nt)
    z = rng.normal(size=(2, 4, 9, 8, 14)).astype(np.float32).astype(nt)[..., ::2]
    zt = torch.from_numpy(np.ascontiguousarray(z)).to(dev).permute(0, 2, 3, 4, 1)   # NDHWC view, strided
    dec = pkg.vq.VqDecoder({"quantize.embedding.weight": cb})
    got = dec.quantize(zt, tt)
    torch.cuda.synchronize()
    flat = z.transpose(0, 2, 3, 4, 1).reshape(-1, 4)
    _, want = ovq.quantize4(flat, cb, nt)
    np.testing.assert_array_equal(_bits(got.cpu().numpy().reshape(-1, 4)), _bits(want))


def test_replacing_the_codebook_replaces_its_norms(pkg, dev) -> None:
    """A decoder whose codebook is replaced selects from the new codebook
    (tests/test_vq_optimized.py:97-113)."""
    dec = pkg.vq.VqDecoder({"quantize.embedding.weight": np.array([[0, 0, 0, 0], [2, 0, 0, 0]], np.float32)})
    z = torch.tensor([[[[[1.75, 0, 0, 0]]]]], dtype=torch.float32, device=dev)
    first = dec.quantize(z, torch.float32)
    dec.set_codebook(np.array([[1, 0, 0, 0], [20, 0, 0, 0]], np.float32))
    second = dec.quantize(z, torch.float32)
    torch.cuda.synchronize()
    assert first.reshape(4).tolist() == [2, 0, 0, 0]
    assert second.reshape(4).tolist() == [1, 0, 0, 0]


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_config_sized_search_on_sampled_rows(pkg, dev, dtype) -> None:
    """51,200 latent vectors (a 32 x 40 x 40 latent) against 8,192 codes, four code chunks
    through LDS: 1,024 sampled rows (first and last included) equal the oracle."""
    tt, nt = DTYPES[dtype]
    rng = np.random.default_rng(99)
    cb = rng.normal(size=(8192, 4)).astype(nt)
    flat = rng.normal(size=(51200, 4)).astype(nt)
    idx, q, _ = _search(pkg, dev, flat, cb, tt)
    rows = np.unique(np.concatenate([[0, 51199], rng.integers(0, 51200, 1022)]))
    want_idx, want_q = ovq.quantize4(flat[rows], cb, nt)
    np.testing.assert_array_equal(idx[rows], want_idx)
    np.testing.assert_array_equal(_bits(q[rows]), _bits(want_q))


def test_search_rejects_bad_arguments(pkg, dev) -> None:
    """Shape and dtype errors raise before anything is launched."""
    z = torch.zeros((3, 4), dtype=torch.float16, device=dev)
    cb = torch.zeros((5, 4), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError):
        pkg.ops.nearest_codebook4(z, cb, torch.zeros(5, dtype=torch.float32, device=dev))
    with pytest.raises(ValueError):
        pkg.ops.nearest_codebook4(torch.zeros((3, 3), dtype=torch.float16, device=dev), cb.half(),
                                  torch.zeros(5, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        pkg.ops.squared_norms4(torch.zeros((0, 4), dtype=torch.float16, device=dev))
