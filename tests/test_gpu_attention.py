"""Flash-attention parity on the MI355X against the float64 softmax oracle
(tests/test_native_kernels.py:380-450: fp16 atol = rtol = 2e-3) and the fp16 bar."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from tests.conftest import assert_fp16_bar

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize(("batch", "length", "heads", "ties"), [
    (2, 32, 1, False), (1, 96, 2, False), (1, 96, 2, True), (1, 1056, 2, False),
    (1, 512, 4, False), (1, 512, 8, False), (1, 512, 16, False),
])
def test_projection_layout_head32_matches_float64(pkg, dev, batch, length, heads, ties) -> None:
    """The reference's nax-half cases (tests/test_native_kernels.py:395-450): inputs
    q, k * 2, v * 1 from rng(length + keys), head-interleaved (B, L, heads * 32)."""
    rng = np.random.default_rng(length + length)
    q, k, v = (rng.normal(size=(batch, length, heads * 32)) * s for s in (2.0, 2.0, 1.0))
    if ties:
        q = np.zeros_like(q)
    q, k, v = (a.astype(np.float16) for a in (q, k, v))
    out = pkg.ops.flash_attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), heads=heads,
                                  scale=32 ** -0.5)
    torch.cuda.synchronize()
    exp = oatt.attention_projected(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                                   heads, 32 ** -0.5)
    act = host(out)
    assert out.dtype == torch.float16 and np.all(np.isfinite(act))
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize(("b", "h", "lq", "lk", "d"), [
    (1, 8, 1600, 1600, 64),   # config 2 self-attention
    (1, 8, 1600, 77, 64),     # config 2 cross-attention
    (2, 4, 100, 77, 32),      # LINet lowest-level cross attention
    (1, 2, 64, 64, 16),       # the fixture UNet's 16-wide heads
    (1, 1, 300, 300, 256),    # VQ mid attention head width
    (1, 2, 129, 200, 128),
    (2, 3, 1, 5, 64),         # single query, ragged keys
])
def test_attention_matches_float64(pkg, dev, b, h, lq, lk, d) -> None:
    rng = np.random.default_rng(lq * 7 + lk + d)
    q = rng.normal(size=(b, h, lq, d)).astype(np.float16)
    k = rng.normal(size=(b, h, lk, d)).astype(np.float16)
    v = rng.normal(size=(b, h, lk, d)).astype(np.float16)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d ** -0.5)
    torch.cuda.synchronize()
    exp = oatt.attention(q, k, v, d ** -0.5)
    act = host(out)
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)
    assert_fp16_bar(act, exp)


def test_attention_additive_and_boolean_masks(pkg, dev) -> None:
    """Additive -inf / boolean key masks (mlx_model.py:843-847); a fully masked row is 0."""
    rng = np.random.default_rng(3)
    b, h, lq, lk, d = 2, 3, 40, 77, 64
    q, k, v = (rng.normal(size=(b, h, n, d)).astype(np.float16) for n in (lq, lk, lk))
    keep = rng.random((b, 1, 1, lk)) > 0.3
    keep[..., 0] = True
    add = np.where(keep, 0.0, -np.inf).astype(np.float32)
    add2 = add + rng.normal(size=(b, 1, lq, lk)).astype(np.float32)  # general additive bias
    for m_host, m_dev in ((add, to_dev(keep, dev)), (add2, to_dev(add2, dev))):
        out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 0.125, m_dev)
        torch.cuda.synchronize()
        np.testing.assert_allclose(host(out), oatt.attention(q, k, v, 0.125, m_host), rtol=2e-3, atol=2e-3)
    none = np.zeros((b, 1, lq, lk), bool)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 0.125, to_dev(none, dev))
    torch.cuda.synchronize()
    assert np.all(host(out) == 0)


def test_attention_large_magnitudes_keep_running_max(pkg, dev) -> None:
    """Peaked rows whose maximum moves across key tiles."""
    rng = np.random.default_rng(5)
    q = (rng.normal(size=(1, 2, 200, 64)) * 3).astype(np.float16)
    k = (rng.normal(size=(1, 2, 700, 64)) * 3).astype(np.float16)
    v = rng.normal(size=(1, 2, 700, 64)).astype(np.float16)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), 0.125)
    torch.cuda.synchronize()
    np.testing.assert_allclose(host(out), oatt.attention(q, k, v, 0.125), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("split", ["1", "4", "8", "-4", "-42", "-8"])
@pytest.mark.parametrize(("b", "h", "lq", "lk", "d", "masked"), [
    (1, 8, 1600, 1600, 64, False),   # config 2 self-attention
    (2, 3, 100, 77, 32, False),      # ragged last key block
    (1, 2, 33, 5, 64, False),        # fewer key blocks than waves
    (2, 3, 70, 77, 64, True),        # additive mask; three query blocks (a half pair)
])
def test_attention_key_split_variants_match_float64(pkg, dev, monkeypatch, split, b, h, lq, lk, d,
                                                     masked) -> None:
    """Every kernel the launcher can pick (LDX_ATTN_SPLIT: 128 queries per workgroup,
    four- and eight-way key splits, the DMA-fed pipelined four-way split with one or two
    query blocks per workgroup and eight-way split) on the same inputs."""
    monkeypatch.setenv("LDX_ATTN_SPLIT", split)
    rng = np.random.default_rng(lq + 3 * lk + d)
    q, k, v = (rng.normal(size=(b, h, n, d)).astype(np.float16) for n in (lq, lk, lk))
    m_host = m_dev = None
    if masked:
        m_host = rng.normal(size=(b, 1, lq, lk)).astype(np.float32)
        m_host[..., 5:9] = -np.inf
        m_dev = to_dev(m_host, dev)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d ** -0.5, m_dev)
    torch.cuda.synchronize()
    exp = oatt.attention(q, k, v, d ** -0.5, m_host)
    act = host(out)
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)
    assert_fp16_bar(act, exp)


@pytest.mark.parametrize("shares", ["1,1,1,1", "5,1,3,2", "16,1,1,1"])
@pytest.mark.parametrize("split", ["-4", "-42"])
@pytest.mark.parametrize(("b", "h", "lq", "lk", "d", "masked"), [
    (1, 4, 96, 1000, 64, False),     # long keys: several periods and a ragged last block
    (2, 3, 70, 77, 32, True),        # additive mask; fewer blocks than one period
])
def test_attention_key_share_patterns_match_float64(pkg, dev, monkeypatch, shares, split, b, h, lq, lk, d,
                                                    masked) -> None:
    """The pipelined key split with uneven key shares (LDX_ATTN_SHARES: blocks per period of
    each share, interleaved by due time) gives the same attention."""
    monkeypatch.setenv("LDX_ATTN_SPLIT", split)
    monkeypatch.setenv("LDX_ATTN_SHARES", shares)
    rng = np.random.default_rng(lk + d)
    q, k, v = (rng.normal(size=(b, h, n, d)).astype(np.float16) for n in (lq, lk, lk))
    m_host = m_dev = None
    if masked:
        m_host = rng.normal(size=(b, 1, lq, lk)).astype(np.float32)
        m_host[..., 3:11] = -np.inf
        m_dev = to_dev(m_host, dev)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d ** -0.5, m_dev)
    torch.cuda.synchronize()
    exp = oatt.attention(q, k, v, d ** -0.5, m_host)
    act = host(out)
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)
    assert_fp16_bar(act, exp)


@pytest.mark.parametrize("split", ["default", "1", "-1"])
@pytest.mark.parametrize(("b", "h", "lq", "lk", "d", "masked", "mag"), [
    (1, 1, 300, 300, 256, False, 1.0),   # VQ mid-attention width, ragged query and key blocks
    (2, 2, 129, 77, 128, True, 1.0),     # additive mask, one query past a 128-query block
    (1, 1, 70, 1000, 256, False, 3.0),   # many key blocks, peaked rows (base moves)
    (1, 2, 256, 96, 128, False, 1.0),    # whole blocks only
])
def test_attention_wide_heads_match_float64(pkg, dev, monkeypatch, split, b, h, lq, lk, d, masked, mag) -> None:
    """Head widths 128 and 256: the launcher's choice, the register-staged 128-query
    kernel (LDX_ATTN_SPLIT=1) and the DMA-fed pipelined one (=-1) against float64
    softmax attention."""
    if split == "default":
        monkeypatch.delenv("LDX_ATTN_SPLIT", raising=False)
    else:
        monkeypatch.setenv("LDX_ATTN_SPLIT", split)
    rng = np.random.default_rng(lq + 7 * lk + d)
    q, k = ((rng.normal(size=(b, h, n, d)) * mag).astype(np.float16) for n in (lq, lk))
    v = rng.normal(size=(b, h, lk, d)).astype(np.float16)
    m_host = m_dev = None
    if masked:
        m_host = rng.normal(size=(b, 1, lq, lk)).astype(np.float32)
        m_host[..., 3:7] = -np.inf
        m_dev = to_dev(m_host, dev)
    out = pkg.ops.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), d ** -0.5, m_dev)
    torch.cuda.synchronize()
    exp = oatt.attention(q, k, v, d ** -0.5, m_host)
    act = host(out)
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)
    assert_fp16_bar(act, exp)


@pytest.mark.parametrize(("h", "lq", "lk", "d", "masked"), [
    (1, 12800, 12800, 256, False),   # 100 tiles of 128 queries on 256 CUs
    (2, 19200, 4000, 128, False),    # 300 tiles, two workgroups per CU
    (1, 12800, 9000, 256, True),     # additive mask with removed keys, ragged last key block
])
def test_attention_balanced_wide_schedule(pkg, dev, monkeypatch, h, lq, lk, d, masked) -> None:
    """Wide heads whose query tiles fill the resident workgroups' rounds poorly take the
    balanced schedule: an even share of (tile, key block) units per workgroup, the pieces
    of a split tile's key range combined by the merge kernel. Sampled rows against float64
    over all keys, and the whole output against the one-workgroup-per-tile schedule."""
    monkeypatch.delenv("LDX_ATTN_SPLIT", raising=False)
    rng = np.random.default_rng(lq + lk + d)
    q, k, v = (rng.normal(size=(1, h, n, d)).astype(np.float16) for n in (lq, lk, lk))
    m_host = m_dev = None
    if masked:
        m_host = rng.normal(size=(1, 1, 1, lk)).astype(np.float32)
        m_host[..., 100:4200] = -np.inf   # whole key blocks removed, inside one piece or across two
        m_dev = to_dev(m_host, dev)
    qd, kd, vd = to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    a = pkg.ops._attn_args(qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2), qd.transpose(1, 2),
                           d ** -0.5, None)
    assert a.workspace_bytes > 0, "this shape should take the balanced schedule"
    print(f"balanced attention h {h} lq {lq} lk {lk} d {d} masked {masked}", flush=True)
    out = pkg.ops.attention(qd, kd, vd, d ** -0.5, m_dev)
    monkeypatch.setenv("LDX_ATTN_NO_BALANCE", "1")
    ref = pkg.ops.attention(qd, kd, vd, d ** -0.5, m_dev)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 127, 128, lq - 1], rng.integers(0, lq, 60)]))
    mh = None if m_host is None else m_host
    exp = oatt.attention(q[:, :, rows], k, v, d ** -0.5, mh)
    act = host(out)[:, :, rows]
    np.testing.assert_allclose(act, exp, rtol=2e-3, atol=2e-3)
    assert_fp16_bar(act, exp)
    # the two schedules differ only in fp32 summation order before one fp16 rounding
    assert_fp16_bar(host(out), host(ref))
