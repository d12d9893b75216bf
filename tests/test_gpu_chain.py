"""Token-row chains (ldx_token_chain through ops.token_chain): the transformer block's dense
layers and LayerNorms on a 32-row tile per workgroup (mlx_model.py:204-220, 360-374,
522-552).

Each stage is checked against float64 evaluated from the chain's own rounded input to that
stage (the stored y1, or the float64 stages rounded to fp16 where the chain keeps its
tiles on chip), at the reference's per-element error model (tests/test_native_kernels.py:
37-39): half an ulp of each stored result, 8 * 2^-23 of the summed magnitudes for the fp32
accumulation, 2^-10 of the magnitudes where an input was itself rounded to fp16 (the
LayerNorm output), and each stage's input error carried through |W|. The chain is also held
to the separate dense / LayerNorm launches at the same bound, and whole UNets with and
without chains are compared.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import norm as onm
from oracle import unet as oun
from tests.conftest import ACCUMULATION_EPS, assert_fp16_bar, half_spacing

pytestmark = pytest.mark.gpu
GELU_SLOPE_MAX = 1.13   # max |d gelu / dx|


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def host(t) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def f16(a: np.ndarray) -> np.ndarray:
    return np.asarray(a).astype(np.float16).astype(np.float64)


class Stage:
    def __init__(self, rng, c_in: int, c_out: int, pkg, dev, act=None):
        self.w = (rng.normal(size=(c_out, c_in)) / np.sqrt(c_in)).astype(np.float16)
        self.b = (rng.normal(size=c_out) * 0.1).astype(np.float32)
        self.act = act
        self.packed = pkg.ops.pack_weight(to_dev(self.w, dev))
        self.bias = to_dev(self.b, dev)

    def g(self):
        return (self.packed, self.bias, self.act)

    def ref(self, inp: np.ndarray, err_in: np.ndarray, res: np.ndarray | None = None):
        """float64 stage from an fp16-valued input with per-element error ``err_in``:
        (rounded output, its error bound)."""
        w = self.w.astype(np.float64)
        pre = inp @ w.T + self.b.astype(np.float64) + (0 if res is None else res)
        mag = np.abs(inp) @ np.abs(w).T
        err_pre = err_in @ np.abs(w).T + ACCUMULATION_EPS * (mag + np.abs(pre))
        if self.act == "gelu":
            h = f16(pre)
            out = f16(onm.gelu(h))
            err = GELU_SLOPE_MAX * (err_pre + half_spacing(pre)) + half_spacing(out)
        else:
            out = f16(pre)
            err = err_pre + half_spacing(out)
        return out, err


def ln_ref(y1: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float = 1e-5):
    z = f16(onm.layer_norm(y1, g.astype(np.float64), b.astype(np.float64), eps))
    return z, 2.0 ** -10 * np.abs(z) + 2 * half_spacing(z)


def within(got, want, err, what):
    excess = np.abs(got - want) - 2 * err
    assert np.all(np.isfinite(got)), f"{what}: non-finite"
    assert np.all(excess <= 0), f"{what}: max excess {excess.max():.3e} (max err {np.abs(got - want).max():.3e})"


@pytest.mark.parametrize("rows,tokens,c,c2,form", [
    (800, 800, 256, 768, "in"),      # LINet level 2: proj_in (+ GroupNorm affine) -> norm1 -> q/k/v
    (200, 100, 256, 256, "mid"),     # level 3, batch 2: to_out (+ x) -> norm2 -> to_q
    (100, 100, 256, 1024, "out"),    # to_out (+ x) -> norm3 -> ff GELU -> ff (+ x) -> proj_out (+ x)
    (37, 37, 128, 512, "out"),       # a ragged tile, narrower rows
    (64, 32, 64, 256, "out"),        # two batch items in a tile pair
])
def test_token_chain_stages_match_float64(pkg, dev, rows, tokens, c, c2, form) -> None:
    rng = np.random.default_rng(rows * 7 + c + c2)
    x = (rng.normal(size=(rows, c)) * 1.5).astype(np.float16)
    g1 = Stage(rng, c, c, pkg, dev)
    g2 = Stage(rng, c, c2, pkg, dev, act="gelu" if form == "out" else None)
    gam = (1 + 0.2 * rng.normal(size=c)).astype(np.float32)
    bet = (0.2 * rng.normal(size=c)).astype(np.float32)
    ln = (to_dev(gam, dev), to_dev(bet, dev), 1e-5)
    xd = to_dev(x, dev)
    y1 = torch.empty((rows, c), dtype=torch.float16, device=dev)
    kw = dict(tokens=tokens, y1=y1)
    inp = x.astype(np.float64)
    err_in = np.zeros_like(inp)
    res1 = None
    if form == "in":
        aff = np.stack([1 + 0.3 * rng.normal(size=(rows // tokens, c)), 0.3 * rng.normal(size=(rows // tokens, c))],
                       -1).astype(np.float32)
        kw["affine"] = to_dev(aff, dev)
        a = np.repeat(aff, tokens, axis=0)
        inp = f16(inp * a[..., 0] + a[..., 1])
        err_in = half_spacing(inp)       # fp32 fma then one rounding vs float64 then rounding
    else:
        res1 = rng.normal(size=(rows, c)).astype(np.float16)
        kw["res1"] = to_dev(res1, dev)
    g3 = g4 = None
    if form == "out":
        g3 = Stage(rng, c2, c, pkg, dev)
        g4 = Stage(rng, c, c, pkg, dev)
        res4 = rng.normal(size=(rows, c)).astype(np.float16)
        kw.update(g3=g3.g(), g4=g4.g(), res4=to_dev(res4, dev))
    print(f"token_chain {form} rows {rows} c {c} c2 {c2}", flush=True)
    out = pkg.ops.token_chain(xd, g1.g(), ln, g2.g(), **kw)
    torch.cuda.synchronize()
    y1h = host(y1)
    want1, err1 = g1.ref(inp, err_in, None if res1 is None else res1.astype(np.float64))
    within(y1h, want1, err1, "G1")
    z, errz = ln_ref(y1h, gam, bet)
    h, errh = g2.ref(z, errz)
    if form != "out":
        within(host(out), h, errh, "G2")
        return
    y3, err3 = g3.ref(h, errh, y1h)
    o, erro = g4.ref(y3, err3, res4.astype(np.float64))
    within(host(out), o, erro, "G4")
    # the same layers as separate launches
    d = pkg.ops.dense
    sy1 = d(xd, g1.packed, g1.bias, residual=kw["res1"])
    sh = d(sy1, g2.packed, g2.bias, act="gelu", ln=ln)
    sy3 = d(sh, g3.packed, g3.bias, residual=sy1)
    so = d(sy3, g4.packed, g4.bias, residual=kw["res4"])
    within(host(out), host(so), erro, "chain vs separate launches")


def test_token_chain_bf16(pkg, dev) -> None:
    """The bf16 compile on the feed-forward chain, against float64 at the bf16 bar."""
    rng = np.random.default_rng(5)
    rows, c, c2 = 96, 128, 512
    mk = lambda co, ci: (rng.normal(size=(co, ci)) / np.sqrt(ci)).astype(np.float32)
    ws = [mk(c, c), mk(c2, c), mk(c, c2), mk(c, c)]
    bs = [(rng.normal(size=w.shape[0]) * 0.1).astype(np.float32) for w in ws]
    x = rng.normal(size=(rows, c)).astype(np.float32)
    res1 = rng.normal(size=(rows, c)).astype(np.float32)
    res4 = rng.normal(size=(rows, c)).astype(np.float32)
    gam = np.ones(c, np.float32)
    bet = np.zeros(c, np.float32)
    bf = torch.bfloat16
    g = [(pkg.ops.pack_weight(to_dev(w, dev, bf)), to_dev(b, dev), a) for w, b, a in
         zip(ws, bs, (None, "gelu", None, None))]
    out = pkg.ops.token_chain(to_dev(x, dev, bf), g[0], (to_dev(gam, dev), to_dev(bet, dev), 1e-5), g[1], tokens=rows,
                              res1=to_dev(res1, dev, bf), g3=g[2], g4=g[3], res4=to_dev(res4, dev, bf))
    torch.cuda.synchronize()
    r = lambda a: torch.from_numpy(a).to(bf).double().numpy()
    y1 = r(x) @ r(ws[0]).T + bs[0] + r(res1)
    z = onm.layer_norm(y1, gam.astype(np.float64), bet.astype(np.float64), 1e-5)
    h = onm.gelu(z @ r(ws[1]).T + bs[1])
    y3 = h @ r(ws[2]).T + bs[2] + y1
    o = y3 @ r(ws[3]).T + bs[3] + r(res4)
    assert_fp16_bar(host(out), o, max_abs=0.16, rel_l2=8e-3)


@pytest.mark.parametrize("skip_context", [False, True])
def test_unet_with_and_without_chains(pkg, dev, skip_context) -> None:
    """The 16^3 UNet with attention at its two coarse levels and the middle: chained
    transformer blocks against the per-layer launches and against the float64 oracle."""
    cfg = pkg.unet.UnetConfig(32, 1, (2, 4), (1, 2, 4, 4), 32, skip_context)
    w = pkg.unet.unet_state_dict(cfg, in_channels=4, out_channels=4, context_dim=None if skip_context else 64,
                                 seed=3)
    w16 = {k: v.astype(np.float16) for k, v in w.items()}
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 4, 16, 16, 16)).astype(np.float16)
    t = np.array([321], np.int32)
    ctx = None if skip_context else rng.standard_normal((1, 7, 64)).astype(np.float16)
    outs = []
    for chain in (True, False):
        net = pkg.unet.LdmUnet(w16, cfg, chain=chain)
        y = net(to_dev(x, dev), to_dev(t, dev), None if ctx is None else to_dev(ctx, dev))
        torch.cuda.synchronize()
        outs.append(host(y))
    ocfg = oun.UnetConfig(model_channels=cfg.model_channels, num_res_blocks=cfg.num_res_blocks,
                          attention_resolutions=cfg.attention_resolutions, channel_mult=cfg.channel_mult,
                          num_head_channels=cfg.num_head_channels, skip_context=cfg.skip_context)
    exact = oun.Unet(w16, ocfg, half=False).forward(x, t, ctx)
    for o in outs:
        assert_fp16_bar(o, exact, rel_l2=5e-3)
    assert_fp16_bar(outs[0], outs[1], max_abs=1e-2, rel_l2=2e-3)
