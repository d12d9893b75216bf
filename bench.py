"""Benchmark of the MI355X dense hot path (one GPU).

Headline (``value``): config 1 -- one 3x3x3 stride-1 conv3d, NDHWC fp16, N=1,
C_in = C_out = 64, 32x40x40 -- in TFLOP/s, with its MFMA roofline. The same JSON line
also carries config 2 (flash attention, self 1x8x1600x64 and 1600 x 77 cross) and,
when the model layer is present, the config-3/4/5 figures.

A "step" is one launch of the op over one batch of synthetic input resident in HBM.
K steps are captured in one HIP graph and replayed; HIP events recorded on the stream
the kernels are launched on bracket the K launches (after a device synchronise on both
sides), so the per-launch time excludes host launch overhead.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-model] [--skip-cpu]``
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "conv3d & flash-attn TFLOP/s (% MFMA peak); ms per 3D-UNet denoise step"
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3    # MI355X vector fp32 (the source-order conv runs on the VALU)
# HBM bytes per config-1 conv launch come from the committed profile of the benched kernel:
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over this script with --copy-calibration,
# each divided by what the counter reports per byte of a plain 512 MiB device copy. The
# profile states them on a line "roofline.traffic: <bytes> bytes per launch (revision <rev>)".
CONV_PROFILE = REPO / "profiles" / "conv3d_config1.txt"


def profiled_traffic() -> tuple[float | None, str | None]:
    """(HBM bytes per config-1 launch, "profile @ revision") from CONV_PROFILE, or (None,
    None) when the profile states none."""
    import re

    try:
        text = CONV_PROFILE.read_text()
    except OSError:
        return None, None
    m = re.search(r"roofline\.traffic:\s*([0-9.eE+]+) bytes per launch \(revision ([0-9a-f]+)\)", text)
    if not m:
        return None, None
    return float(m.group(1)), f"{CONV_PROFILE.relative_to(REPO)} @ {m.group(2)}"


class SclkSampler:
    """The GPU's shader clock while a figure is measured: a thread reads the device's
    ``pp_dpm_sclk`` (sysfs; the level marked ``*`` is the current clock) every
    ``interval_s`` between ``__enter__`` and ``__exit__``. Figures from different boxes differ with it
    (the same kernel runs ~12 % slower at 1.95 GHz than at 2.2 GHz), so each figure carries
    the median, min and max MHz it ran at (``None`` where sysfs is not readable)."""

    def __init__(self, interval_s: float = 0.002):
        self.interval = interval_s
        self.path = self._find()
        self.samples: list[int] = []
        self._stop = None
        self._thread = None

    @staticmethod
    def _find():
        import glob

        import torch

        p = torch.cuda.get_device_properties(0)
        cand = Path(f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
                    "/pp_dpm_sclk")
        if cand.exists():
            return cand
        found = glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")
        return Path(found[0]) if len(found) == 1 else None

    def _read(self):
        import re

        try:
            for line in self.path.read_text().splitlines():
                if line.rstrip().endswith("*"):
                    m = re.search(r"(\d+)\s*[Mm]hz", line)
                    return int(m.group(1)) if m else None
        except OSError:
            return None
        return None

    def __enter__(self):
        import threading

        if self.path is None:
            return self
        self._stop = threading.Event()

        def run():
            while not self._stop.is_set():
                v = self._read()
                if v is not None:
                    self.samples.append(v)
                self._stop.wait(self.interval)

        self._thread = threading.Thread(target=run, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc):
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
        return False

    def summary(self):
        if not self.samples:
            return None
        return {"median": int(np.median(self.samples)), "min": min(self.samples), "max": max(self.samples),
                "samples": len(self.samples)}


# Each timed region is one replay of the K captured launches; the reported figure is the
# median over this many such regions. A replay occasionally stalls for a few hundred
# microseconds while the host is still submitting its packets (seen in kernel traces as a
# run of idle gaps inside one replay), and the median keeps that out of the per-launch time.
TIMED_REPLAYS = 5
# Seconds of untimed replays before each figure (the first figure of a process takes 3x);
# --settle sets it (short for profiling runs, whose every replay is traced).
SETTLE_S = [0.5]
# The 200-step config-5 loop is timed this many times; the median is reported.
CONFIG5_RUNS = 5


def _graph_time(launch, steps: int, warmup: int, clock: "SclkSampler | None" = None, settle: float = 1.0) -> float:
    """Per-launch ms: ``warmup`` eager launches, then ``steps`` launches captured in one
    graph, replayed untimed for ``settle`` x SETTLE_S seconds, then TIMED_REPLAYS times between HIP
    events (``clock`` samples the shader clock over those); the median replay time divided
    by ``steps``."""
    import torch

    for _ in range(max(warmup, 1)):
        launch()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()  # first call on the capture stream outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for _ in range(steps):
            launch()
    # Untimed replays first: the clocks climb to their loaded steady state. From idle that
    # takes several hundred ms (the first figure of a process, sampled over 0.2 s of
    # replays, ran at a median 1,370 MHz and 30 % slower).
    t0 = time.perf_counter()
    while True:
        g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 > settle * SETTLE_S[0]:
            break
    times = []
    if clock is not None:
        clock.__enter__()
    for _ in range(TIMED_REPLAYS):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        g.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / steps)
    if clock is not None:
        clock.__exit__(None, None, None)
    return float(np.median(times))


def bench_conv(pkg, steps: int, warmup: int) -> dict:
    import torch

    ops, lib = pkg.ops, pkg._lib
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 64)).astype(np.float16)).to(dev)
    w = torch.from_numpy((rng.standard_normal((64, 64, 3, 3, 3)) / math.sqrt(27 * 64)).astype(np.float16)).to(dev)
    b = torch.from_numpy((rng.standard_normal(64) * 0.01).astype(np.float32)).to(dev)
    pk = ops.pack_weight(w)
    y = torch.empty((1, 32, 40, 40, 64), dtype=torch.float16, device=dev)
    a = lib.ConvArgs()
    a.batch, a.in_d, a.in_h, a.in_w = 1, 32, 40, 40
    a.c0, a.c1, a.out_c, a.ksize, a.stride, a.upsample = 64, 0, 64, 3, 1, 0
    a.x0, a.x0_pitch, a.weight = x.data_ptr(), 64, pk.data.data_ptr()
    a.bias, a.bias_batched, a.output_scale, a.act = b.data_ptr(), 0, 1.0, 0
    a.y, a.y_pitch = y.data_ptr(), 64
    ref = ctypes.byref(a)

    def launch():
        lib.check(lib.lib.ldx_conv3d(ref, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "conv3d")

    clk = SclkSampler(0.0005)
    ms = _graph_time(launch, steps, warmup, clk, settle=3.0)   # the first figure: the GPU starts idle
    flop = 2.0 * 51200 * 64 * 64 * 27
    tflops = flop / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tflops, "flop": flop, "sclk_mhz": clk.summary(),
            "bytes": (51200 * 64 * 2) * 2 + 64 * 64 * 27 * 2, "x": x, "w": w, "b": b}


def bench_attention(pkg, steps: int, warmup: int) -> dict:
    import torch

    ops, lib = pkg.ops, pkg._lib
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    q = torch.from_numpy(rng.standard_normal((1, 8, 1600, 64)).astype(np.float16)).to(dev)
    k = torch.from_numpy(rng.standard_normal((1, 8, 1600, 64)).astype(np.float16)).to(dev)
    v = torch.from_numpy(rng.standard_normal((1, 8, 1600, 64)).astype(np.float16)).to(dev)
    ctx = torch.from_numpy(rng.standard_normal((1, 77, 768)).astype(np.float16)).to(dev)
    wk = torch.from_numpy((rng.standard_normal((512, 768)) / math.sqrt(768)).astype(np.float16)).to(dev)
    wv = torch.from_numpy((rng.standard_normal((512, 768)) / math.sqrt(768)).astype(np.float16)).to(dev)
    kc = ops.dense(ctx, ops.pack_weight(wk)).view(1, 77, 8, 64).transpose(1, 2)
    vc = ops.dense(ctx, ops.pack_weight(wv)).view(1, 77, 8, 64).transpose(1, 2)
    out = {}
    for name, kk, vv, lk in (("self", k, v, 1600), ("cross", kc, vc, 77)):
        o = torch.empty((1, 8, 1600, 64), dtype=torch.float16, device=dev)
        a = ops._attn_args(q.transpose(1, 2), kk.transpose(1, 2), vv.transpose(1, 2), o.transpose(1, 2),
                           0.125, None)
        ref = ctypes.byref(a)

        def launch(ref=ref):
            lib.check(lib.lib.ldx_attention(ref, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                      "attention")

        clk = SclkSampler(0.0005)
        ms = _graph_time(launch, steps, warmup, clk)
        flop = 4.0 * 8 * 1600 * lk * 64
        byts = 2.0 * (2 * 8 * 1600 * 64 + 2 * 8 * lk * 64)
        out[name] = {"ms": ms, "tflops": flop / (ms * 1e-3) / 1e12, "flop": flop, "sclk_mhz": clk.summary(),
                     "frac_peak": flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS,
                     "gbs": byts / (ms * 1e-3) / 1e9}
    out["_tensors"] = (q, k, v)
    return out


def bench_source(pkg, steps: int, warmup: int, cpu: bool) -> dict:
    """The reference's source-order fp16 arithmetic at config-1 size: ``conv3d_half`` (Torch-CPU's
    four-partial reduction order on the VALU, NCDHW) and ``group_norm_half`` (32 groups) on the
    config-1 tensor. With ``cpu``, Torch-CPU's own fp16 conv3d (oneDNN off: the order these
    kernels reproduce) on 4 of the 32 output planes, scaled to the whole conv."""
    import torch
    import torch.nn.functional as F

    ops = pkg.ops
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)
    xh = rng.standard_normal((1, 64, 32, 40, 40)).astype(np.float16)
    wh = (rng.standard_normal((64, 64, 3, 3, 3)) / math.sqrt(27 * 64)).astype(np.float16)
    bh = (rng.standard_normal(64) * 0.01).astype(np.float16)
    x, w, b = (torch.from_numpy(a).to(dev) for a in (xh, wh, bh))
    gamma = torch.ones(64, dtype=torch.float16, device=dev)
    conv_ms = _graph_time(lambda: ops.conv3d_half(x, w, b, padding=1, stride=1), steps, warmup)
    gn_ms = _graph_time(lambda: ops.group_norm_half(x, gamma, b, groups=32, eps=1e-5), steps, warmup)
    flop = 2.0 * 51200 * 64 * 64 * 27
    out = {"conv_ms": round(conv_ms, 5), "conv_tflops": round(flop / (conv_ms * 1e-3) / 1e12, 2),
           "conv_frac_fp32_peak": round(flop / (conv_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4),
           "gn_ms": round(gn_ms, 5),
           "gn_gbs": round(3 * 51200 * 64 * 2 / (gn_ms * 1e-3) / 1e9, 1),
           "config": "config-1 tensor (1, 64, 32, 40, 40) NCDHW fp16; conv 3x3x3 padding 1; GroupNorm 32 groups "
                     "(reads x twice, writes y: 3 x 6.55 MB)"}
    if cpu:
        threads = _cpu_threads()
        xs, ws, bs = torch.from_numpy(xh[:, :, :4]), torch.from_numpy(wh), torch.from_numpy(bh)
        with torch.no_grad(), torch.backends.mkldnn.flags(enabled=False):
            t0 = time.perf_counter()
            F.conv3d(xs, ws, bs, padding=1)
            sec = (time.perf_counter() - t0) * 8
        out["cpu_torch_conv_ms"] = round(sec * 1e3, 1)
        out["cpu_sample"] = (f"Torch {torch.__version__} CPU fp16 conv3d (oneDNN off) on 4 of 32 output planes, "
                             f"x8; {threads} threads")
    return out


def _graph_replay_ms(fn, reps: int, warmup: int = 2) -> float:
    """Average ms of ``fn`` (a whole forward) captured once as a HIP graph and replayed
    ``reps`` times between HIP events."""
    import torch

    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _half(w: dict) -> dict:
    return {k: v.astype(np.float16) for k, v in w.items()}


def bench_config3(pkg, reps: int) -> dict:
    """3-D UNet ResBlock stack: 4-channel 32x40x40 latent, levels 64/128/256/256, two
    ResBlocks each (1x1 skip on channel change), stride-2 conv between levels."""
    import torch

    cfg = pkg.unet.UnetConfig(64, 2, (), (1, 2, 4, 4), 32, True)
    net = pkg.unet.LdmUnet(_half(pkg.unet.unet_state_dict(cfg, in_channels=4, out_channels=4, context_dim=None,
                                                          seed=0)), cfg)
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 4)).astype(np.float16)).cuda()
    t = torch.tensor([500], dtype=torch.int32, device="cuda")
    with pkg.ops.count_flops() as fc:
        net.encoder_stack(x, t)
    with SclkSampler() as clk:
        ms = _graph_replay_ms(lambda: net.encoder_stack(x, t), reps)
    return {"ms": round(ms, 4), "sclk_mhz": clk.summary(), "conv_gflop": round(fc.conv / 1e9, 2),
            "tflops": round(fc.total / ms / 1e9, 1),
            "frac_peak": round(fc.total / ms / 1e9 / PEAK_FP16_TFLOPS, 4),
            "config": "config 3: encoder stack 4->64/128/256/256 at 32x40x40 .. 4x5x5, 2 ResBlocks per level, "
                      "fp16, random init"}


def bench_config4(pkg, reps: int) -> dict:
    """VQ decoder at full resolution: 8x32x40x40 latent -> 1x128x160x160 volume, channels
    256/128/64/32, two nearest-2x upsamplings, single-head mid attention over 51,200
    tokens at head width 256."""
    import torch

    w, kw = pkg.vq.vq_decoder_state_dict(latent_channels=8, levels=[(3, 256, True), (2, 128, True), (1, 64, False),
                                                                    (0, 32, False)],
                                         mid_channels=256, mid_attention=True, seed=0)
    dec = pkg.vq.VqDecoder(_half(w), **kw)
    rng = np.random.default_rng(0)
    z = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 8)).astype(np.float16)).cuda()
    with pkg.ops.count_flops() as fc:
        y = dec.decode(z, quantize=False)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (1, 128, 160, 160, 1)
    del y
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    dec.decode(z, quantize=False)
    torch.cuda.synchronize()
    with SclkSampler() as clk:
        start.record()
        for _ in range(reps):
            dec.decode(z, quantize=False)
        end.record()
        torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return {"ms": round(ms, 3), "sclk_mhz": clk.summary(), "conv_gflop": round(fc.conv / 1e9, 1),
            "attention_gflop": round(fc.attention / 1e9, 1),
            "tflops": round(fc.total / ms / 1e9, 1), "frac_peak": round(fc.total / ms / 1e9 / PEAK_FP16_TFLOPS, 4),
            "config": "config 4: VQ decoder 8x32x40x40 -> 1x128x160x160, channels 256/128/64/32, mid attention "
                      "51,200 tokens x 256, fp16, random init, eager launches"}


def ldm_alphas_cumprod(n: int = 1000) -> np.ndarray:
    """The LDM 'linear' schedule (sqrt-spaced betas 0.00085 .. 0.012), stored in fp16 as
    the LINet checkpoint stores it."""
    betas = np.linspace(0.00085 ** 0.5, 0.012 ** 0.5, n, dtype=np.float64) ** 2
    return np.cumprod(1.0 - betas).astype(np.float16)


def bench_config5(pkg, steps: int = 200) -> dict:
    """One full conditioned LINet-style denoise step (UNet 9 -> 4 channels at 32x40x40,
    levels 64/128/256/256, self + cross attention at the two lowest levels and the middle,
    77x768 context), DDIM, ``steps`` steps replayed from one captured step graph."""
    import torch

    cfg = pkg.unet.UnetConfig(64, 2, (4, 8), (1, 2, 4, 4), 32, False)
    net = pkg.unet.LdmUnet(_half(pkg.unet.unet_state_dict(cfg, in_channels=9, out_channels=4, context_dim=768,
                                                          seed=0)), cfg)
    rng = np.random.default_rng(0)
    dev = torch.device("cuda")
    ctx = torch.from_numpy(rng.standard_normal((1, 77, 768)).astype(np.float16)).to(dev)
    cond = torch.from_numpy(rng.standard_normal((1, 32, 40, 40, 4)).astype(np.float32)).to(dev)
    mask = np.zeros((1, 32, 40, 40), np.float32)
    d0, h0, w0 = rng.integers(0, 32 - 6), rng.integers(0, 40 - 8), rng.integers(0, 40 - 8)
    mask[0, d0:d0 + 6, h0:h0 + 8, w0:w0 + 8] = (rng.random((6, 8, 8)) < 0.05).astype(np.float32)
    sampler = pkg.sampling.DdimSampler(ldm_alphas_cumprod(), steps)
    prep = sampler.prepare(net.prepare_denoiser(ctx), cond, torch.from_numpy(mask).to(dev),
                           masked_conditioning=True)
    g = torch.Generator(device=dev).manual_seed(0)
    init = torch.randn((1, 32, 40, 40, 4), generator=g, device=dev)
    noise = torch.randn((prep.num_steps, 1, 32, 40, 40, 4), generator=g, device=dev)
    prep.set_noise(init, noise)
    with pkg.ops.count_flops() as fc:
        prep.denoiser(prep.net_in, prep.t)
    torch.cuda.synchronize()
    prep.capture()
    prep.set_noise(init, noise)
    prep.run()  # warm replay
    torch.cuda.synchronize()
    totals = []
    clk = SclkSampler().__enter__()
    for _ in range(CONFIG5_RUNS):
        prep.set_noise(init, noise)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        out = prep.run()
        end.record()
        torch.cuda.synchronize()
        totals.append(start.elapsed_time(end))
        assert bool(torch.isfinite(out).all())
    clk.__exit__(None, None, None)
    total = float(np.median(totals))
    per = total / prep.num_steps
    return {"ms_per_step": round(per, 4), "total_ms": round(total, 2), "steps": prep.num_steps,
            "sclk_mhz": clk.summary(),
            "total_ms_runs": [round(t, 2) for t in totals],
            "step_gflop": round(fc.total / 1e9, 1), "step_conv_gflop": round(fc.conv / 1e9, 1),
            "step_attention_gflop": round(fc.attention / 1e9, 2),
            "tflops": round(fc.total / per / 1e9, 1), "frac_peak": round(fc.total / per / 1e9 / PEAK_FP16_TFLOPS, 4),
            "config": "config 5: LINet-style UNet 9->4 ch at 32x40x40, 64/128/256/256, 2 ResBlocks/level, "
                      "self+cross attention at the 8x10x10 and 4x5x5 levels (heads of 32), 77x768 context, fp16 random init, "
                      f"DDIM {prep.num_steps} steps, one HIP graph per step; total_ms is the median of "
                      f"{CONFIG5_RUNS} runs"}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    import torch

    n = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(n)
    return torch.get_num_threads()


def cpu_baseline_conv(x, w, b, budget_s: float = 10.0) -> dict:
    """The headline CPU baseline: torch CPU fp32 ``F.conv3d`` (channels-last-3d input) of the
    same seeded config-1 tensors on the host cores -- the stand-in for the reference's
    ``mx.cpu`` path, which needs macOS arm64 -- repeated full config-1 convolutions until
    ``budget_s`` seconds have elapsed."""
    import torch
    import torch.nn.functional as F

    cores = _cpu_threads()
    xc = x.float().cpu().permute(0, 4, 1, 2, 3).contiguous(memory_format=torch.channels_last_3d)
    wc, bc = w.float().cpu(), b.float().cpu()
    n = 0
    with torch.no_grad():
        F.conv3d(xc, wc, bc, padding=1)
        t0 = time.perf_counter()
        while True:
            F.conv3d(xc, wc, bc, padding=1)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    flop = 2.0 * 51200 * 64 * 64 * 27
    return {"value": round(flop * n / el / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{n} full config-1 convolutions in {el:.1f} s: torch {torch.__version__} CPU fp32 F.conv3d "
                      f"(channels_last_3d) on {cores} threads of a {cpu_model()}; a stand-in for the reference's "
                      "MLX mx.cpu path, which needs macOS arm64"}


def cpu_oracle_conv(x, w, b, budget_s: float = 5.0) -> dict:
    """The float64 oracle conv (oracle/conv.py, per-tap BLAS products) on the host cores,
    repeated full config-1 convolutions until ``budget_s`` seconds have elapsed."""
    from oracle import conv as ocv

    xn = x.float().cpu().numpy().astype(np.float64).transpose(0, 4, 1, 2, 3)
    wn = w.float().cpu().numpy().astype(np.float64)
    bn = b.float().cpu().numpy().astype(np.float64)
    ocv.conv3d(xn[:, :, :4], wn, bn)  # warm BLAS
    n, t0 = 0, time.perf_counter()
    while True:
        ocv.conv3d(xn, wn, bn)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    flop = 2.0 * 51200 * 64 * 64 * 27
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(flop * n / el / 1e12, 4), "unit": "TFLOP/s", "threads": threads,
            "sample": f"{n} full config-1 convolutions (float64 NumPy oracle) in {el:.1f} s"}


def cpu_torch_attention(qkv) -> dict:
    """torch CPU fp32 ``F.scaled_dot_product_attention`` on config 2's self-attention
    tensors: median of 5 timed calls after one warm-up."""
    import torch
    import torch.nn.functional as F

    cores = _cpu_threads()
    q, k, v = (t.float().cpu() for t in qkv)
    with torch.no_grad():
        F.scaled_dot_product_attention(q, k, v, scale=0.125)
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            F.scaled_dot_product_attention(q, k, v, scale=0.125)
            ts.append(time.perf_counter() - t0)
    ta = float(np.median(ts))
    return {"self_attention_tflops": round(4.0 * 8 * 1600 * 1600 * 64 / ta / 1e12, 4),
            "self_attention_ms": round(ta * 1e3, 2), "cores": cores}


def cpu_models(pkg) -> dict:
    """Configs 3, 4 and 5 on the host cores in torch CPU fp32 (oracle/torch_cpu.py: the same
    layer graphs, the same seeded weights and inputs as the GPU runs): config 3 the median
    of 3 runs, config 5 two UNet forwards (the DDIM update's elementwise work is left out)
    extrapolated to 200 steps, config 4 one decode."""
    import torch

    from oracle import torch_cpu as tcpu
    from oracle import unet as oun

    cores = _cpu_threads()
    out = {"cores": cores, "cpu": cpu_model(),
           "note": "torch CPU fp32 (not MLX: the reference's mx.cpu path needs macOS arm64)"}
    rng = np.random.default_rng(0)
    cfg3 = oun.UnetConfig(64, 2, (), (1, 2, 4, 4), 32, True)
    w3 = _half(pkg.unet.unet_state_dict(pkg.unet.UnetConfig(64, 2, (), (1, 2, 4, 4), 32, True), in_channels=4,
                                        out_channels=4, context_dim=None, seed=0))
    net3 = tcpu.TorchUnet(w3, cfg3)
    x3 = rng.standard_normal((1, 4, 32, 40, 40)).astype(np.float32)
    t = np.array([500], np.int32)
    net3.encoder_stack(x3, t)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        net3.encoder_stack(x3, t)
        ts.append(time.perf_counter() - t0)
    out["config3_ms"] = round(1e3 * float(np.median(ts)), 1)

    cfg5 = oun.UnetConfig(64, 2, (4, 8), (1, 2, 4, 4), 32, False)
    w5 = _half(pkg.unet.unet_state_dict(pkg.unet.UnetConfig(64, 2, (4, 8), (1, 2, 4, 4), 32, False), in_channels=9,
                                        out_channels=4, context_dim=768, seed=0))
    net5 = tcpu.TorchUnet(w5, cfg5)
    x5 = rng.standard_normal((1, 9, 32, 40, 40)).astype(np.float32)
    ctx = rng.standard_normal((1, 77, 768)).astype(np.float32)
    net5.forward(x5, np.array([996], np.int32), ctx)
    t0 = time.perf_counter()
    for step_t in (996, 991):
        net5.forward(x5, np.array([step_t], np.int32), ctx)
    per = (time.perf_counter() - t0) / 2
    out["config5_ms_per_step"] = round(per * 1e3, 1)
    out["config5_200_steps_s_extrapolated"] = round(per * 200, 1)

    w4, kw = pkg.vq.vq_decoder_state_dict(latent_channels=8, levels=[(3, 256, True), (2, 128, True), (1, 64, False),
                                                                     (0, 32, False)],
                                          mid_channels=256, mid_attention=True, seed=0)
    dec = tcpu.TorchVqDecoder(_half(w4), levels=kw["levels"], upsample_levels=kw["upsample_levels"])
    z = rng.standard_normal((1, 8, 32, 40, 40)).astype(np.float32)
    t0 = time.perf_counter()
    y = dec.decode(z)
    out["config4_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    assert tuple(y.shape) == (1, 1, 128, 160, 160)
    del y
    torch.set_num_threads(cores)
    return out


def copy_calibration(mib: int = 512, reps: int = 3) -> None:
    """``reps`` plain device copies of ``mib`` MiB (larger than the 256 MiB last-level
    cache): each reads and writes exactly ``mib`` MiB of HBM, so the counters these
    launches report give the counter-to-byte factors."""
    import torch

    src = torch.ones(mib * 2 ** 20 // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-model", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 512 MiB device copy (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--settle", type=float, default=SETTLE_S[0],
                    help="seconds of untimed replays before each figure (0.05 for profiling runs)")
    ap.add_argument("--only", type=int, choices=(3, 4, 5),
                    help="run just model config 3, 4 or 5 and print its figures (profiling runs)")
    args = ap.parse_args()
    SETTLE_S[0] = args.settle
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(collectives and sharding are out of scope); run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    torch.cuda.synchronize()
    if args.only is not None:
        run = {3: lambda: bench_config3(pkg, max(args.steps // 5, 5)), 4: lambda: bench_config4(pkg, 3),
               5: lambda: bench_config5(pkg, args.steps)}[args.only]
        print(json.dumps(run()))
        if args.copy_calibration:
            copy_calibration()
        return 0
    conv = bench_conv(pkg, args.steps, args.warmup)
    traffic, traffic_src = profiled_traffic()
    att = bench_attention(pkg, args.steps, args.warmup)
    if args.copy_calibration:
        copy_calibration()
    line = {
        "metric": METRIC,
        "value": round(conv["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(conv["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config 1: conv3d 3x3x3 stride 1 pad 1, NDHWC fp16, N=1, C_in=C_out=64, "
                               "D x H x W = 32 x 40 x 40, seed 0", "global_batch": 1},
        "sclk_mhz": conv["sclk_mhz"],
        "roofline": {"bound": "mfma", "achieved": round(conv["tflops"], 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(conv["tflops"] / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src},
        "attention": {
            "self_tflops": round(att["self"]["tflops"], 2), "self_ms": round(att["self"]["ms"], 5),
            "self_frac_peak": round(att["self"]["frac_peak"], 4),
            "cross_tflops": round(att["cross"]["tflops"], 2), "cross_ms": round(att["cross"]["ms"], 5),
            "cross_gbs": round(att["cross"]["gbs"], 1),
            "self_sclk_mhz": att["self"]["sclk_mhz"], "cross_sclk_mhz": att["cross"]["sclk_mhz"],
            "config": "config 2: fp16, B=1, 8 heads x 64, 1600 queries; self 1600 keys, cross 77 keys "
                      "(context 77x768 projected by to_k/to_v once, outside the timed launches)"},
    }
    line["source_order"] = bench_source(pkg, args.steps, args.warmup, not args.skip_cpu)
    if not args.skip_model:
        line["unet_block_stack"] = bench_config3(pkg, max(args.steps // 5, 5))
        line["vq_decoder"] = bench_config4(pkg, 3)
        line["denoise_step"] = bench_config5(pkg, 200)
    if not args.skip_cpu:
        line["cpu_baseline"] = cpu_baseline_conv(conv["x"], conv["w"], conv["b"])
        line["cpu_baseline_attention"] = cpu_torch_attention(att["_tensors"])
        line["cpu_oracle_float64"] = cpu_oracle_conv(conv["x"], conv["w"], conv["b"])
        if not args.skip_model:
            line["cpu_models"] = cpu_models(pkg)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
