"""The converted-weight bundle (model.safetensors with stage prefixes): header validation and
stage loading on the CPU (the reference's require_weights / load_stage,
src/lesiondiffusion_mlx/medmlx.py:1539-1602, and its missing / corrupt bundle cases,
tests/test_medmlx.py:330-357), and on the GPU a UNet built from a loaded stage computing
exactly what the same weights give when passed directly."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors.numpy import save_file

SMALL_UNET = dict(model_channels=16, num_res_blocks=1, attention_resolutions=(2,), channel_mult=(1, 2),
                  num_head_channels=16, skip_context=False)


def _bundle(pkg, directory, *, drop_stage: str | None = None):
    """A bundle with every stage: a small LINet-style UNet under ``linet.``, a VQ decoder
    with its codebook under ``vq.``, and stand-in tensors for the other stages."""
    cfg = pkg.unet.UnetConfig(**SMALL_UNET)
    unet = pkg.unet.unet_state_dict(cfg, in_channels=5, out_channels=4, context_dim=12, seed=7)
    vq, _ = pkg.vq.vq_decoder_state_dict(latent_channels=4, levels=[(1, 16, True), (0, 8, False)], mid_channels=16,
                                         mid_attention=False, seed=8)
    vq["quantize.embedding.weight"] = np.random.default_rng(9).standard_normal((32, 4)).astype(np.float32)
    tensors = {f"linet.{k}": v for k, v in unet.items()}
    tensors.update({f"vq.{k}": v for k, v in vq.items()})
    for stage in ("lmnet", "lmnet_text", "linet_text"):
        tensors[f"{stage}.stand_in.weight"] = np.ones((2, 2), np.float32)
    if drop_stage:
        tensors = {k: v for k, v in tensors.items() if not k.startswith(drop_stage + ".")}
    directory.mkdir(parents=True, exist_ok=True)
    save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, str(directory / "model.safetensors"))
    return unet, vq


def test_require_weights_accepts_a_complete_bundle_and_names_what_is_missing(pkg, tmp_path) -> None:
    w = pkg.weights
    _bundle(pkg, tmp_path / "ok")
    assert w.require_weights(tmp_path / "ok") == tmp_path / "ok"
    with pytest.raises(w.WeightsNotReadyError, match="does not exist"):
        w.require_weights(tmp_path / "absent")
    (tmp_path / "empty").mkdir()
    with pytest.raises(w.WeightsNotReadyError, match="missing"):
        w.require_weights(tmp_path / "empty")
    _bundle(pkg, tmp_path / "no_linet_text", drop_stage="linet_text")
    with pytest.raises(w.WeightsNotReadyError, match="linet_text"):
        w.require_weights(tmp_path / "no_linet_text", inference_mode="conditioned")
    # source mode does not condition LINet on text
    assert w.require_weights(tmp_path / "no_linet_text", inference_mode="source") == tmp_path / "no_linet_text"
    (tmp_path / "corrupt").mkdir()
    (tmp_path / "corrupt" / "model.safetensors").write_bytes(b"not a safetensors header")
    with pytest.raises(w.WeightsNotReadyError, match="not a readable"):
        w.require_weights(tmp_path / "corrupt")


def test_load_stage_strips_the_prefix_filters_and_casts(pkg, tmp_path) -> None:
    unet, vq = _bundle(pkg, tmp_path)
    got = pkg.weights.load_stage(tmp_path, "linet", dtype=torch.float16, device="cpu")
    assert set(got) == set(unet)
    for k, v in unet.items():
        assert got[k].dtype == torch.float16
        np.testing.assert_array_equal(got[k].numpy(), v.astype(np.float16))
    dec = pkg.weights.load_stage(tmp_path, "vq", dtype=torch.float32, device="cpu",
                                 prefixes=("decoder.", "post_quant_conv."))
    assert set(dec) == {k for k in vq if k.startswith(("decoder.", "post_quant_conv."))}
    cb = pkg.weights.load_stage(tmp_path, "vq", dtype=torch.float32, device="cpu", prefixes=("quantize.",))
    assert list(cb) == ["quantize.embedding.weight"]
    np.testing.assert_array_equal(cb["quantize.embedding.weight"].numpy(), vq["quantize.embedding.weight"])
    assert pkg.weights.load_stage(tmp_path, "lin", dtype=torch.float32, device="cpu") == {}


@pytest.mark.gpu
def test_unet_from_a_loaded_stage_equals_unet_from_the_same_weights(pkg, dev, tmp_path) -> None:
    """A LINet-style UNet whose weights come through load_stage (fp16, on the device)
    computes bit for bit what the same weights give when passed directly."""
    unet, _ = _bundle(pkg, tmp_path)
    cfg = pkg.unet.UnetConfig(**SMALL_UNET)
    loaded = pkg.unet.LdmUnet(pkg.weights.load_stage(tmp_path, "linet", dtype=torch.float16, device=dev), cfg)
    direct = pkg.unet.LdmUnet({k: v.astype(np.float16) for k, v in unet.items()}, cfg)
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((1, 5, 8, 8, 8)).astype(np.float16)).to(dev)
    ctx = torch.from_numpy(rng.standard_normal((1, 3, 12)).astype(np.float16)).to(dev)
    t = torch.tensor([321], dtype=torch.int32, device=dev)
    a, b = loaded(x, t, ctx), direct(x, t, ctx)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
