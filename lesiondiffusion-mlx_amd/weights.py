"""Converted-weight bundle: one ``model.safetensors`` whose tensor names carry a stage
prefix (``lmnet.``, ``linet.``, ``vq.``, ...), as the reference ships it
(src/lesiondiffusion_mlx/medmlx.py:93-94, 1539-1602).

``require_weights`` validates the bundle from its header alone; ``load_stage`` reads one
stage's tensors -- only those, straight from the file, without materialising the rest --
strips the stage prefix, optionally keeps only some component prefixes, and casts. The
result is a dict keyed by upstream names that ``LdmUnet`` and ``VqDecoder`` take as their
weights. Reading is host code (safetensors' own reader, which executes nothing from the
file); tensors land on ``device`` in ``dtype``.
"""

from __future__ import annotations

from os import PathLike
from pathlib import Path

import torch

WEIGHT_FILE = "model.safetensors"
# Stages of the converted bundle (medmlx.py:93); the text encoders are outside this build,
# but a complete bundle still carries them.
WEIGHT_STAGES = ("lmnet", "linet", "vq", "lmnet_text", "linet_text")
# Source-mode inference does not condition LINet on text (medmlx.py:94).
SOURCE_INFERENCE_STAGES = tuple(name for name in WEIGHT_STAGES if name != "linet_text")


class WeightsNotReadyError(RuntimeError):
    """The converted weight bundle is missing, unreadable or lacks a required stage."""


def require_weights(path: str | PathLike, *, inference_mode: str = "conditioned") -> Path:
    """Check that ``path`` is a directory holding a readable ``model.safetensors`` with every
    stage the inference mode needs (``source``: all but ``linet_text``); only the header is
    read (require_weights, medmlx.py:1539-1582). Returns the directory."""
    directory = Path(path).expanduser()
    if not directory.is_dir():
        raise WeightsNotReadyError(f"weights directory {directory} does not exist")
    packed = directory / WEIGHT_FILE
    if not packed.is_file():
        raise WeightsNotReadyError(f"{packed} is missing")
    from safetensors import SafetensorError, safe_open

    try:
        with safe_open(str(packed), framework="pt") as f:
            names = list(f.keys())
    except (SafetensorError, OSError) as exc:
        raise WeightsNotReadyError(f"{packed} is not a readable safetensors file: {exc}") from exc
    present = {key.split(".", 1)[0] for key in names}
    stages = SOURCE_INFERENCE_STAGES if inference_mode == "source" else WEIGHT_STAGES
    missing = [name for name in stages if name not in present]
    if missing:
        raise WeightsNotReadyError(f"{packed} has no tensors for stage(s) {', '.join(missing)}")
    return directory


def load_stage(directory: str | PathLike, name: str, *, dtype: torch.dtype,
               prefixes: tuple[str, ...] | None = None, device: torch.device | str = "cuda") -> dict[str, torch.Tensor]:
    """The tensors of stage ``name`` with the ``name.`` prefix removed, cast to ``dtype`` on
    ``device``; with ``prefixes``, only names (after the stage prefix) that start with one
    of them (load_stage, medmlx.py:1585-1602). Tensors of other stages are never read."""
    from safetensors import safe_open

    stage = name + "."
    out: dict[str, torch.Tensor] = {}
    with safe_open(str(Path(directory) / WEIGHT_FILE), framework="pt") as f:
        for key in f.keys():
            if not key.startswith(stage):
                continue
            short = key[len(stage):]
            if prefixes is not None and not short.startswith(prefixes):
                continue
            out[short] = f.get_tensor(key).to(device=device, dtype=dtype)
    return out


__all__ = ["WEIGHT_FILE", "WEIGHT_STAGES", "SOURCE_INFERENCE_STAGES", "WeightsNotReadyError", "require_weights",
           "load_stage"]
