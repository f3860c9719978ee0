"""Checkpoint ingest: the reference's checkpoint files -> a TinyTransformer on the HIP path.

``load_model_from_checkpoint`` follows ``src/eval.py:881-951`` (the model is built from the
checkpoint's ``model_config``, else from ``config["model_size"]``, else with the defaults, and
the weights come from ``model_state_dict`` / ``model_state`` / ``model`` / the file itself), with
two differences:

* Files are read without executing anything they contain: ``torch.load(weights_only=True)``
  (the reference passes ``weights_only=False``).  The reference's training checkpoints
  (``src/train.py:938-950``) also hold ``np.random.get_state()`` in their ``rng_state``; such a
  file is read with numpy's array and dtype reconstructors allow-listed for the restricted
  unpickler -- data constructors only, still ``weights_only=True``.  ``.safetensors`` files
  hold the state dict, with the model config as JSON in the ``model_config`` metadata entry.
* On a GPU the kernels' weight operands (bf16 tiles in the MFMA layout, with the low parts of
  fp32 weights for an fp32 model) are built once at load, so the first generation does not pay
  for them.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from .transformer import MODEL_SIZES, TinyTransformer, create_model

_STATE_KEYS = ("model_state_dict", "model_state", "model")


def _numpy_safe_globals() -> list:
    """Reconstructors of numpy arrays and dtypes (for np.random.get_state() inside rng_state)."""
    core = getattr(np, "_core", None) or np.core
    allowed = [core.multiarray._reconstruct, np.ndarray, np.dtype]
    for t in (np.uint32, np.int64, np.float64, np.uint8):
        allowed.append(type(np.dtype(t)))
    return allowed


def read_checkpoint(path: str | Path) -> dict:
    """The checkpoint as a dict, read with loaders that execute nothing from the file."""
    path = Path(path)
    if path.suffix == ".safetensors":
        from safetensors import safe_open

        with safe_open(str(path), framework="pt") as f:
            meta = f.metadata() or {}
            state = {k: f.get_tensor(k) for k in f.keys()}
        ckpt: dict = {"model_state": state}
        if "model_config" in meta:
            ckpt["model_config"] = json.loads(meta["model_config"])
        return ckpt
    try:
        obj = torch.load(path, map_location="cpu", weights_only=True)
    except Exception as first:  # noqa: BLE001 - retried with the numpy reconstructors allowed
        try:
            with torch.serialization.safe_globals(_numpy_safe_globals()):
                obj = torch.load(path, map_location="cpu", weights_only=True)
        except Exception:
            raise RuntimeError(
                f"{path}: not loadable with torch.load(weights_only=True) ({first}); this "
                "build never unpickles arbitrary objects") from first
    if not isinstance(obj, dict):
        raise RuntimeError(f"{path}: expected a dict checkpoint, got {type(obj).__name__}")
    return obj


def model_from_checkpoint_dict(ckpt: dict) -> TinyTransformer:
    """Build the model the way src/eval.py:898-928 does and load its weights (:930-940)."""
    if "model_config" in ckpt:
        model = create_model(**dict(ckpt["model_config"]))
    elif isinstance(ckpt.get("config"), dict) and "model_size" in ckpt["config"]:
        size = ckpt["config"]["model_size"]
        model = create_model(**MODEL_SIZES.get(size, MODEL_SIZES["small"]))
    else:
        model = create_model()
    for key in _STATE_KEYS:
        if key in ckpt:
            state = ckpt[key]
            break
    else:
        state = ckpt
    model.load_state_dict(state)
    return model


def load_model_from_checkpoint(checkpoint_path: str | Path, device: torch.device | str,
                               return_task_id_map: bool = False):
    """``load_model_from_checkpoint`` of src/eval.py:881-951 on the HIP path: the model in eval
    mode on ``device`` (and the checkpoint's task_id -> example_id map when asked)."""
    ckpt = read_checkpoint(checkpoint_path)
    model = model_from_checkpoint_dict(ckpt).to(device).eval()
    dev = torch.device(device)
    if dev.type == "cuda":
        from .engine import engine_for

        engine_for(model).packed(dev)
    if return_task_id_map:
        return model, ckpt.get("task_id_to_example_id")
    return model


def save_safetensors(model: TinyTransformer, path: str | Path) -> None:
    """The model's state dict as safetensors with its config in the metadata (the format
    ``read_checkpoint`` reads back without any unpickling)."""
    from dataclasses import asdict

    from safetensors.torch import save_file

    state = {k: v.detach().contiguous().cpu() for k, v in model.state_dict().items()}
    save_file(state, str(path), metadata={"model_config": json.dumps(asdict(model.config))})
