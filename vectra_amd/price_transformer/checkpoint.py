"""Model checkpoints: weights as safetensors, architecture as JSON.

Same files and layout as the reference's models/training/checkpoint.py:
`model.safetensors` (fp32 state dict) and `model_config.json`
({"model": ModelConfig fields, "metadata": {...}}).  safetensors holds raw
tensors only, so loading a checkpoint executes nothing from the file.
"""

import dataclasses
import json
import os

from safetensors import torch as safetensors_torch
import torch

from vectra_amd.price_transformer import model as model_lib

WEIGHTS = 'model.safetensors'
CONFIG = 'model_config.json'


def save(directory: str, model: model_lib.PriceTransformer, metadata: dict | None = None) -> None:
    """Writes `directory`/{model.safetensors, model_config.json}."""
    os.makedirs(directory, exist_ok=True)
    state = {name: t.detach().float().cpu().contiguous() for name, t in model.state_dict().items()}
    safetensors_torch.save_file(state, os.path.join(directory, WEIGHTS))
    with open(os.path.join(directory, CONFIG), 'w', encoding='utf-8') as f:
        json.dump({'model': dataclasses.asdict(model.config), 'metadata': metadata or {}}, f,
                  indent=2, sort_keys=True)
        f.write('\n')


def load(directory: str, device: torch.device | str = 'cpu') -> model_lib.PriceTransformer:
    """Rebuilds the model from `directory`, in eval mode on `device`."""
    with open(os.path.join(directory, CONFIG), encoding='utf-8') as f:
        config = model_lib.ModelConfig.from_dict(json.load(f)['model'])
    model = model_lib.PriceTransformer(config)
    model.load_state_dict(safetensors_torch.load_file(os.path.join(directory, WEIGHTS)))
    return model.to(device).eval()
