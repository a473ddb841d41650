"""``.npz`` save / load of models, state_dicts and tensors (reference
src/wxx/serialization.py:1-54): one array per dotted parameter name."""

import os

import numpy as np

from .nn.module import Module


def _to_arrays(obj):
    if isinstance(obj, Module):
        obj = obj.state_dict()
    if isinstance(obj, dict):
        return {str(k): np.asarray(v.numpy() if hasattr(v, "numpy") and
                                   not isinstance(v, np.ndarray) else v)
                for k, v in obj.items()}
    if hasattr(obj, "numpy") and not isinstance(obj, np.ndarray):
        obj = obj.numpy()
    return {"tensor": np.asarray(obj)}


def save(obj, path):
    """Save a model, state_dict or tensor to ``path`` (``.npz`` appended if missing)."""
    path = str(path)
    if not path.endswith(".npz"):
        path += ".npz"
    np.savez(path, **_to_arrays(obj))
    return path


def load(path, model=None):
    """Load an ``.npz`` archive (numpy arrays only, no pickles); with ``model``
    fill its parameters and return it, else return the dict of arrays."""
    path = str(path)
    if not path.endswith(".npz") and not os.path.exists(path):
        path += ".npz"
    with np.load(path, allow_pickle=False) as data:
        state = {k: data[k] for k in data.files}
    if model is not None:
        model.load_state_dict(state)
        return model
    return state
