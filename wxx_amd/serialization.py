"""On-disk format: numpy ``.npz`` archives (reference src/wxx/serialization.py:1-54).

``save`` / ``load`` keep the reference's contract: a model (or any
``state_dict``) is stored as one array per dotted parameter name, a lone
tensor under the key ``"tensor"``, and ``load(path, model)`` fills the model
and returns it.  Archives are read with ``allow_pickle=False``: they hold
plain arrays only.

``save_checkpoint`` / ``load_checkpoint`` add what the reference cannot
persist: the AdamW moments and step count and the LR scheduler position, in
the same archive as the weights, under the prefixes ``model.``, ``optim.``
and ``sched.``, so that a resumed run continues bit for bit.
"""

import os

import numpy as np

_PREFIXES = ("model.", "optim.", "sched.")


def _npz_path(path, reading=False):
    path = str(path)
    if path.endswith(".npz") or (reading and os.path.exists(path)):
        return path
    return path + ".npz"


def _as_array(v):
    if isinstance(v, np.ndarray):
        return v
    if hasattr(v, "numpy"):  # a device Tensor
        return np.asarray(v.numpy())
    return np.asarray(v)


def _flatten(obj):
    """Name -> array for a model / optimizer / scheduler, dict or tensor."""
    if hasattr(obj, "state_dict") and callable(obj.state_dict):
        obj = obj.state_dict()
    if isinstance(obj, dict):
        return {str(k): _as_array(v) for k, v in obj.items()}
    return {"tensor": _as_array(obj)}


def _read(path):
    with np.load(_npz_path(path, reading=True), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def save(obj, path):
    """Write a model, optimizer, scheduler, state_dict or tensor to ``path``
    (``.npz`` appended when missing); returns the path written."""
    out = _npz_path(path)
    np.savez(out, **_flatten(obj))
    return out


def load(path, model=None):
    """Read an archive.  With ``model`` (anything with ``load_state_dict``)
    the arrays are loaded into it and it is returned; otherwise the dict of
    arrays is returned."""
    arrays = _read(path)
    if model is None:
        return arrays
    model.load_state_dict(arrays)
    return model


def save_checkpoint(path, model, optimizer=None, scheduler=None):
    """Weights, optimizer state and scheduler position in one archive."""
    arrays = {}
    for prefix, part in zip(_PREFIXES, (model, optimizer, scheduler)):
        if part is not None:
            arrays.update({prefix + k: v for k, v in _flatten(part).items()})
    out = _npz_path(path)
    np.savez(out, **arrays)
    return out


def load_checkpoint(path, model, optimizer=None, scheduler=None):
    """Restore what :func:`save_checkpoint` wrote into the given objects; a
    part requested but absent from the archive raises ``KeyError``."""
    arrays = _read(path)
    for prefix, part in zip(_PREFIXES, (model, optimizer, scheduler)):
        if part is None:
            continue
        sub = {k[len(prefix):]: v for k, v in arrays.items() if k.startswith(prefix)}
        if not sub:
            raise KeyError(f"{path}: no '{prefix[:-1]}' entries in the checkpoint")
        part.load_state_dict(sub)
    return model


__all__ = ["save", "load", "save_checkpoint", "load_checkpoint"]
