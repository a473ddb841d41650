"""wxx_amd: the wxx tensor library on a native MI355X (gfx950) HIP backend.

``import wxx_amd as wxx`` exposes the reference package's surface
(reference src/wxx/__init__.py:1-17): ``Tensor``, ``Parameter``,
``functional``, ``autograd``, ``nn``, ``backend``, ``serialization``,
``save``/``load``.  Importing does not touch the GPU; the device opens on the
first allocation.
"""

from .Tensor import Parameter, Tensor
from . import autograd, backend, functional, graphs, nn, serialization
from .graphs import StepGraph
from .backend.device import get_device
from .serialization import load, save

__all__ = ["Tensor", "Parameter", "functional", "autograd", "backend", "nn", "serialization",
           "get_device", "save", "load"]
