"""HIP runtime for wxx_amd: ctypes binding, device buffers, the stream and
the autograd mode flag (counterpart of reference src/wxx/backend/__init__.py)."""

from . import compat
from .context import inferenceMode
from .device import (
    CommandStream,
    DeviceBuffer,
    DeviceBufferPool,
    HIPContext,
    device_available,
    ensure_device,
    get_buffer_pool,
    get_cmd_buffer,
    get_ctx,
    get_device,
    synchronize,
)

__all__ = [
    "compat",
    "inferenceMode",
    "CommandStream",
    "DeviceBuffer",
    "DeviceBufferPool",
    "HIPContext",
    "device_available",
    "ensure_device",
    "get_buffer_pool",
    "get_cmd_buffer",
    "get_ctx",
    "get_device",
    "synchronize",
]
