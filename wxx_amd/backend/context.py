"""Global autograd recording mode (mirrors reference src/wxx/backend/context.py:1-15).

``MODE == 0`` records the autograd graph (training); ``MODE == 1`` is
inference: autograd functions compute without recording, dropout is the
identity and batch norm uses running statistics.
"""

MODE = 0


class inferenceMode:
    """Context manager that switches ``MODE`` to 1 and restores it on exit."""

    def __enter__(self):
        global MODE
        self._prev = MODE
        MODE = 1
        return MODE

    def __exit__(self, exc_type, exc_val, exc_tb):
        global MODE
        MODE = self._prev
        return False
