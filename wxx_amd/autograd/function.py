"""Base class of the differentiable ops (reference src/wxx/autograd/function.py:6-49).

A ``Function`` is built with the tensors it consumes, records them in
``inputs`` (with ``needs_input_grad`` flags taken from ``requires_grad`` while
the global mode records, all ``False`` in inference mode), computes its output
in ``forward`` and attaches itself as the output's ``creator``; ``backward``
maps the output gradient to one gradient per input (``None`` where not needed).
"""

import weakref

from ..backend import context


class Function:
    def __init__(self, *inputs):
        from ..Tensor import Tensor

        self.inputs = list(inputs)
        recording = context.MODE == 0
        self.needs_input_grad = [
            bool(recording and isinstance(t, Tensor) and t.requires_grad) for t in inputs
        ]

    def forward(self, *args):
        raise NotImplementedError

    def backward(self, grad_output):
        raise NotImplementedError

    def hold_output(self, out):
        """Keep ``out`` reachable for backward without a creator<->output cycle."""
        self._out_ref = weakref.ref(out)

    def held_output(self):
        ref = getattr(self, "_out_ref", None)
        self._out_ref = None
        return None if ref is None else ref()

    def attach(self, out, **saved):
        """Make ``self`` the creator of ``out`` when recording; save tensors for backward."""
        if out.requires_grad and context.MODE == 0:
            out.creator = self
            for k, v in saved.items():
                setattr(self, k, v)
        return out
