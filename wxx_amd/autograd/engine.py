"""Reverse-mode sweep (the behaviour of reference src/wxx/Tensor.py:430-517).

Topologically orders the tensors that require grad, then walks them in
reverse under inference mode, calling each creator's ``backward`` and summing
gradients per tensor.  Leaf tensors (no creator) receive ``.grad``.  Nodes
that receive no gradient are unlinked so their activations can be freed.

Gradient sums are formed out of place (``a + b`` into a new buffer) rather
than by in-place accumulation: a backward may hand the same gradient object
to two inputs (``x + y`` passes ``g`` to both), and an in-place add into one
would silently change the other.
"""

from .. import functional
from ..backend.context import inferenceMode


def _add(acc, grad):
    if getattr(acc, "type", "f32") == "c64":
        return functional.complex_add(acc, grad)
    return functional.pointwise(acc, grad, 0)


def run_backward(root):
    from ..Tensor import Tensor

    if not root.requires_grad:
        raise RuntimeError("cannot call backward on a tensor that does not require gradients")
    if root.grad is None:
        root.grad = Tensor(shape=root.shape, dtype=root.type)

    order = []
    seen = set()
    stack = [(root, False)]
    while stack:
        t, expanded = stack.pop()
        if expanded:
            order.append(t)
            continue
        if id(t) in seen or not isinstance(t, Tensor) or not t.requires_grad:
            continue
        seen.add(id(t))
        stack.append((t, True))
        if t.creator is not None:
            for parent in reversed(t.creator.inputs or []):
                if isinstance(parent, Tensor) and parent.requires_grad and id(parent) not in seen:
                    stack.append((parent, False))

    with inferenceMode():
        grads = {id(root): root.grad}
        while order:
            t = order.pop()
            g = grads.pop(id(t), None)
            if g is None:
                if t.creator is not None:
                    t.creator.inputs = None
                    t.creator = None
                continue
            fn = t.creator
            if fn is not None:
                pg = fn.backward(g)
                if len(fn.inputs) == 1:
                    pg = (pg,)
                elif not isinstance(pg, (tuple, list)):
                    raise TypeError(f"{type(fn).__name__}.backward must return one gradient per input")
                if len(pg) != len(fn.inputs):
                    raise RuntimeError(
                        f"{type(fn).__name__}.backward returned {len(pg)} gradients for "
                        f"{len(fn.inputs)} inputs"
                    )
                for parent, pgrad in zip(fn.inputs, pg):
                    if parent is None or pgrad is None or not getattr(parent, "requires_grad", False):
                        continue
                    prev = grads.get(id(parent))
                    grads[id(parent)] = pgrad if prev is None else _add(prev, pgrad)
                fn.inputs = None
                t.creator = None
            elif t is not root:
                t.grad = g if t.grad is None else _add(t.grad, g)
