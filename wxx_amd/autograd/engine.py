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


class SliceGrad:
    """A gradient that is zero outside slices of a tensor of ``shape``: each
    part ``(dim, start, g)`` holds ``g`` at ``[start, start + len)`` along
    ``dim``.  The backward of narrow / chunk / a basic slice returns one;
    gradients reaching the same tensor from several slices are merged here
    and written into one buffer when the tensor's backward runs, instead of
    a zero-filled full-size tensor per slice added together.  The values
    are those of the dense sum (x + 0 == x), up to the sign of a zero."""

    __slots__ = ("shape", "parts")

    def __init__(self, shape, dim, start, g):
        self.shape = list(shape)
        self.parts = [(dim, start, g)]

    def merged(self, other):
        out = SliceGrad.__new__(SliceGrad)
        out.shape = self.shape
        out.parts = self.parts + other.parts
        return out

    def dense(self):
        from ..Tensor import Tensor
        from ..functional._common import empty

        dims = {d for d, _, _ in self.parts}
        disjoint = covered = False
        if len(dims) == 1:
            (d,) = dims
            spans = sorted((st, st + g.shape[d]) for _, st, g in self.parts)
            disjoint = all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
            covered = disjoint and spans[0][0] == 0 and spans[-1][1] == self.shape[d] and all(
                a[1] == b[0] for a, b in zip(spans, spans[1:]))
        if disjoint:
            out = empty(self.shape) if covered else Tensor(self.shape, value=0.0)
            for d, st, g in self.parts:
                functional.assign(out.narrow(d, st, g.shape[d]), g)
            return out
        # overlapping slices: add each part into a zero tensor, in arrival order
        out = Tensor(self.shape, value=0.0)
        for d, st, g in self.parts:
            view = out.narrow(d, st, g.shape[d])
            functional.assign(view, functional.pointwise(view, g, 0))
        return out


def _dense(g):
    return g.dense() if isinstance(g, SliceGrad) else g


def _add(acc, grad):
    if isinstance(acc, SliceGrad) and isinstance(grad, SliceGrad) and acc.shape == grad.shape:
        return acc.merged(grad)
    acc, grad = _dense(acc), _dense(grad)
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
            g = _dense(g)
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
