"""Differentiable matmul, views, slicing, concat and FFT / complex ops
(gradients as in reference src/wxx/autograd/utils.py:40-718).

The one departure in mechanism: when a batched activation multiplies an
unbatched weight (``(b, S, in) @ (in, out)``, every Linear layer), the
weight gradient is formed as a single GEMM with K = b*S over the flattened
activations instead of ``b`` per-batch GEMMs followed by a sum over the batch
(reference autograd/utils.py:95-102).  It is the same sum, accumulated in a
different order.
"""

import math

from .. import functional, validation
from ..backend.dispatch import _sum_to_shape
from ..Tensor import Tensor
from .engine import SliceGrad
from .function import Function


def _single_slice(index, shape):
    """``(dim, start)`` when ``index`` is one unit-step slice with every other axis full."""
    if not isinstance(index, tuple):
        index = (index,)
    if len(index) > len(shape):
        return None
    index = index + (slice(None),) * (len(shape) - len(index))
    found = None
    for axis, item in enumerate(index):
        if not isinstance(item, slice):
            return None
        start, stop, step = item.indices(shape[axis])
        if step != 1:
            return None
        if start == 0 and stop == shape[axis]:
            continue
        if found is not None:
            return None
        found = (axis, start)
    return found


def _as_matrix(t):
    """View a contiguous (..., r, c) tensor as (prod(...) * r, c)."""
    if not t.is_contiguous():
        t = t.contiguous()
    rows = math.prod(t.shape[:-1])
    out = Tensor((rows, t.shape[-1]), buffer=t.buffer, offset=t.offset, dtype=t.type)
    out._base = t
    return out


def _weight_grad(a, g, trans_a, target_shape):
    """d(B) for C = op(A) @ B with a 2-D B: A^T g over all batch rows in one GEMM."""
    if not trans_a and len(a.shape) >= 3 and len(g.shape) == len(a.shape) and len(target_shape) == 2:
        return functional.matmul_add(_as_matrix(a), _as_matrix(g), None, True, False)
    return _sum_to_shape(functional.matmul_add(a, g, None, not trans_a, False), target_shape)


# Triangular modes of the attention products under a causal mask (see
# functional.matmul_add): forward mode, and the modes of the two gradient
# products.  "scores" = Q K^T, whose entries above the diagonal the mask
# sends to probability 0 (their gradient is 0); "probs" = P V with P lower
# triangular.
_CAUSAL = {
    "scores": (1, 2, 3),  # C = Q K^T; dQ = dC K (dC lower); dK = dC^T Q
    "probs": (2, 1, 3),   # C = P V; dP = dC V^T (only below the diagonal used); dV = P^T dC
    # the same with the tiles above the diagonal left unwritten (every
    # consumer reads only the lower triangle)
    "scores_skip": (4, 2, 3),
    "probs_skip": (2, 4, 3),
}


class matmul(Function):
    def forward(self, tensor1, tensor2, transpose_a=False, transpose_b=False, causal=None):
        if causal is not None and (causal not in _CAUSAL or transpose_a
                                   or transpose_b != causal.startswith("scores")):
            raise ValueError(f"unsupported causal product {causal!r}")
        modes = _CAUSAL.get(causal, (0, 0, 0))
        out = functional.matmul_add(tensor1, tensor2, None, transpose_A=transpose_a,
                                    transpose_B=transpose_b, tri=modes[0])
        out.requires_grad = tensor1.requires_grad or tensor2.requires_grad
        return self.attach(out, tensor1=tensor1, tensor2=tensor2, transpose_a=transpose_a,
                           transpose_b=transpose_b, modes=modes)

    def backward(self, g):
        a, b = self.tensor1, self.tensor2
        ta, tb = self.transpose_a, self.transpose_b
        _, tri_a, tri_b = self.modes
        self.tensor1 = self.tensor2 = None
        ga = gb = None
        if self.needs_input_grad[0]:
            if ta:
                ga = functional.matmul_add(b, g, None, tb, True)
            else:
                ga = functional.matmul_add(g, b, None, False, not tb, tri=tri_a)
            ga = _sum_to_shape(ga, self.inputs[0].shape)
        if self.needs_input_grad[1]:
            target = tuple(self.inputs[1].shape)
            if tri_b:  # causal: both operands batched, no reduction
                gb = functional.matmul_add(g if tb else a, a if tb else g, None, True, False,
                                           tri=tri_b)
            elif tb:
                if not ta and len(a.shape) >= 3 and len(target) == 2:
                    gb = functional.matmul_add(_as_matrix(g), _as_matrix(a), None, True, False)
                else:
                    gb = _sum_to_shape(functional.matmul_add(g, a, None, True, ta), target)
            else:
                gb = _weight_grad(a, g, ta, target)
        return ga, gb


class matmuladd(Function):
    def forward(self, tensor1, tensor2, tensor3):
        out = functional.matmul_add(tensor1, tensor2, tensor3)
        out.requires_grad = any(self.needs_input_grad)
        return self.attach(out, tensor1=tensor1, tensor2=tensor2)

    def backward(self, g):
        a, b = self.tensor1, self.tensor2
        self.tensor1 = self.tensor2 = None
        ga = (_sum_to_shape(functional.matmul_add(g, b, None, False, True), self.inputs[0].shape)
              if self.needs_input_grad[0] else None)
        gb = (_weight_grad(a, g, False, tuple(self.inputs[1].shape))
              if self.needs_input_grad[1] else None)
        gc = _sum_to_shape(g, self.inputs[2].shape) if self.needs_input_grad[2] else None
        return ga, gb, gc


class flatten(Function):
    def forward(self, tensor1, start_dim=0, end_dim=-1):
        self.shape = list(tensor1.shape)
        nd = len(self.shape)
        s = validation.normalize_dim(start_dim, nd, name="start_dim")
        e = validation.normalize_dim(end_dim, nd, name="end_dim")
        if s > e:
            raise ValueError(f"start_dim ({s}) must be <= end_dim ({e})")
        new = self.shape[:s] + [math.prod(self.shape[s:e + 1])] + self.shape[e + 1:]
        out = functional.reshape(tensor1, new)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        return functional.reshape(g, self.shape) if self.needs_input_grad[0] else None


class permute(Function):
    def forward(self, tensor1, axes):
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        axes = validation.normalize_dims(tuple(axes), len(tensor1.shape), name="axes",
                                         allow_duplicates=False)
        out = functional.permute(tensor1, *axes)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, axes=axes)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        inv = [0] * len(self.axes)
        for i, a in enumerate(self.axes):
            inv[a] = i
        return functional.permute(g, *inv)


class reshape(Function):
    def forward(self, tensor1, shape):
        out = functional.reshape(tensor1, shape)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, in_shape=list(tensor1.shape))

    def backward(self, g):
        return functional.reshape(g, self.in_shape) if self.needs_input_grad[0] else None


class narrow(Function):
    def forward(self, tensor1, dim, start, length):
        out = tensor1.narrow(dim, start, length)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, in_shape=list(tensor1.shape), in_type=tensor1.type,
                           dim=dim % len(tensor1.shape), start=start, length=length)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        if self.in_type == "f32" and g.type == "f32":
            # deferred: the engine writes the slices of one tensor into one buffer
            return SliceGrad(self.in_shape, self.dim, self.start, g)
        dx = Tensor(self.in_shape, value=0, dtype=self.in_type)
        functional.assign(dx.narrow(self.dim, self.start, self.length), g)
        return dx


class diagonal(Function):
    def forward(self, tensor1, offset, dim1, dim2):
        out = functional.diagonal(tensor1, offset, dim1, dim2)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, in_shape=list(tensor1.shape), in_type=tensor1.type,
                           offset=offset, dim1=dim1, dim2=dim2)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        dx = Tensor(self.in_shape, value=0, dtype=self.in_type)
        functional.assign(functional.diagonal(dx, self.offset, self.dim1, self.dim2), g)
        return dx


class unfold(Function):
    def forward(self, tensor1, dimension, size, step):
        out = functional.unfold(tensor1, dimension, size, step)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, in_shape=tuple(tensor1.shape), dimension=dimension, size=size,
                           step=step)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        return functional.unfolddx(g, self.in_shape, self.dimension, self.size, self.step)


class getitem(Function):
    def forward(self, tensor1, index):
        out = tensor1._basic_getitem(index)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, in_shape=list(tensor1.shape), in_type=tensor1.type, index=index)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        target = _single_slice(self.index, self.in_shape)
        if target is not None and self.in_type == "f32" and g.type == "f32":
            return SliceGrad(self.in_shape, target[0], target[1], g)
        dx = Tensor(self.in_shape, value=0, dtype=self.in_type)
        functional.assign(dx._basic_getitem(self._full_index()), g)
        return dx

    def _full_index(self):
        idx = self.index if isinstance(self.index, tuple) else (self.index,)
        return idx + (slice(None),) * (len(self.in_shape) - len(idx))


class concat(Function):
    def forward(self, tensors, dim=-1):
        if not tensors:
            raise ValueError("concat expects at least one tensor")
        rank = len(tensors[0].shape)
        dim = validation.normalize_dim(dim, rank, name="dim")
        base = list(tensors[0].shape)
        for i, t in enumerate(tensors):
            if len(t.shape) != rank:
                raise ValueError(
                    f"concat expects every tensor to have rank {rank}, got {len(t.shape)} at index {i}"
                )
            if t.type != tensors[0].type:
                raise TypeError(
                    f"concat expects matching dtypes, got {tensors[0].type!r} and {t.type!r} at index {i}"
                )
            for axis, (s, e) in enumerate(zip(t.shape, base)):
                if axis != dim and s != e:
                    raise ValueError(
                        f"concat shapes must match except on dim {dim}, got {tuple(t.shape)} at "
                        f"index {i} and {tuple(base)}"
                    )
        self.starts, self.lengths = [], []
        off = 0
        for t in tensors:
            self.starts.append(off)
            self.lengths.append(t.shape[dim])
            off += t.shape[dim]
        shape = list(base)
        shape[dim] = off
        out = functional.empty_like_shape(shape, tensors[0].type)
        for t, s, n in zip(tensors, self.starts, self.lengths):
            functional.assign(out.narrow(dim, s, n), t)
        out.requires_grad = any(t.requires_grad for t in tensors)
        self.dim = dim
        self.inputs = list(tensors)
        from ..backend import context

        self.needs_input_grad = [context.MODE == 0 and t.requires_grad for t in tensors]
        return self.attach(out)

    def backward(self, g):
        grads = []
        for need, s, n in zip(self.needs_input_grad, self.starts, self.lengths):
            if not need:
                grads.append(None)
                continue
            gi = g.narrow(self.dim, s, n)
            grads.append(gi if gi.is_contiguous() else gi.contiguous())
        return grads


class unsqueeze(Function):
    def forward(self, tensor1, dim):
        self.in_shape = list(tensor1.shape)
        rank = len(tensor1.shape)
        dims = (rank,) if dim is None else ((dim,) if isinstance(dim, int) else tuple(dim))
        final = rank + len(dims)
        norm = sorted(validation.normalize_dim(d, final, name="dim") for d in dims)
        if len(set(norm)) != len(norm):
            raise ValueError(f"duplicate unsqueeze dimensions: {norm}")
        shape, stride = list(tensor1.shape), list(tensor1.stride)
        for a in norm:
            shape.insert(a, 1)
            stride.insert(a, 0)
        out = Tensor(shape=shape, buffer=tensor1.buffer, stride=stride, offset=tensor1.offset,
                     requires_grad=tensor1.requires_grad, dtype=tensor1.type)
        out._base = tensor1
        return self.attach(out)

    def backward(self, g):
        return functional.reshape(g, self.in_shape) if self.needs_input_grad[0] else None


class squeeze(Function):
    def forward(self, tensor1, dim):
        self.in_shape = list(tensor1.shape)
        rank = len(tensor1.shape)
        if dim is None:
            removed = {i for i, s in enumerate(tensor1.shape) if s == 1}
        else:
            dims = (dim,) if isinstance(dim, int) else tuple(dim)
            norm = {validation.normalize_dim(d, rank, name="dim") for d in dims}
            removed = {d for d in norm if tensor1.shape[d] == 1}
        keep = [a for a in range(rank) if a not in removed]
        out = Tensor(shape=[tensor1.shape[a] for a in keep], buffer=tensor1.buffer,
                     stride=[tensor1.stride[a] for a in keep], offset=tensor1.offset,
                     requires_grad=tensor1.requires_grad, dtype=tensor1.type)
        out._base = tensor1
        return self.attach(out)

    def backward(self, g):
        return functional.reshape(g, self.in_shape) if self.needs_input_grad[0] else None


# ---------------------------------------------------------------- FFT / complex

def _rfft_backward_weights(n):
    return [1.0] if n == 1 else [1.0] + [0.5] * (n // 2 - 1) + [1.0]


def _irfft_backward_weights(n):
    return [1.0] if n == 1 else [1.0] + [2.0] * (n // 2 - 1) + [1.0]


def _match_last_dim_real(t, target):
    cur = t.shape[-1]
    if cur == target:
        return t
    if target < cur:
        return t.narrow(-1, 0, target)
    out = Tensor(list(t.shape[:-1]) + [target], value=0)
    functional.assign(out.narrow(-1, 0, cur), t)
    return out


def _sum_to_shape_complex(g, target_shape):
    """Broadcast adjoint for c64 gradients, reducing the (..., 2) float view."""
    target_shape = tuple(target_shape)
    if tuple(g.shape) == target_shape:
        return g
    if not g.is_contiguous():
        g = functional.complex_contiguous(g)
    real = Tensor(buffer=g.buffer, shape=list(g.shape) + [2],
                  stride=tuple(s * 2 for s in g.stride) + (1,), offset=g.offset * 2, dtype="f32")
    real._base = g
    red = _sum_to_shape(real, target_shape + (2,))
    if not red.is_contiguous():
        red = functional.contiguous(red)
    out = Tensor(buffer=red.buffer, shape=list(target_shape),
                 stride=tuple(s // 2 for s in red.stride[:-1]), offset=red.offset // 2, dtype="c64")
    out._base = red
    return out


class rfft(Function):
    def forward(self, tensor1, n=None):
        out, self.N = functional.rfft(tensor1, n)
        self.in_len = tensor1.shape[-1]
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        w = functional.complex_weights(_rfft_backward_weights(self.N))
        # irfft(g w, N) * N cropped to the input length, in one kernel (the
        # crop and the factor N are the same arithmetic as separate passes)
        ga = functional.irfft(functional.complex_mul(g, w), self.N,
                              length=min(self.in_len, self.N), scale=float(self.N))
        return _match_last_dim_real(ga, self.in_len)


class irfft(Function):
    """``length`` keeps the first ``length`` output samples (the crop
    ``irfft(x, n)[..., :length]``); its backward is the rfft of the cropped
    gradient zero-padded to n, which rfft's own padding provides."""

    def forward(self, tensor1, n=None, length=None):
        out = functional.irfft(tensor1, n, length=length)
        self.N = 2 * (tensor1.shape[-1] - 1) if n is None else int(n)
        self.in_len = tensor1.shape[-1]
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        if not self.needs_input_grad[0]:
            return None
        spec, _ = functional.rfft(g, self.N)
        w = functional.complex_weights([x / float(self.N) for x in _irfft_backward_weights(self.N)])
        gs = functional.complex_mul(spec, w)
        # the spectrum already has the input's N / 2 + 1 bins when n matched
        # it: no pad (a copy of the whole spectrum otherwise)
        return gs if gs.shape[-1] == self.in_len else functional.complex_pad(gs, self.in_len)


class complex_mul(Function):
    def forward(self, tensor1, tensor2):
        out = functional.complex_mul(tensor1, tensor2)
        out.requires_grad = tensor1.requires_grad or tensor2.requires_grad
        return self.attach(out, tensor1=tensor1, tensor2=tensor2)

    def backward(self, g):
        a, b = self.tensor1, self.tensor2
        self.tensor1 = self.tensor2 = None
        ga = (_sum_to_shape_complex(functional.complex_mul(g, b, conj_b=True), self.inputs[0].shape)
              if self.needs_input_grad[0] else None)
        gb = (_sum_to_shape_complex(functional.complex_mul(g, a, conj_b=True), self.inputs[1].shape)
              if self.needs_input_grad[1] else None)
        return ga, gb


class fft_conv(Function):
    """``irfft(rfft(x, n) * rfft(h, n), n)[..., :length]``: the long
    convolution of (..., D, Lx) signals with (D, Lh) filters broadcast over
    the leading dims (reference nn/hyena.py:208-216), with every spectrum
    product fused into a transform: the forward product into the inverse
    transform's load, the irfft adjoint's bin weights into the rfft's store,
    the filter product and the rfft adjoint's bin weights into the inverse
    transform of the signal gradient, and the filter gradient's product and
    batch sum into one pass.  Values and gradients equal those of the
    composed rfft / complex_mul / irfft Functions bit for bit (each fused
    product rounds as complex_mul does, the batch sum adds in the reduction's
    order).  Built as ``fft_conv(x, h)``, run as ``.forward(x, h, n, length)``
    for a power-of-two n <= ``functional.FUSED_MAX_N``."""

    def forward(self, x, h, n, length):
        n = int(n)
        self.N, self.x_len, self.h_len = n, x.shape[-1], h.shape[-1]
        X, _ = functional.rfft(x, n)
        H, _ = functional.rfft(h, n)
        out = functional.irfft_mul(X, n, h=H, length=length)
        out.requires_grad = x.requires_grad or h.requires_grad
        return self.attach(out, X=X, H=H)

    def backward(self, g):
        X, H = self.X, self.H
        self.X = self.H = None
        n = self.N
        # the adjoints' bin weights as (edge, interior) scalars: the irfft
        # adjoint rfft(g, n) * (1, 2, ..., 2, 1) / n, the rfft adjoint's
        # (1, 0.5, ..., 0.5, 1) (_irfft_backward_weights, _rfft_backward_weights;
        # at n = 2 both bins are edges and the interior value is unused)
        gs = functional.rfft_mul(g, n, (1.0 / float(n), 2.0 / float(n)))
        wr = (1.0, 0.5)
        gx = gh = None
        if self.needs_input_grad[0]:
            # the rfft adjoint of gs * conj(H): irfft(gs conj(H) w_rfft) * n
            gx = functional.irfft_mul(gs, n, h=H, conj_h=True, bin_weights=wr,
                                      length=min(self.x_len, n), scale=float(n))
            gx = _match_last_dim_real(gx, self.x_len)
        if self.needs_input_grad[1]:
            gH = functional.complex_mul_batch_sum(gs, X, conj_c=True, keep=len(H.shape))
            gh = functional.irfft_mul(gH, n, bin_weights=wr, length=min(self.h_len, n),
                                      scale=float(n))
            gh = _match_last_dim_real(gh, self.h_len)
        return gx, gh


class complex_conj(Function):
    def forward(self, tensor1):
        out = functional.complex_conj(tensor1)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out)

    def backward(self, g):
        return functional.complex_conj(g) if self.needs_input_grad[0] else None
