"""GPU parity: elementwise, scalar, unary and layout kernels vs the oracle."""

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import activations as oa
from oracle import elementwise as oe

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


@pytest.mark.parametrize("op", [0, 1, 2, 3])
@pytest.mark.parametrize("sa,sb", [((5, 7), (5, 7)), ((3, 1), (1, 4)), ((8, 1024, 768), (768,)),
                                   ((96, 128, 128), (128, 128)), ((2, 3, 4, 5), (3, 1, 5)),
                                   ((1,), (6,)), ((4097,), (4097,))])
def test_pointwise_broadcast(device, op, sa, sb):
    a = rng(1).standard_normal(sa).astype(np.float32)
    b = rng(2).standard_normal(sb).astype(np.float32) + (3.0 if op == 3 else 0.0)
    got = F().pointwise(up(a), up(b), op).numpy()
    assert_close(got, oe.pointwise(a, b, op), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_pointwise_inplace_broadcast_and_misaligned(device, op):
    # in place (out aliases a), broadcast over the middle dim, and a view
    # whose base is 1 float off 16 bytes, all bit-exact against float32
    a = rng(30 + op).standard_normal((4, 6, 16)).astype(np.float32)
    b = rng(40 + op).standard_normal((4, 1, 16)).astype(np.float32) + (3.0 if op == 3 else 0.0)
    want = oe.pointwise(a, b, op)
    ta = up(a)
    F()._pointwise(ta, up(b), op)
    assert np.array_equal(ta.numpy(), want)
    assert np.array_equal(F().pointwise(up(a), up(b), op).numpy(), want)
    x = rng(50 + op).standard_normal((4, 6, 17)).astype(np.float32)
    got = F().pointwise(up(x).narrow(2, 1, 16), up(b), op).numpy()
    assert np.array_equal(got, oe.pointwise(x[:, :, 1:], b, op))


def test_pointwise_strided_views(device):
    # reference tests/test_pointwise.py:90-112
    x = rng(4).standard_normal((4, 6, 8)).astype(np.float32)
    y = rng(5).standard_normal((4, 6, 8)).astype(np.float32)
    xt = F().permute(up(x), 0, 2, 1)
    yt = F().permute(up(y), 0, 2, 1)
    assert not xt.is_contiguous()
    assert_close(F().pointwise(xt, yt, 2).numpy(), np.transpose(x, (0, 2, 1)) * np.transpose(y, (0, 2, 1)))
    X, Y = up(x), up(y)
    assert_close(F().pointwise(X[1:], Y[1:], 0).numpy(), x[1:] + y[1:])
    assert_close(F().scalarpointwise(X[:, ::2, :], 3.0, 2).numpy(), x[:, ::2, :] * 3.0)
    col = F().permute(X, 0, 2, 1)[:, :, :1]
    assert_close(F().pointwise(col, F().permute(Y, 0, 2, 1), 0).numpy(),
                 np.transpose(x, (0, 2, 1))[:, :, :1] + np.transpose(y, (0, 2, 1)))


@pytest.mark.parametrize("op", [0, 2, 3])
@pytest.mark.parametrize("cols,off", [(16, 0), (682, 0), (682, 682), (33, 0), (12, 1)])
def test_pointwise_row_views_every_access_width(device, op, cols, off):
    # rank-2 views of unit column stride (the halves of a chunked (rows, 2
    # cols + 8) tensor, a row broadcast, in place): rows whose bases allow
    # 16-byte (cols 16), 8-byte (cols 682, also the second half first) or
    # 4-byte (cols 33; offset 1) accesses, bit-exact against float32
    rows, width = 300, 2 * cols + 8
    h = rng(60 + cols + off).standard_normal((rows, width)).astype(np.float32)
    v = rng(70 + cols).standard_normal((cols,)).astype(np.float32) + (3.0 if op == 3 else 0.0)
    o2 = 0 if off == cols else cols + 4
    h1, h2 = h[:, off:off + cols], h[:, o2:o2 + cols] + (3.0 if op == 3 else 0.0)
    th = up(h)
    x1 = th.narrow(1, off, cols)
    x2 = th.narrow(1, o2, cols)
    if op == 3:
        x2 = F().scalarpointwise(x2, 3.0, 0)
    assert np.array_equal(F().pointwise(x1, x2, op).numpy(), oe.pointwise(h1, h2, op))
    assert np.array_equal(F().pointwise(x1, up(v), op).numpy(), oe.pointwise(h1, v, op))
    tc = up(np.ascontiguousarray(h1))
    F()._pointwise(tc, up(v), op)
    assert np.array_equal(tc.numpy(), oe.pointwise(h1, v, op))


@pytest.mark.parametrize("op", [0, 1, 2, 3])
@pytest.mark.parametrize("shape", [(3, 70, 130), (130, 70), (2, 256, 512)])
@pytest.mark.parametrize("which", ["a", "b"])
def test_pointwise_one_operand_transposed(device, op, shape, which):
    # one operand a transposed view (unit stride along the second-last dim),
    # the other and the output row-major: the LDS-tiled path, ragged 64 x 64
    # tiles, bit-exact against float32
    t_shape = shape[:-2] + (shape[-1], shape[-2])
    src = rng(80 + op).standard_normal(t_shape).astype(np.float32)
    other = rng(90 + op).standard_normal(shape).astype(np.float32)
    if op == 3:
        src, other = src + 3.0, other + 3.0
    perm = tuple(range(len(shape) - 2)) + (len(shape) - 1, len(shape) - 2)
    tv = F().permute(up(src), *perm)
    sv = np.transpose(src, perm)
    assert not tv.is_contiguous()
    if which == "a":
        got, want = F().pointwise(tv, up(other), op), oe.pointwise(sv, other, op)
    else:
        got, want = F().pointwise(up(other), tv, op), oe.pointwise(other, sv, op)
    assert np.array_equal(got.numpy(), want)


def test_pointwise_inplace_and_alias(device):
    a = rng(6).standard_normal((3, 4)).astype(np.float32)
    b = rng(7).standard_normal((4,)).astype(np.float32)
    ta = up(a)
    F()._pointwise(ta, up(b), 0)
    assert_close(ta.numpy(), a + b)
    c = up(np.array([1.0, 2.0, 3.0]))
    F()._pointwise(c, c, 0)
    assert np.array_equal(c.numpy(), np.array([2.0, 4.0, 6.0], np.float32))


@pytest.mark.parametrize("op,c,rev", [(0, 2.5, 0), (1, 2.5, 0), (1, 2.5, 1), (2, -1.5, 0),
                                      (3, 3.0, 0), (3, -1.0, 0), (3, 2.0, 0), (3, 0.5, 0),
                                      (3, 2.5, 1), (4, 2.0, 0), (4, 2.0, 1)])
def test_scalarpointwise(device, op, c, rev):
    x = np.array([[-2.0, -0.5, 0.5, 2.0], [0.25, 1.5, 3.0, 4.0], [-3.0, -2.0, 2.0, 3.0]],
                 np.float32)
    x = np.concatenate([x, rng(8).standard_normal((5, 4)).astype(np.float32)])
    got = F().scalarpointwise(up(x), c, op, rev).numpy()
    assert_close(got, oe.scalarpointwise(x, c, op, rev), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("name", sorted(oa.UNARY))
def test_unary(device, name):
    from wxx_amd.functional import activations as fa

    x = (rng(9).standard_normal(10001) * 4).astype(np.float32)
    x[:4] = [0.0, 10.5, -10.5, 100.0]
    if name in ("log", "sqrt", "rsqrt"):
        x = np.abs(x) + 0.1
    if name == "sigmoidbackwards":
        x = oa.sigmoid(x)
    got = fa.unary(up(x), name).numpy()
    assert_close(got, oa.UNARY[name](x), rtol=2e-6, atol=2e-6)


def test_clamp_equal_masked_fill(device):
    x = rng(10).standard_normal(1000).astype(np.float32)
    x[:3] = 0.0
    assert np.array_equal(F().clamp(up(x), -0.5, 0.7).numpy(), oe.clamp(x, -0.5, 0.7))
    assert np.array_equal(F().clampbackwards(up(x), -0.5, 0.7).numpy(),
                          oe.clampbackwards(x, -0.5, 0.7))
    assert np.array_equal(F().masked_fill(up(x), -1e9).numpy(), oe.masked_fill(x, -1e9))
    assert np.array_equal(F().equal(up(x), up(x)).numpy(), np.ones(1000, np.float32))
    assert np.array_equal(F().equal_number(up(x), 0.0).numpy(), oe.equal(x, 0.0))
    u = F().from_numpy(np.arange(10) % 3, dtype=np.uint32)
    assert np.array_equal(F().equal_number(u, 2).numpy(), (np.arange(10) % 3 == 2).astype(np.float32))


@pytest.mark.parametrize("shape", [(7, 9), (8, 256, 64)])  # scalar and float4 paths
def test_mul_backward(device, shape):
    g, a, b = (rng(i).standard_normal(shape).astype(np.float32) for i in (11, 12, 13))
    da, db = F().mul_backward(up(g), up(a), up(b))
    ea, eb = oe.mul_backward(g, a, b)
    assert np.array_equal(da.numpy(), ea) and np.array_equal(db.numpy(), eb)


@pytest.mark.parametrize("B,L,D,parts", [(2, 70, 33, 3), (3, 128, 64, 4)])
def test_assign_transposed_source_into_slice(device, B, L, D, parts):
    # a (B, D, L) tensor viewed as (B, L, D) written into a channel slice of a
    # (B, L, parts * D) buffer: the LDS-tiled transpose with a strided destination
    g = rng(18).standard_normal((B, D, L)).astype(np.float32)
    buf = rng(19).standard_normal((B, L, parts * D)).astype(np.float32)
    t = up(buf)
    src = F().permute(up(g), 0, 2, 1)
    F().assign(t.narrow(2, D, D), src)
    want = buf.copy()
    want[:, :, D:2 * D] = g.transpose(0, 2, 1)
    assert np.array_equal(t.numpy(), want)


@pytest.mark.parametrize("shape,perm", [((4, 6, 8), (0, 2, 1)), ((8, 1024, 12, 64), (0, 2, 1, 3)),
                                        ((64, 96), (1, 0)), ((2, 3, 4, 5, 6), (4, 2, 0, 3, 1)),
                                        ((1000, 3), (1, 0))])
def test_contiguous_bit_exact(device, shape, perm):
    x = rng(14).standard_normal(shape).astype(np.float32)
    got = F().contiguous(F().permute(up(x), *perm)).numpy()
    assert np.array_equal(got, np.ascontiguousarray(np.transpose(x, perm)))


@pytest.mark.parametrize("start", [0, 1, 4])
@pytest.mark.parametrize("inner", [8, 6])
def test_contiguous_quads_and_fallbacks(device, start, inner):
    # copies whose innermost dim is unit stride in both views move 16-byte
    # quads when that length, the outer strides and both bases allow it;
    # a length of 6 or a base 1 float off 16 bytes takes the element path
    x = rng(20 + start + inner).standard_normal((2, 5, 3, 12)).astype(np.float32)
    v = F().permute(up(x).narrow(3, start, inner), 0, 2, 1, 3)
    got = F().contiguous(v).numpy()
    assert np.array_equal(got, np.ascontiguousarray(
        np.transpose(x[..., start:start + inner], (0, 2, 1, 3))))


def test_assign_and_scatter_and_unfold(device):
    x = np.zeros((5, 6), np.float32)
    t = up(x)
    F().assign(t[1:4, ::2], 7.0)
    x[1:4, ::2] = 7.0
    assert np.array_equal(t.numpy(), x)
    src = rng(15).standard_normal((3, 3)).astype(np.float32)
    F().assign(t[1:4, ::2], up(src))
    x[1:4, ::2] = src
    assert np.array_equal(t.numpy(), x)
    g = rng(16).standard_normal((2, 3, 4)).astype(np.float32)
    out = F().scatter_zeros(up(g), (2, 7, 4), 1, 2).numpy()
    ref = np.zeros((2, 7, 4), np.float32)
    ref[:, 2:5] = g
    assert np.array_equal(out, ref)
    # unfold backward: scatter-add of overlapping windows
    inp = (2, 10, 3)
    size, step = 4, 2
    windows = (10 - size) // step + 1
    dy = rng(17).standard_normal((2, windows, 3, size)).astype(np.float32)
    dx = F().unfolddx(up(dy), inp, 1, size, step).numpy()
    ref = np.zeros(inp, np.float64)
    for l in range(windows):
        for w in range(size):
            ref[:, l * step + w, :] += dy[:, l, :, w]
    assert_close(dx, ref, atol=1e-6)


@pytest.mark.parametrize("name", ["relu", "gelu", "sigmoid", "selu", "sin", "cos"])
def test_unary_backward_is_derivative_times_grad(device, name):
    from wxx_amd.functional import activations as fa

    x = (rng(18).standard_normal(4099) * 4).astype(np.float32)
    g = rng(19).standard_normal(4099).astype(np.float32)
    src = oa.sigmoid(x) if name == "sigmoid" else x
    got = fa.unary_backward(up(src), up(g), name).numpy()
    deriv = {"relu": "relubackwards", "gelu": "gelubackwards", "sigmoid": "sigmoidbackwards",
             "selu": "selubackwards", "sin": "sinback", "cos": "cosback"}[name]
    assert_close(got, oa.UNARY[deriv](src) * g, rtol=4e-6, atol=2e-6)
