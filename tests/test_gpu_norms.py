"""GPU parity: LayerNorm, RMSNorm and BatchNorm forward/backward vs the oracle."""

import numpy as np
import pytest

from conftest import assert_close, assert_error_floor, rng
from oracle import norms as on

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


SHAPES = [((2, 3, 4), -1), ((8192, 4096), -1), ((8, 1024, 768), -1), ((4, 128, 256), -1),
          ((5, 100), -1), ((3, 7, 5), 1), ((6, 20000), -1), ((9, 130), -1), ((2, 3), 0)]


F32 = np.float32


@pytest.mark.parametrize("shape,axis", SHAPES)
def test_layernorm_fwd_bwd(device, shape, axis):
    # every output against the float64 restatement, within 4x what the same
    # formulas evaluated in float32 miss by (plus rtol 1e-4 of the element)
    r = rng(len(shape) * 10 + shape[-1] % 97)
    x = (r.standard_normal(shape) * 2 + 0.5).astype(np.float32)
    red = shape[axis]
    g = r.standard_normal(red).astype(np.float32)
    b = r.standard_normal(red).astype(np.float32)
    y, mu, inv = F().meanvarnorm(up(x), up(g), up(b), axis=axis)
    ey, emu, einv = on.meanvarnorm(x, g, b, axis=axis)
    fy, fmu, finv = on.meanvarnorm(x, g, b, axis=axis, dtype=F32)
    assert_error_floor(mu.numpy(), emu, fmu, msg="mean")
    assert_error_floor(inv.numpy(), einv, finv, msg="inv_std")
    assert_error_floor(y.numpy(), ey, fy, msg="y")
    dy = r.standard_normal(shape).astype(np.float32)
    dx = F().meanvarnormdx(up(dy), up(x), up(g), mu, inv, axis=axis)
    assert_error_floor(dx.numpy(), on.meanvarnormdx(dy, x, g, emu, einv, axis=axis),
                       on.meanvarnormdx(dy, x, g, emu, einv, axis=axis, dtype=F32), msg="dx")
    dg, db = F().meanvarnormdg(up(dy), up(x), mu, inv, axis=axis)
    edg, edb = on.meanvarnormdg(dy, x, emu, einv, axis=axis)
    fdg, fdb = on.meanvarnormdg(dy, x, emu, einv, axis=axis, dtype=F32)
    assert_error_floor(dg.numpy(), edg, fdg, msg="dgamma")
    assert_error_floor(db.numpy(), edb, fdb, msg="dbeta")


def test_layernorm_reference_test_case(device):
    x = rng(0).standard_normal((2, 3, 4)).astype(np.float32)
    y, _, _ = F().meanvarnorm(up(x), up(np.ones(4)), up(np.zeros(4)), axis=-1)
    ref = (x - x.mean(axis=-1, keepdims=True)) / np.sqrt(x.var(axis=-1, keepdims=True) + 1e-5)
    assert_close(y.numpy(), ref, atol=1e-4)


def test_norm_zero_rows_and_row_cap(device):
    from wxx_amd.backend import compat

    x = rng(1).standard_normal((65537, 8)).astype(np.float32)
    x[3] = 0.0
    g = rng(2).standard_normal(8).astype(np.float32)
    b = rng(3).standard_normal(8).astype(np.float32)
    y, mu, inv = F().meanvarnorm(up(x), up(g), up(b), axis=-1)
    assert inv.numpy()[3] == 0.0
    assert_close(y.numpy()[3], b)
    assert np.any(y.numpy()[65535:] != 0)  # default: every row computed
    yr, rr = F().rmsnorm(up(x), up(g), axis=-1)
    assert rr.numpy()[3] == 0.0
    compat.REFERENCE_ROW_CAP = True
    try:
        yc, muc, invc = F().meanvarnorm(up(x), up(g), up(b), axis=-1)
        ey, emu, einv = on.meanvarnorm(x, g, b, row_cap=65535)
        assert np.all(yc.numpy()[65535:] == 0) and np.all(invc.numpy()[65535:] == 0)
        assert_close(yc.numpy(), ey, atol=1e-4)
        yrc, rrc = F().rmsnorm(up(x), up(g), axis=-1)
        assert np.all(yrc.numpy()[65535:] == 0) and np.all(rrc.numpy()[65535:] == 0)
    finally:
        compat.REFERENCE_ROW_CAP = False


@pytest.mark.parametrize("shape,axis", [((2, 4), -1), ((8, 8192, 256), -1), ((3, 5, 7), 1),
                                        ((4, 3000), -1)])
def test_rmsnorm_fwd_bwd(device, shape, axis):
    r = rng(50 + shape[-1] % 13)
    x = r.standard_normal(shape).astype(np.float32)
    red = shape[axis]
    g = r.standard_normal(red).astype(np.float32)
    y, irms = F().rmsnorm(up(x), up(g), axis=axis)
    ey, er = on.rmsnorm(x, g, axis=axis)
    fy, fr = on.rmsnorm(x, g, axis=axis, dtype=F32)
    assert_error_floor(irms.numpy(), er, fr, msg="inv_rms")
    assert_error_floor(y.numpy(), ey, fy, msg="y")
    dy = r.standard_normal(shape).astype(np.float32)
    dx = F().rmsnormdx(up(dy), up(x), up(g), irms, axis=axis)
    assert_error_floor(dx.numpy(), on.rmsnormdx(dy, x, g, er, axis=axis),
                       on.rmsnormdx(dy, x, g, er, axis=axis, dtype=F32), msg="dx")
    dg = F().rmsnormdg(up(dy), up(x), up(g), irms, axis=axis)
    assert_error_floor(dg.numpy(), on.rmsnormdg(dy, x, er, axis=axis),
                       on.rmsnormdg(dy, x, er, axis=axis, dtype=F32), msg="dgamma")


# B*H*W <= 8192 take the one-launch kernels; (128, 64, 16, 16) and (64, 3, 48, 48) the
# two-launch split path
@pytest.mark.parametrize("shape", [(4, 3, 2, 2), (128, 64, 16, 16), (128, 512, 1, 1),
                                   (2, 5, 7, 3), (64, 3, 48, 48)])
@pytest.mark.parametrize("training", [True, False])
def test_batchnorm(device, shape, training):
    r = rng(60)
    C = shape[1]
    x = r.standard_normal(shape).astype(np.float32)
    g = r.standard_normal(C).astype(np.float32)
    b = r.standard_normal(C).astype(np.float32)
    rm0 = r.standard_normal(C).astype(np.float32)
    rv0 = (r.random(C) + 0.5).astype(np.float32)
    rm, rv = up(rm0), up(rv0)
    y, mu, inv = F().batchnorm(up(x), up(g), up(b), rm, rv, training=training)
    ey, emu, einv, erm, erv = on.batchnorm(x, g, b, rm0, rv0, training)
    fy, fmu, finv, frm, frv = on.batchnorm(x, g, b, rm0, rv0, training, dtype=F32)
    for name, got, want, f32 in (("mean", mu, emu, fmu), ("inv_std", inv, einv, finv),
                                 ("y", y, ey, fy), ("running mean", rm, erm, frm),
                                 ("running var", rv, erv, frv)):
        assert_error_floor(got.numpy(), want, f32, msg=name)
    dy = r.standard_normal(shape).astype(np.float32)
    dg, db = F().batchnormdg(up(dy), up(x), mu, inv)
    edg, edb = on.batchnormdg(dy, x, emu, einv)
    fdg, fdb = on.batchnormdg(dy, x, emu, einv, dtype=F32)
    assert_error_floor(dg.numpy(), edg, fdg, msg="dgamma")
    assert_error_floor(db.numpy(), edb, fdb, msg="dbeta")
    dx = F().batchnormdx(up(dy), up(x), up(g), dg, db, mu, inv)
    assert_error_floor(dx.numpy(), on.batchnormdx(dy, x, g, edg, edb, emu, einv),
                       on.batchnormdx(dy, x, g, edg, edb, emu, einv, dtype=F32), msg="dx")
    # the autograd backward's one call: the same three results
    dx2, dg2, db2 = F().batchnorm_backward(up(dy), up(x), up(g), mu, inv)
    assert_error_floor(dg2.numpy(), edg, fdg, msg="batchnorm_backward dgamma")
    assert_error_floor(db2.numpy(), edb, fdb, msg="batchnorm_backward dbeta")
    assert_error_floor(dx2.numpy(), on.batchnormdx(dy, x, g, edg, edb, emu, einv),
                       on.batchnormdx(dy, x, g, edg, edb, emu, einv, dtype=F32),
                       msg="batchnorm_backward dx")


@pytest.mark.parametrize("shape", [(4, 3, 2, 2), (128, 64, 8, 8), (128, 512, 1, 1),
                                   (128, 64, 16, 16), (2, 5, 7, 3), (64, 3, 48, 48)])
@pytest.mark.parametrize("residual,relu", [(True, True), (False, True), (True, False)])
def test_batchnorm_act_equals_composed_ops(device, shape, residual, relu):
    # relu(batchnorm(x) + r) as one kernel, and its backward, equal the
    # composed ops (batchnorm twice for the two running-statistic updates,
    # the add, the ReLU, and their autograd backwards) bit for bit
    import wxx_amd as wxx
    from wxx_amd.nn import BatchNorm

    r = rng(sum(shape) + 7 * residual + relu)
    C = shape[1]
    x = r.standard_normal(shape).astype(np.float32)
    res = r.standard_normal(shape).astype(np.float32) if residual else None
    dz = r.standard_normal(shape).astype(np.float32)
    g = r.standard_normal(C).astype(np.float32)
    b = r.standard_normal(C).astype(np.float32)
    rm0 = r.standard_normal(C).astype(np.float32)
    rv0 = (r.random(C) + 0.5).astype(np.float32)
    outs = []
    for fused in (True, False):
        bn = BatchNorm(C)
        bn.weight = wxx.Parameter(up(g))
        bn.bias = wxx.Parameter(up(b))
        bn.running_mean, bn.running_std = up(rm0), up(rv0)
        tx = up(x)
        tx.requires_grad = True
        tr = None
        if residual:
            tr = up(res)
            tr.requires_grad = True
        if fused:
            assert F().batchnorm_act_supported(tx)
            z = bn.act(tx, residual=tr, relu=relu, updates=2)
        else:
            bn(tx)
            z = bn(tx)
            if residual:
                z = z + tr
            if relu:
                z = z.relu()
        (z * up(dz)).sum().backward()  # z's gradient is dz
        outs.append([z.numpy(), bn.running_mean.numpy(), bn.running_std.numpy(), tx.grad.numpy(),
                     bn.weight.grad.numpy(), bn.bias.grad.numpy()]
                    + ([tr.grad.numpy()] if residual else []))
    names = ["y", "running mean", "running var", "dx", "dgamma", "dbeta", "dresidual"]
    for name, a, e in zip(names, *outs):
        assert np.array_equal(a, e), name
    # and the forward against the float64 oracle: relu(bn(x) + r)
    ey, _, _, erm, erv = on.batchnorm(x, g, b, rm0, rv0, True)
    ey = ey + (res if residual else 0)
    ey = np.maximum(ey, 0) if relu else ey
    assert_close(outs[0][0], ey, rtol=1e-5, atol=1e-5, msg="y against the oracle")


def test_batchnorm_act_rejects_empty_channels(device):
    x = up(np.zeros((0, 3, 4, 4)))
    assert not F().batchnorm_act_supported(x)
    one = up(np.ones(3))
    with pytest.raises(Exception):
        F().batchnorm_act(x, one, one, None, up(np.zeros(3)), up(np.ones(3)))


def test_norm_parameter_size_is_validated(device):
    # gamma/beta are indexed by the reduce coordinate: a mismatch must be
    # rejected on the host, never read out of bounds on the device
    x = up(rng(4).standard_normal((16, 8)))
    g8 = up(np.ones(8))
    with pytest.raises(ValueError):
        F().meanvarnorm(x, g8, g8)          # axis=None normalises all 128 elements
    with pytest.raises(ValueError):
        F().rmsnorm(x, g8)
    with pytest.raises(ValueError):
        F().meanvarnorm(x, up(np.ones(7)), g8, axis=-1)
    with pytest.raises(ValueError):
        F().batchnorm(up(np.ones((2, 3, 2, 2))), up(np.ones(2)), up(np.ones(3)), up(np.ones(3)),
                      up(np.ones(3)), training=True)
