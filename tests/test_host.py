"""Host-side logic that needs no device: validation, reduction views,
broadcasting and the error behaviour of the reference's validators."""

import pytest

from wxx_amd import validation
from wxx_amd.backend import dispatch


def test_reduce_dims_match_reference_mapping():
    assert dispatch._get_reduce_dims((4, 5)) == (1, 20, 1, (1,))
    assert dispatch._get_reduce_dims((4, 5), 0) == (1, 4, 5, (5,))
    assert dispatch._get_reduce_dims((4, 5), -1) == (4, 5, 1, (4,))
    assert dispatch._get_reduce_dims((2, 3, 4, 5), (1, 2)) == (2, 12, 5, (2, 5))
    with pytest.raises(ValueError):
        dispatch._get_reduce_dims((2, 3, 4), (0, 2))
    with pytest.raises(ValueError):
        dispatch._get_reduce_dims((), None)


def test_broadcast_rules():
    out, pa, pb = dispatch.broadcast_shapes((3, 1), (1, 4))
    assert out == (3, 4) and pa == (3, 1) and pb == (1, 4)
    assert dispatch.compute_broadcast_strides((1, 4), (3, 4)) == (0, 1)
    with pytest.raises(ValueError):
        dispatch.broadcast_shapes((3, 2), (4,))


def test_validation_errors():
    with pytest.raises(TypeError):
        validation.normalize_shape((2, 1.5))
    with pytest.raises(ValueError):
        validation.normalize_shape((2, -3))
    assert validation.infer_shape((-1, 4), 8) == (2, 4)
    with pytest.raises(ValueError):
        validation.infer_shape((-1, 3), 8)
    with pytest.raises(IndexError):
        validation.normalize_dim(3, 3)
    assert validation.normalize_dim(-1, 3) == 2
    assert validation.is_contiguous_layout((2, 1, 3), (3, 99, 1))
    assert not validation.is_contiguous_layout((2, 3), (1, 2))


def test_keepdims_shape():
    assert dispatch.keepdims_shape((4, 5), 1) == (4, 1)
    assert dispatch.keepdims_shape((4, 5), None) == (1, 1)


def test_reference_import_name_resolves_to_this_package():
    # code written against the reference imports ``wxx`` and its submodules
    # (e.g. nn/module.py:5 ``from wxx.functional.utils import from_numpy``);
    # both names must give the very same module objects (one device, one
    # set of classes), and importing opens no device
    import wxx
    import wxx_amd
    from wxx.functional.utils import from_numpy
    from wxx.nn.gpt import GPT2
    import wxx.autograd.function as waf
    import wxx_amd.autograd.function as aaf

    assert wxx is wxx_amd
    assert from_numpy is wxx_amd.functional.utils.from_numpy
    assert GPT2 is wxx_amd.nn.GPT2
    assert waf is aaf
    with pytest.raises(ModuleNotFoundError):
        __import__("wxx.no_such_module")


def test_graph_hooks_outside_a_recording_are_refused():
    # the per-replay words, hooks and checks exist only while a step graph is
    # being recorded; outside one they raise instead of silently doing nothing
    from wxx_amd import graphs

    assert not graphs.capturing()
    for fn, args in [(graphs.per_replay, (1, lambda w: None)), (graphs.on_replay, (print,)),
                     (graphs.after_replay, (print,)), (graphs.keep_alive, (1,))]:
        with pytest.raises(RuntimeError, match="recorded"):
            fn(*args)
    g = graphs.StepGraph(lambda: None)
    with pytest.raises(RuntimeError, match="capture"):
        g.replay()
    g.close()  # closing an unrecorded graph is a no-op
