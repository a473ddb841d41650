"""GPU: the allocation-free GEMM entry point (wxx_matmul_add_noalloc).

It must give wxx_matmul_add's results bit for bit (same kernels, same tile
and split choice) while allocating nothing: the library's allocator count
does not move across its calls, its split-K partials living in a fixed
device array.  Two calls in a row, the second smaller, check that a call
does not depend on what the previous one left in that array; a call whose
partials exceed the array fails with a clear error before enqueuing work.
"""

import ctypes as C

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

P = C.c_void_p
SCRATCH_FLOATS = 16 << 20


def _up(a):
    from wxx_amd import functional

    return functional.from_numpy(np.asarray(a, np.float32))


def _n_malloc():
    from wxx_amd.backend import lib

    vals = [C.c_size_t() for _ in range(4)]
    lib.call("wxx_mem_stats", *[C.byref(v) for v in vals])
    return vals[3].value


def _run(entry, A, B, bias, out, M, N, K, batch, sA, sB, sBias, mode, ta, tb, tile):
    from wxx_amd.backend import lib

    lib.call(entry, P(A.data_ptr()), P(B.data_ptr()), P(bias.data_ptr()) if bias is not None
             else None, P(out.data_ptr()), M, N, K, batch, sA, sB, sBias, mode, int(ta), int(tb),
             tile)
    return out.numpy()


@pytest.mark.parametrize("first,second", [
    # (M, N, K, batch, ta, tb, tile code): explicit K splits on 128 x 128
    # direct-to-LDS tiles, then a smaller automatic split-K launch
    ((1024, 1024, 4096, 1, False, False, 11 | (8 << 8)), (256, 200, 4097, 1, False, True, 0)),
    # automatic choice on a few tiles over a long K (64 x 64 tiles, split),
    # then an unsplit call that uses no scratch at all
    ((100, 70, 5000, 1, True, False, 0), (64, 48, 96, 3, False, False, 0)),
    # the Hyena SwiGLU weight-gradient shape (128 x 128 tiles, up to 64 splits)
    ((256, 682, 65536, 1, True, False, 0), (130, 300, 40000, 1, True, False, 0)),
])
def test_noalloc_matches_matmul_add_bit_for_bit(device, first, second):
    from wxx_amd.functional._common import empty

    # warm the allocator for the outputs and inputs below, then count
    for M, N, K, batch, ta, tb, tile in (first, second):
        r = rng(M + N + K)
        A = r.standard_normal((batch, K, M) if ta else (batch, M, K)).astype(np.float32)
        B = r.standard_normal((batch, N, K) if tb else (batch, K, N)).astype(np.float32)
        bias = r.standard_normal(N).astype(np.float32)
        tA, tB, tbias = _up(A), _up(B), _up(bias)
        sA, sB = M * K, K * N
        want = _run("wxx_matmul_add", tA, tB, tbias, empty([batch, M, N]), M, N, K, batch, sA,
                    sB, 0, 1, ta, tb, tile)
        out = empty([batch, M, N])
        before = _n_malloc()
        got = _run("wxx_matmul_add_noalloc", tA, tB, tbias, out, M, N, K, batch, sA, sB, 0, 1,
                   ta, tb, tile)
        assert _n_malloc() == before, "the allocation-free entry point allocated"
        assert np.array_equal(got, want), (M, N, K, batch, tile)
        # and it is a correct product (float64 check on a few rows)
        Ad = (np.swapaxes(A, 1, 2) if ta else A).astype(np.float64)
        Bd = (np.swapaxes(B, 1, 2) if tb else B).astype(np.float64)
        rows = [0, M // 2, M - 1]
        ref = Ad[:, rows] @ Bd + bias
        assert np.allclose(got[:, rows], ref, rtol=1e-4, atol=1e-5 * np.sqrt(K) + 1e-5)


def test_noalloc_rejects_partials_beyond_the_scratch(device):
    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    # 2048 x 2048 outputs in 8 explicit K splits need 32 Mi floats of
    # partials, twice the scratch: a clear error, nothing written
    M = N = 2048
    K = 1024
    assert M * N * 8 > SCRATCH_FLOATS
    A, B = _up(np.ones((M, K))), _up(np.ones((K, N)))
    out = _up(np.full((M, N), 7.0))
    with pytest.raises(lib.HIPError, match="allocation-free scratch holds"):
        _run("wxx_matmul_add_noalloc", A, B, None, out, M, N, K, 1, 0, 0, 0, 0, False, False,
             11 | (8 << 8))
    assert np.all(out.numpy() == 7.0)
    # the same shape unsplit needs no scratch and works
    got = _run("wxx_matmul_add_noalloc", A, B, None, empty([M, N]), M, N, K, 1, 0, 0, 0, 0,
               False, False, 11)
    assert np.all(got == K)
