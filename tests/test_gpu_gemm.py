"""GPU parity: the fp32 MFMA GEMM (functional.matmul_add) against the oracle.

Every shape, the BASELINE config-2 sizes included, is compared element by
element against the float64 product, within 4x the error of the reference's
own fp32 arithmetic on the same operands (the exact-order fma chain of
matmul.wgsl, restated in oracle/csrc/gemm_ref.c)."""

import numpy as np
import pytest

from conftest import assert_close, assert_error_floor, rng
from oracle import gemm as og

pytestmark = pytest.mark.gpu


def F():
    from wxx_amd import functional

    return functional


def up(a):
    return F().from_numpy(np.asarray(a, np.float32))


def check(got, A, B, bias=None, ta=False, tb=False, msg=""):
    """The device product against the float64 product, within 4x what the
    reference's own fp32 arithmetic (the exact-order fma chain of
    matmul.wgsl, oracle/csrc/gemm_ref.c) misses it by: a wrong, dropped or
    doubled K chunk is far outside that floor."""
    want = og.matmul_add(A, B, bias, ta, tb, rounded=False)
    ref32 = og.matmul_add_fma(A, B, bias, ta, tb)
    assert_error_floor(np.asarray(got), want, ref32, msg=msg)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 5, 9), (64, 64, 16), (128, 128, 128),
                                   (130, 67, 33), (256, 384, 96), (17, 682, 256),
                                   (300, 200, 1000), (64, 1024, 17), (5, 3, 0)])
def test_matmul_transposes_ragged(device, ta, tb, M, N, K):
    r = rng(M * 7 + N * 3 + K)
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    got = F().matmul_add(up(A), up(B), None, transpose_A=ta, transpose_B=tb).numpy()
    check(got, A, B, None, ta, tb)


@pytest.mark.parametrize("bias_kind", ["none", "vec", "mat", "batched"])
@pytest.mark.parametrize("layout", ["A_batched", "both_batched", "B_batched"])
def test_matmul_batch_and_bias_modes(device, bias_kind, layout):
    r = rng(11)
    b, M, K, N = 3, 37, 20, 45
    A = r.standard_normal((b, M, K) if layout != "B_batched" else (M, K)).astype(np.float32)
    B = r.standard_normal((b, K, N) if layout != "A_batched" else (K, N)).astype(np.float32)
    bias = {"none": None, "vec": r.standard_normal(N), "mat": r.standard_normal((M, N)),
            "batched": r.standard_normal((b, M, N))}[bias_kind]
    bt = None if bias is None else up(bias)
    got = F().matmul_add(up(A), up(B), bt).numpy()
    check(got, A, B, bias)


def test_matmul_attention_shapes(device):
    r = rng(12)
    q = r.standard_normal((12, 128, 64)).astype(np.float32)
    k = r.standard_normal((12, 128, 64)).astype(np.float32)
    s = F().matmul_add(up(q), up(k), None, transpose_B=True).numpy()
    check(s, q, k, None, False, True)
    p = r.standard_normal((12, 128, 128)).astype(np.float32)
    o = F().matmul_add(up(p), up(k), None).numpy()
    check(o, p, k)
    # weight-gradient shape: A^T @ g with batch
    g = r.standard_normal((12, 128, 64)).astype(np.float32)
    dw = F().matmul_add(up(q), up(g), None, transpose_A=True).numpy()
    check(dw, q, g, None, True, False)


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                                   (8192, 3072, 768), (8192, 768, 3072), (8192, 768, 768)])
def test_matmul_config2_sizes(device, M, N, K):
    # every element of BASELINE config 2's GEMMs against float64, within 4x
    # the reference's own fp32 fma-chain error on the same operands
    r = rng(10 + M % 7)
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    C = F().matmul_add(up(A), up(B), None).numpy()
    check(C, A, B, msg=f"{M}x{N}x{K}")


def test_matmul_errors(device):
    a = up(np.ones((3, 4)))
    with pytest.raises(ValueError):
        F().matmul_add(a, up(np.ones((5, 2))), None)
    with pytest.raises(ValueError):
        F().matmul_add(up(np.ones((2, 3, 4))), up(np.ones((3, 4, 2))), None)
    with pytest.raises(ValueError):
        F().matmul_add(a, up(np.ones((4, 2))), up(np.ones(3)))


@pytest.mark.parametrize("ta,tb,M,N,K,bias_kind", [
    (True, False, 768, 768, 8192, "none"),     # Linear dW at GPT-2 small: K = batch x seq
    (True, False, 768, 3072, 8192, "vec"),
    (False, False, 100, 70, 5000, "mat"),      # 64x64 tiles, split K
    (False, True, 256, 200, 4097, "vec"),      # ragged K tail in the last split
    (True, True, 130, 129, 2048, "none"),
    (True, False, 256, 682, 65536, "vec"),     # Hyena SwiGLU dW: 128x128 tiles, 64 splits
    (True, False, 130, 300, 40000, "none"),    # 38 splits of 1056, the last one shorter
])
def test_matmul_split_k(device, ta, tb, M, N, K, bias_kind):
    # few output tiles over a long K: the K range is split across workgroups
    # and the partials are added in split order by a second pass
    r = rng(M + N + K)
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = {"none": None, "vec": r.standard_normal(N), "mat": r.standard_normal((M, N))}[bias_kind]
    got = F().matmul_add(up(A), up(B), None if bias is None else up(bias), transpose_A=ta,
                         transpose_B=tb).numpy()
    check(got, A, B, bias, ta, tb)
    again = F().matmul_add(up(A), up(B), None if bias is None else up(bias), transpose_A=ta,
                           transpose_B=tb).numpy()
    assert np.array_equal(got, again), "split-K result must be deterministic"


def test_matmul_split_k_batched(device):
    r = rng(99)
    A = r.standard_normal((3, 64, 2048)).astype(np.float32)
    B = r.standard_normal((3, 2048, 48)).astype(np.float32)
    bias = r.standard_normal((3, 64, 48)).astype(np.float32)
    got = F().matmul_add(up(A), up(B), up(bias)).numpy()
    check(got, A, B, bias)


@pytest.mark.parametrize("code", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_every_tile_code(device, code, splits, ta, tb):
    # each tile / K-chunk / buffering variant of the kernel on a ragged shape
    # (edge tiles in M and N, a K tail shorter than the chunk) and an aligned one
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    for M, N, K in [(300, 270, 133), (256, 256, 512)]:
        r = rng(M + 3 * code + splits)
        A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        bias = r.standard_normal(N).astype(np.float32)
        tA, tB, tbias = up(A), up(B), up(bias)
        out = empty([M, N])
        P = C.c_void_p
        lib.call("wxx_matmul_add", P(tA.data_ptr()), P(tB.data_ptr()), P(tbias.data_ptr()),
                 P(out.data_ptr()), M, N, K, 1, 0, 0, 0, 1, int(ta), int(tb), code + 256 * splits)
        check(out.numpy(), A, B, bias, ta, tb)


@pytest.mark.parametrize("code", [11, 12, 13, 14, 15])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("batch,M,N,K,splits,bias_mode", [
    (1, 128, 256, 96, 1, 1),
    (2, 256, 128, 160, 3, 3),  # batched operands; K splits of 64, 64 and 32; per-batch bias
    (3, 128, 128, 64, 1, 2),   # one (M, N) bias for every batch
])
def test_matmul_direct_to_lds(device, code, ta, tb, batch, M, N, K, splits, bias_mode):
    # tiles 11 / 12 / 13: 128 x 128 / 128 x 192 / 128 x 64 operand tiles
    # loaded straight into LDS in swizzled layouts (14: 128 x 64 with three
    # buffers, two chunks of loads in flight; 15: 64 x 64 with three
    # buffers); only for M a multiple of the tile height, N of its width,
    # and whole 32-deep K chunks (N scaled to 192 / 384 for tile 12)
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    if code == 12:
        N = N * 3 // 2
    r = rng(M + N + K + batch)
    A = r.standard_normal((batch, K, M) if ta else (batch, M, K)).astype(np.float32)
    B = r.standard_normal((batch, N, K) if tb else (batch, K, N)).astype(np.float32)
    bias = r.standard_normal({1: (N,), 2: (M, N), 3: (batch, M, N)}[bias_mode]).astype(np.float32)
    tA, tB, tbias = up(A), up(B), up(bias)
    out = empty([batch, M, N])
    P = C.c_void_p
    lib.call("wxx_matmul_add", P(tA.data_ptr()), P(tB.data_ptr()), P(tbias.data_ptr()),
             P(out.data_ptr()), M, N, K, batch, M * K, K * N, M * N if bias_mode == 3 else 0,
             bias_mode, int(ta), int(tb), code + 256 * splits)
    check(out.numpy(), A, B, bias, ta, tb)


@pytest.mark.parametrize("K", [768, 3072])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_n768_every_transpose(device, ta, tb, K):
    # GPT-2 small's 8192 x 768 outputs under the automatic tile choice: the
    # q/k/v/out projections (K = 768) and the MLP's down projection and
    # up-projection input gradient (K = 3072; 128 x 192 tiles when B is
    # k-contiguous)
    M, N = 8192, 768
    r = rng(K + 2 * ta + tb)
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    got = F().matmul_add(up(A), up(B), up(bias), transpose_A=ta, transpose_B=tb).numpy()
    check(got, A, B, bias, ta, tb)


def test_matmul_direct_to_lds_rejects_edge_tiles(device):
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    A, B, out = up(np.ones((130, 64), np.float32)), up(np.ones((64, 128), np.float32)), empty([130, 128])
    P = C.c_void_p
    with pytest.raises(lib.HIPError, match="tile 11"):
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                 130, 128, 64, 1, 0, 0, 0, 0, 0, 0, 11)
    # tile 12 needs N a multiple of 192, tile 13 M a multiple of 128
    with pytest.raises(lib.HIPError, match="tile 12"):
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                 128, 128, 64, 1, 0, 0, 0, 0, 0, 0, 12)
    with pytest.raises(lib.HIPError, match="tile 13"):
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                 130, 128, 64, 1, 0, 0, 0, 0, 0, 0, 13)
    with pytest.raises(lib.HIPError, match="tile 14"):
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                 130, 128, 64, 1, 0, 0, 0, 0, 0, 0, 14)
    with pytest.raises(lib.HIPError, match="tile 15"):
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                 130, 128, 64, 1, 0, 0, 0, 0, 0, 0, 15)


def test_matmul_three_buffer_tiles_equal_two_buffer_tiles(device):
    # tile 14 runs tile 13's arithmetic with a deeper load pipeline: the same
    # products added in the same order, so the results are equal bit for bit
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    P = C.c_void_p
    for (M, N, K, splits) in [(1024, 1024, 1024, 2), (256, 192, 800, 1), (384, 128, 96, 3)]:
        r = rng(M + K)
        A, B = up(r.standard_normal((M, K)).astype(np.float32)), up(r.standard_normal((K, N)).astype(np.float32))
        outs = []
        for code in (13, 14):
            out = empty([M, N])
            lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), None, P(out.data_ptr()),
                     M, N, K, 1, 0, 0, 0, 0, 0, 0, code + 256 * splits)
            outs.append(out.numpy())
        np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("S,d", [(64, 64), (130, 64), (256, 32), (300, 64), (640, 64),
                                 (1024, 64)])
def test_matmul_tri_modes(device, S, d):
    # causal-attention products with their zero triangle skipped; in modes 2
    # and 3 a workgroup runs row tiles p and T - 1 - p of the T row tiles
    # (S = 300 and 640: an odd T, whose middle tile runs alone)
    b = 3
    r = rng(S + d)
    q = r.standard_normal((b, S, d)).astype(np.float32)
    k = r.standard_normal((b, S, d)).astype(np.float32)
    P = np.tril(r.standard_normal((b, S, S))).astype(np.float32)  # exact zeros above
    on_or_below = np.tril(np.ones((S, S), bool))
    # tri 1: scores, needed on / below the diagonal; above it 0 or the value
    s1 = F().matmul_add(up(q), up(k), None, transpose_B=True, tri=1).numpy()
    ref = og.matmul_add(q, k, None, False, True)
    want = og.matmul_add(q, k, None, False, True, rounded=False)
    assert_error_floor(s1[:, on_or_below], want[:, on_or_below],
                       og.matmul_add_fma(q, k, None, False, True)[:, on_or_below])
    above = s1[:, ~on_or_below]
    assert np.all((above == 0) | np.isclose(above, ref[:, ~on_or_below], rtol=1e-4, atol=1e-3))
    # tri 2: P V with P lower triangular; tri 3: P^T V
    s2 = F().matmul_add(up(P), up(k), None, tri=2).numpy()
    check(s2, P, k)
    s3 = F().matmul_add(up(P), up(k), None, transpose_A=True, tri=3).numpy()
    check(s3, P, k, None, True, False)
    # equal to the untriangular product bit for bit (only exact zeros skipped)
    full2 = F().matmul_add(up(P), up(k), None).numpy()
    assert np.array_equal(s2, full2)
    # the zero triangle is never used: NaN there changes nothing
    Pn = P.copy()
    Pn[:, ~on_or_below] = np.nan
    assert np.array_equal(F().matmul_add(up(Pn), up(k), None, tri=2).numpy(), s2)
    assert np.array_equal(F().matmul_add(up(Pn), up(k), None, transpose_A=True, tri=3).numpy(),
                          s3)
    with pytest.raises(ValueError):
        F().matmul_add(up(q), up(k), up(np.zeros(S)), transpose_B=True, tri=1)


def test_matmul_explicit_splits_empty_k(device):
    # K == 0 with an explicit split count: nothing to split, C = bias
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    M, N = 5, 3
    bias = rng(5).standard_normal(N).astype(np.float32)
    A, B, tbias = up(np.ones((M, 1))), up(np.ones((1, N))), up(bias)
    P = C.c_void_p
    for code in (1, 2, 4, 9):
        out = empty([M, N])
        lib.call("wxx_matmul_add", P(A.data_ptr()), P(B.data_ptr()), P(tbias.data_ptr()),
                 P(out.data_ptr()), M, N, 0, 1, 0, 0, 0, 1, 0, 0, code | (3 << 8))
        assert np.array_equal(out.numpy(), np.broadcast_to(bias, (M, N)))


@pytest.mark.parametrize("sbias_kind", ["shared", "padded"])
def test_matmul_per_batch_bias_strides(device, sbias_kind):
    # bias_mode 3 with a batch stride other than M * N over a shared B (the
    # batch must not be folded into M then): stride 0 = one (M, N) bias for
    # every batch; a padded stride leaves a gap between the batches' biases
    import ctypes as C

    from wxx_amd.backend import lib
    from wxx_amd.functional._common import empty

    b, M, K, N = 3, 40, 24, 36
    r = rng(77)
    A = r.standard_normal((b, M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    sb = 0 if sbias_kind == "shared" else M * N + 17
    store = r.standard_normal(sb * (b - 1) + M * N).astype(np.float32)
    bias = np.stack([store[i * sb:i * sb + M * N].reshape(M, N) for i in range(b)])
    tA, tB, tbias = up(A), up(B), up(store)
    out = empty([b, M, N])
    P = C.c_void_p
    lib.call("wxx_matmul_add", P(tA.data_ptr()), P(tB.data_ptr()), P(tbias.data_ptr()),
             P(out.data_ptr()), M, N, K, b, M * K, 0, sb, 3, 0, 0, 0)
    check(out.numpy(), A, B, bias)
