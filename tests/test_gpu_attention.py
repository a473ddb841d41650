"""GPU: the fused attention kernels against the float64 attention oracle.

The oracle (oracle/attention.py, pinned against torch's float64 attention)
follows the reference's composition (nn/module.py:460-495).  The fused
kernels sum in another order than that composition, so outputs and
gradients are held to the fp32 error floor: within 4x the largest error of
the same composition computed in float32 (plus rtol 1e-4 of the value).
Dropout masks are bit-exact by construction (same hash of the same flat
index), which the p > 0 cases check through the values.
"""

import numpy as np
import pytest

from conftest import assert_error_floor, rng
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def W():
    import wxx_amd

    return wxx_amd


CASES = [
    # B, S, H, d, causal, p
    (2, 128, 8, 32, True, 0.0),    # config-1 attention
    (1, 256, 4, 64, True, 0.1),
    (2, 100, 2, 64, False, 0.0),   # ragged: partial row blocks
    (1, 77, 2, 128, True, 0.0),
    (1, 130, 3, 32, False, 0.2),
    (1, 1, 1, 64, True, 0.0),      # a single position
    (3, 64, 2, 32, True, 0.5),
    (1, 300, 2, 64, True, 0.0),    # several 128-row blocks, causal skipping
]


@pytest.mark.parametrize("B,S,H,d,causal,p", CASES)
def test_fused_attention_matches_oracle(device, B, S, H, d, causal, p):
    F = W().functional
    r = rng(B * 1000 + S)
    q, k, v, do = (r.standard_normal((B, S, H * d)).astype(np.float32) for _ in range(4))
    seed = 987654321
    out, lse = F.fused_attention(*(F.from_numpy(t) for t in (q, k, v)), H, causal, p, seed)
    want = oa.attention(q, k, v, H, causal, p, seed)
    ref32 = oa.attention(q, k, v, H, causal, p, seed, dtype=np.float32)
    assert_error_floor(out.numpy(), want, ref32, msg="out")
    grads = F.fused_attention_backward(*(F.from_numpy(t) for t in (q, k, v)), out,
                                       F.from_numpy(do), lse, H, causal, p, seed)
    want_g = oa.attention_grads(q, k, v, do, H, causal, p, seed)
    ref_g = oa.attention_grads(q, k, v, do, H, causal, p, seed, dtype=np.float32)
    for name, g, w, r32 in zip(("dq", "dk", "dv"), grads, want_g, ref_g):
        # at S = 1 (one key per query) dq and dk are exact zeros in the
        # composition, P (dP - D) with P = 1, and sums that cancel to within
        # rounding in the fused order: the north star's atol covers those
        assert_error_floor(g.numpy(), w, r32, msg=name, atol=1e-5 if S == 1 else 0.0)


def test_fused_attention_is_deterministic_and_rejects_bad_heads(device):
    F = W().functional
    r = rng(3)
    q, k, v = (F.from_numpy(r.standard_normal((2, 96, 128)).astype(np.float32)) for _ in range(3))
    a, la = F.fused_attention(q, k, v, 2, True, 0.1, 5)
    b, lb = F.fused_attention(q, k, v, 2, True, 0.1, 5)
    assert np.array_equal(a.numpy(), b.numpy()) and np.array_equal(la.numpy(), lb.numpy())
    with pytest.raises(ValueError, match="D / n_heads"):
        F.fused_attention(q, k, v, 8, True)  # head size 16 is not built


@pytest.mark.parametrize("dropout", [0.0, 0.1])
def test_mha_module_fused_path_matches_composed_path(device, dropout):
    # the same module through the fused kernels (marked causal mask) and
    # through the composed products + softmax (the same mask, unmarked):
    # outputs and parameter gradients agree to the fp32 error floor, and the
    # host RNG advances by one draw per call either way
    import random

    wxx = W()
    F = wxx.functional
    B, S, D, H = 2, 48, 128, 4
    m = wxx.nn.MultiHeadAttention(D, H, dropout=dropout)
    r = rng(8)
    x = r.standard_normal((B, S, D)).astype(np.float32)
    g = r.standard_normal((B, S, D)).astype(np.float32)
    mask_np = np.triu(np.full((S, S), -1e9, np.float32), k=1)
    marked = wxx.nn.gpt._mark_causal(F.from_numpy(mask_np))
    plain = F.from_numpy(mask_np)

    def run(mask):
        params = [p for _, p in m.parameters()]
        for p in params:
            p.grad = None
        xt = wxx.Tensor(list(x.shape), data=x, requires_grad=True)
        random.seed(4)
        out = m(xt, mask)
        after = random.random()
        (out * F.from_numpy(g)).sum().backward()
        return out.numpy(), [p.grad.numpy() for p in params], xt.grad.numpy(), after

    fo, fg, fx, fa = run(marked)
    co, cg, cx, ca = run(plain)
    assert fa == ca
    scale = np.abs(co).max()
    assert np.abs(fo - co).max() <= 1e-5 * scale
    for a, b in zip(fg + [fx], cg + [cx]):
        assert np.abs(a - b).max() <= 1e-4 * np.abs(b).max()
