"""Pin the GPT-2 train-step oracle (CPU-only) against torch autograd in float64.

The torch model is written independently from torch's own layers (F.layer_norm,
F.gelu(approximate="tanh"), F.softmax, F.cross_entropy); on inputs where the
reference's special cases (zero variance, |x| > 10 GELU clamps) do not occur it
must give the same loss and the same gradient for every parameter.
"""

import numpy as np
import pytest

from conftest import assert_close, rng
from oracle import models as om

torch = pytest.importorskip("torch")
TF = torch.nn.functional


def _params(V, D, L, max_len, seed=0):
    r = rng(seed)
    P = {"tok_emb.weight": r.normal(0, 0.02, (V, D)), "pos_emb.weight": r.normal(0, 0.02, (max_len, D))}
    for i in range(L):
        p = f"blocks.{i}."
        for n in ("q", "k", "v", "out"):
            P[p + f"attn.{n}.weight"] = r.normal(0, 0.2, (D, D))
        P[p + "mlp.0.weight"] = r.normal(0, 0.2, (D, 4 * D))
        P[p + "mlp.0.bias"] = r.normal(0, 0.1, 4 * D)
        P[p + "mlp.2.weight"] = r.normal(0, 0.2, (4 * D, D))
        P[p + "mlp.2.bias"] = r.normal(0, 0.1, D)
        for ln in ("ln1", "ln2"):
            P[p + f"{ln}.weightg"] = 1.0 + r.normal(0, 0.1, D)
            P[p + f"{ln}.weightb"] = r.normal(0, 0.1, D)
    P["ln_f.weightg"] = 1.0 + r.normal(0, 0.1, D)
    P["ln_f.weightb"] = r.normal(0, 0.1, D)
    return P


def _torch_gpt2(T, x, y, H, L):
    B, S = x.shape
    V, D = T["tok_emb.weight"].shape
    hd = D // H
    mask = torch.triu(torch.full((S, S), -1e9, dtype=torch.float64), diagonal=1)
    h = T["tok_emb.weight"][x] + T["pos_emb.weight"][:S][None]
    for i in range(L):
        p = f"blocks.{i}."
        a = TF.layer_norm(h, (D,), T[p + "ln1.weightg"], T[p + "ln1.weightb"], eps=1e-5)
        q, k, v = (((a @ T[p + f"attn.{n}.weight"]).view(B, S, H, hd).transpose(1, 2))
                   for n in ("q", "k", "v"))
        att = TF.softmax(q @ k.transpose(-1, -2) / np.sqrt(hd) + mask, dim=-1)
        o = (att @ v).transpose(1, 2).reshape(B, S, D)
        h = h + o @ T[p + "attn.out.weight"]
        a2 = TF.layer_norm(h, (D,), T[p + "ln2.weightg"], T[p + "ln2.weightb"], eps=1e-5)
        m = TF.gelu(a2 @ T[p + "mlp.0.weight"] + T[p + "mlp.0.bias"], approximate="tanh")
        h = h + m @ T[p + "mlp.2.weight"] + T[p + "mlp.2.bias"]
    hf = TF.layer_norm(h, (D,), T["ln_f.weightg"], T["ln_f.weightb"], eps=1e-5)
    logits = hf @ T["tok_emb.weight"].T
    return TF.cross_entropy(logits.reshape(-1, V), y.reshape(-1))


@pytest.mark.parametrize("V,D,H,L,B,S", [(50, 16, 2, 2, 2, 5), (37, 24, 3, 1, 3, 7)])
def test_gpt2_oracle_matches_torch_autograd(V, D, H, L, B, S):
    P = _params(V, D, L, max_len=S + 3, seed=V)
    x = rng(1).integers(0, V, (B, S))
    y = rng(2).integers(0, V, (B, S))
    loss, G = om.gpt2_loss_and_grads(P, x, y, H, L)
    T = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in P.items()}
    tl = _torch_gpt2(T, torch.tensor(x), torch.tensor(y), H, L)
    tl.backward()
    assert abs(loss - tl.item()) < 1e-12 * max(1.0, abs(loss))
    for k, t in T.items():
        assert_close(G[k], t.grad.numpy(), rtol=1e-9, atol=1e-12, msg=k)


def test_adamw_sequence_aliases_step_twice():
    p = {"a": np.array([1.0, -2.0]), "b": np.array([0.5])}
    g = {"a": np.array([0.1, 0.3]), "b": np.array([-1.0])}
    order = ["a", "b", "a"]  # "a" registered under two names
    states = [(np.zeros(2), np.zeros(2)), (np.zeros(1), np.zeros(1)), (np.zeros(2), np.zeros(2))]
    out = om.adamw_sequence(p, g, order, states, 1, 1e-2)
    once, _, _ = om.adamw_apply(p["a"], g["a"], 0, 0, 1e-2, 0.9, 0.999, 1e-7, 1e-4, 0.1, 1 - 0.999)
    twice, _, _ = om.adamw_apply(once, g["a"], 0, 0, 1e-2, 0.9, 0.999, 1e-7, 1e-4, 0.1, 1 - 0.999)
    assert_close(out["a"], twice, rtol=1e-14, atol=1e-15)
    assert not np.allclose(out["a"], once)


# ------------------------------------------------------------ ResNet18 / Hyena

from oracle import conv as oc  # noqa: E402
from oracle import hyena as oh  # noqa: E402
from oracle import norms as on  # noqa: E402
from oracle import resnet as orn  # noqa: E402


def _resnet_params(num_classes=5, seed=3):
    r = rng(seed)
    P, S = {}, {}

    def bn(name, c):
        P[name + ".weight"] = 1.0 + r.normal(0, 0.1, c)
        P[name + ".bias"] = r.normal(0, 0.1, c)
        S[name + ".running_mean"] = r.normal(0, 0.1, c)
        S[name + ".running_std"] = 1.0 + r.uniform(0, 0.1, c)

    P["conv1.W"] = r.normal(0, np.sqrt(2 / 147), (64, 3, 7, 7))
    bn("bn1", 64)
    cin = 64
    for li, cout in enumerate((64, 128, 256, 512), start=1):
        for bi in range(2):
            p = f"layer{li}.{bi}."
            stride = 2 if (bi == 0 and li > 1) else 1
            P[p + "conv1.W"] = r.normal(0, np.sqrt(2 / (9 * cin)), (cout, cin, 3, 3))
            bn(p + "bn1", cout)
            P[p + "conv2.W"] = r.normal(0, np.sqrt(2 / (9 * cout)), (cout, cout, 3, 3))
            bn(p + "bn2", cout)
            if bi == 0 and (stride != 1 or cin != cout):
                P[p + "shortcut.0.W"] = r.normal(0, np.sqrt(2 / cin), (cout, cin, 1, 1))
                bn(p + "shortcut.1", cout)
            cin = cout
    P["fc.weight"] = r.normal(0, 0.05, (512, num_classes))
    P["fc.bias"] = r.normal(0, 0.1, num_classes)
    return P, S


def test_resnet_oracle_ops_match_numpy_op_oracles():
    # the oracle's conv, training batchnorm (+ running statistics) and max-pool
    # gradient routing against the separately pinned numpy per-op oracles
    r = rng(5)
    x = r.standard_normal((3, 4, 9, 9))
    w = r.standard_normal((6, 4, 3, 3))
    got = TF.conv2d(torch.tensor(x), torch.tensor(w), stride=2, padding=1).numpy()
    assert_close(got, oc.conv2d(x, w, (2, 2), (1, 1), (1, 1)), rtol=1e-10, atol=1e-10)
    g, b = 1 + r.normal(0, 0.1, 4), r.normal(0, 0.1, 4)
    rm, rv = r.normal(0, 0.1, 4), 1 + r.uniform(0, 0.1, 4)
    y, nrm, nrv = orn.batchnorm_train(*(torch.tensor(a) for a in (x, g, b, rm, rv)))
    ey, _, _, erm, erv = on.batchnorm(x, g, b, rm, rv, True)
    assert_close(y.numpy(), ey, rtol=1e-5, atol=1e-6)
    assert_close(nrm.numpy(), erm, rtol=1e-5, atol=1e-7)
    assert_close(nrv.numpy(), erv, rtol=1e-5, atol=1e-7)
    # max pool with ties (zeros after relu): the gradient lands on the
    # window's first maximum, as the reference's index rule says
    xp = np.maximum(r.standard_normal((2, 3, 8, 8)), 0.0).astype(np.float32)
    xt = torch.tensor(xp.astype(np.float64), requires_grad=True)
    out = TF.max_pool2d(xt, 3, stride=2, padding=1)
    dy = r.standard_normal(out.shape)
    out.backward(torch.tensor(dy))
    vals, idx = oc.pool2d(xp, (3, 3), (2, 2), (1, 1), False)
    assert_close(out.detach().numpy(), vals, rtol=0, atol=0)
    want = oc.pool2d_backward(dy, idx, xp.shape, (3, 3), (2, 2), (1, 1), False)
    assert_close(xt.grad.numpy(), want, rtol=1e-12, atol=1e-12)


def test_resnet_oracle_gradient_by_finite_differences():
    # directional derivative of the loss along a random unit direction of
    # every parameter at once (32 x 32 inputs reach 2 x 2 at layer4)
    P, S = _resnet_params()
    r = rng(6)
    x = r.standard_normal((4, 3, 32, 32))
    y = r.integers(0, 5, 4)
    loss, G, S2, _ = orn.resnet18_loss_and_grads(P, S, x, y)
    V = {k: r.standard_normal(v.shape) for k, v in P.items()}
    norm = np.sqrt(sum(float((v * v).sum()) for v in V.values()))
    V = {k: v / norm for k, v in V.items()}
    h = 1e-6

    def at(sign):
        Q = {k: torch.tensor(P[k] + sign * h * V[k]) for k in P}
        St = {k: torch.tensor(v) for k, v in S.items()}
        lg = orn.resnet18_forward(Q, St, torch.tensor(x))
        return float((torch.logsumexp(lg, 1) - lg[torch.arange(4), torch.tensor(y)]).mean())

    num = (at(1) - at(-1)) / (2 * h)
    ana = sum(float((G[k] * V[k]).sum()) for k in P)
    assert abs(num - ana) <= 1e-5 * (1 + abs(ana)), (num, ana)
    # a block's bn1 runs twice per forward on the same input: two EMA updates,
    # r2 = 0.81 r0 + 0.19 mu; a single block bn2 gets one, r1 = 0.9 r0 + 0.1 mu
    k = "layer1.0.bn1.running_mean"
    mu = (S2[k] - 0.81 * S[k]) / 0.19
    assert np.all(np.abs(mu) < 50)
    assert not np.allclose(S2[k], 0.9 * S[k] + 0.1 * mu)
    assert np.isfinite(loss)


def test_hyena_oracle_pieces():
    r = rng(7)
    # short conv against the numpy per-op oracle
    x, w, b = r.standard_normal((2, 5, 9)), r.standard_normal((5, 3)), r.standard_normal(5)
    got = oh.causal_short_conv(torch.tensor(x), torch.tensor(w), torch.tensor(b)).numpy()
    assert_close(got, oc.causal_conv1d(x, w, b), rtol=1e-12, atol=1e-12)
    # the FFT long convolution is the direct causal sum z * h
    z, hf = r.standard_normal((2, 3, 10)), r.standard_normal((3, 10))
    got = oh.fft_conv(torch.tensor(z), torch.tensor(hf)).numpy()
    want = np.array([[np.convolve(z[bb, d], hf[d])[:10] for d in range(3)] for bb in range(2)])
    assert_close(got, want, rtol=1e-10, atol=1e-10)
    # RMSNorm with and without the reference's row cap
    xr, g = r.standard_normal((3, 4, 6)), 1 + r.normal(0, 0.1, 6)
    xr[1, 2] = 0.0  # zero mean square: r = 0
    for cap in (0, 7):
        got = oh.rmsnorm(torch.tensor(xr), torch.tensor(g), row_cap=cap).numpy()
        want, _ = on.rmsnorm(xr, g, -1, row_cap=cap)
        assert_close(got, want, rtol=1e-5, atol=1e-6)
    # the positional encoding table of module.py:576-584
    pe = oh.positional_encoding(5, 3).numpy()
    assert pe.shape == (5, 7)
    assert_close(pe[:, 0], np.linspace(0, 1, 5), rtol=0, atol=1e-7)
    assert np.all(pe[:, 1] == 1.0) and np.all(pe[:, 4] == 0.0)
    # the reference test's known answer (tests/test_hyena.py:116-132)
    assert oh.hyena_param_count(2048, 256, 6, 4) == 6_468_864


def _hyena_params(V, D, L, order, seed=8, tie=True):
    r = rng(seed)
    hidden = int(2 * (4 * D) / 3)
    P = {"embed.weight": r.normal(0, 0.3, (V, D)), "norm.weight": 1 + r.normal(0, 0.1, D)}
    for li in range(L):
        p = f"layers.{li}."
        m = p + "mixer."
        P[p + "norm1.weight"] = 1 + r.normal(0, 0.1, D)
        P[p + "norm2.weight"] = 1 + r.normal(0, 0.1, D)
        P[m + "proj_v.weight"] = r.normal(0, 0.3, (D, D))
        P[m + "proj_x.weight"] = r.normal(0, 0.3, (D, order * D))
        P[m + "out_proj.weight"] = r.normal(0, 0.3, (D, D))
        P[m + "short_conv.weight"] = r.normal(0, 0.3, (D, 3))
        P[m + "short_conv.bias"] = r.normal(0, 0.1, D)
        P[m + "decay"] = r.uniform(0, 1, (order, D))
        for i in range(order):
            f = f"{m}filter_mlp.{i}.mlp."
            P[f + "0.weight"] = r.normal(0, 0.3, (17, 64))
            P[f + "0.bias"] = r.normal(0, 0.1, 64)
            P[f + "2.weight"] = r.normal(0, 0.1, (64, D))
            P[f + "2.bias"] = r.normal(0, 0.1, D)
        P[p + "feed_forward.w1.weight"] = r.normal(0, 0.3, (D, hidden))
        P[p + "feed_forward.w2.weight"] = r.normal(0, 0.3, (D, hidden))
        P[p + "feed_forward.w3.weight"] = r.normal(0, 0.3, (hidden, D))
    if not tie:
        P["head.weight"] = r.normal(0, 0.3, (D, V))
        P["head.bias"] = r.normal(0, 0.1, V)
    return P


@pytest.mark.parametrize("tie,cap", [(True, 0), (False, 0), (True, 9)])
def test_hyena_oracle_gradient_by_finite_differences(tie, cap):
    V, D, L, order, B, S = 11, 8, 2, 2, 2, 6
    P = _hyena_params(V, D, L, order, tie=tie)
    r = rng(9)
    ids, tg = r.integers(0, V, (B, S)), r.integers(0, V, (B, S))
    loss, G = oh.hyena_loss_and_grads(P, ids, tg, L, order, row_cap=cap, tie_weights=tie)
    Vd = {k: r.standard_normal(v.shape) for k, v in P.items()}
    h = 1e-6

    def at(sign):
        Q = {k: torch.tensor(P[k] + sign * h * Vd[k]) for k in P}
        return float(oh.cce_mean(oh.hyena_forward(Q, ids, L, order, row_cap=cap,
                                                  tie_weights=tie), tg))

    num = (at(1) - at(-1)) / (2 * h)
    ana = sum(float((G[k] * Vd[k]).sum()) for k in P)
    assert abs(num - ana) <= 1e-5 * (1 + abs(ana)), (num, ana)
    assert np.isfinite(loss)
    if cap:
        # rows at or beyond the cap give no gradient to the final norm's gamma
        # through them: the last token's logits are constant (zero)
        lg = oh.hyena_forward({k: torch.tensor(v) for k, v in P.items()}, ids, L, order,
                              row_cap=cap, tie_weights=tie).detach().numpy().reshape(-1, V)
        assert np.all(lg[cap:] == 0)


def test_resnet_oracle_replaying_its_own_decisions_changes_nothing():
    P, S = _resnet_params()
    r = rng(11)
    x = r.standard_normal((4, 3, 32, 32))
    y = r.integers(0, 5, 4)
    seen = {}
    l1, g1, _, lg1 = orn.resnet18_loss_and_grads(P, S, x, y, record=seen)
    _, idx = oc.pool2d(seen["pool_input"], (3, 3), (2, 2), (1, 1), False)
    forced = {"relu": [a > 0 for a in seen["relu_inputs"]], "pool": idx}
    l2, g2, _, lg2 = orn.resnet18_loss_and_grads(P, S, x, y, forced=forced)
    assert len(seen["relu_inputs"]) == 17
    assert l1 == l2
    assert np.array_equal(lg1, lg2)
    for k in g1:
        assert np.array_equal(g1[k], g2[k]), k
    # a planted wrong decision changes the gradients
    bad = {"relu": [m.copy() for m in forced["relu"]], "pool": idx}
    bad["relu"][3].reshape(-1)[:50] ^= True
    _, g3, _, _ = orn.resnet18_loss_and_grads(P, S, x, y, forced=bad)
    assert any(not np.array_equal(g1[k], g3[k]) for k in g1)


@pytest.mark.parametrize("causal,p", [(False, 0.0), (True, 0.0), (True, 0.3), (False, 0.25)])
def test_attention_oracle_against_torch(causal, p):
    # forward against torch's own float64 scaled_dot_product_attention (no
    # dropout), and forward + gradients against torch autograd of the
    # composition with the oracle's dropout mask as a constant multiplier
    from oracle import attention as oa
    from oracle.layers import dropout_keep

    B, S, H, d, seed = 2, 19, 3, 4, 1234
    r = rng(5)
    q, k, v, do = (r.standard_normal((B, S, H * d)) for _ in range(4))
    got = oa.attention(q, k, v, H, causal, p, seed)
    grads = oa.attention_grads(q, k, v, do, H, causal, p, seed)

    tq, tk, tv = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    split = lambda t: t.reshape(B, S, H, d).permute(0, 2, 1, 3)  # noqa: E731
    if p == 0:
        sd = TF.scaled_dot_product_attention(split(tq), split(tk), split(tv), is_causal=causal)
        assert_close(sd.permute(0, 2, 1, 3).reshape(B, S, H * d).detach().numpy(), got,
                     rtol=1e-12, atol=1e-12)
    scores = split(tq) @ split(tk).transpose(-1, -2) / np.sqrt(d)
    if causal:
        scores = scores.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    probs = torch.softmax(scores, -1)
    if p:
        keep = dropout_keep(B * H * S * S, seed, p).reshape(B, H, S, S)
        probs = probs * torch.tensor(keep / (1 - p), dtype=torch.float64)
    out = (probs @ split(tv)).permute(0, 2, 1, 3).reshape(B, S, H * d)
    assert_close(out.detach().numpy(), got, rtol=1e-12, atol=1e-12)
    out.backward(torch.tensor(do))
    for name, t, g in zip("qkv", (tq, tk, tv), grads):
        assert_close(g, t.grad.numpy(), rtol=1e-10, atol=1e-12, msg=f"d{name}")
    # dropout reaches the gradients (a dropped-out oracle is not the plain one)
    if p:
        plain = oa.attention_grads(q, k, v, do, H, causal, 0.0, seed)
        assert not np.allclose(plain[2], grads[2])
