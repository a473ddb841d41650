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
