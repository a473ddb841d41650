"""GPT-2-style decoder-only language model (reference src/wxx/nn/gpt.py:1-174).

The module tree is the state_dict contract and matches the reference name
for name: ``tok_emb``, ``pos_emb``, ``blocks.<i>.{ln1, attn.{q,k,v,out},
ln2, mlp.0, mlp.2}``, ``ln_f`` and a ``head`` tied to the token embedding
(or an untied bias-free Linear).  Blocks are pre-LayerNorm: attention and
the 4x GELU MLP each add a dropped-out residual.

The causal mask is one (max_len, max_len) device tensor, 0 on and below the
diagonal and -1e9 above, narrowed for shorter sequences.  It is marked as
causal so that MultiHeadAttention may skip the work whose results the mask
zeroes (the numbers do not change).
"""

import numpy as np

from .. import functional
from ..backend import context
from ..functional.utils import from_numpy
from ..Tensor import Tensor
from .module import (
    GELU,
    Dropout,
    Embedding,
    LayerNorm,
    Linear,
    Module,
    ModuleList,
    MultiHeadAttention,
    Sequential,
    TiedLinear,
)

_MASKED = -1e9


class GPT2Block(Module):
    """x + drop(attn(ln1 x)), then + drop(mlp(ln2 x))."""

    def __init__(self, d_model, n_heads, dropout=0.1):
        super().__init__()
        self.ln1 = LayerNorm(d_model)
        self.attn = MultiHeadAttention(d_model, n_heads)
        self.ln2 = LayerNorm(d_model)
        hidden = 4 * d_model
        self.mlp = Sequential(Linear(d_model, hidden), GELU(), Linear(hidden, d_model))
        self.drop = Dropout(dropout)

    def forward(self, x, mask=None):
        attended = x + self.drop(self.attn(self.ln1(x), mask))
        return attended + self.drop(self.mlp(self.ln2(attended)))


def _mark_causal(t):
    t._causal = True
    return t


def _sample_rows(logits, temperature, top_k, rng):
    """One id per row of (batch, vocab) float64 logits: the argmax at
    temperature 0, else a draw from softmax(logits / T) restricted to the
    top_k largest (all values tied with the k-th are kept), by inverse CDF
    with one uniform per row (a row whose total rounds below the draw takes
    id 0)."""
    if temperature == 0.0:
        return logits.argmax(axis=-1)
    z = logits / temperature
    vocab = z.shape[-1]
    if top_k is not None and int(top_k) < vocab:
        kth = np.sort(z, axis=-1)[:, vocab - int(top_k)]
        z = np.where(z < kth[:, None], -np.inf, z)
    w = np.exp(z - z.max(axis=-1, keepdims=True))
    cdf = np.cumsum(w / w.sum(axis=-1, keepdims=True), axis=-1)
    u = rng.random((z.shape[0], 1))
    above = cdf > u
    return np.where(above.any(axis=-1), above.argmax(axis=-1), 0)


class GPT2(Module):
    def __init__(self, vocab_size, d_model=256, n_heads=8, n_layers=6, max_len=256, dropout=0.1,
                 tie_weights=True):
        super().__init__()
        self.vocab_size = vocab_size
        self.max_len = max_len
        self.tok_emb = Embedding(vocab_size, d_model, init_std=0.02)
        self.pos_emb = Embedding(max_len, d_model, init_std=0.02)
        self.blocks = ModuleList([GPT2Block(d_model, n_heads, dropout) for _ in range(n_layers)])
        self.ln_f = LayerNorm(d_model)
        if tie_weights:
            self.head = TiedLinear(self.tok_emb)
        else:
            self.head = Linear(d_model, vocab_size, bias=False)
        self._init_weights()
        self._causal_mask_cache = None

    def _init_weights(self):
        """GPT-2's init: every matrix N(0, 0.02) (the embeddings already are),
        every bias 0; LayerNorm keeps gamma 1, beta 0."""
        embeddings = ("tok_emb.weight", "pos_emb.weight")
        for name, p in self.named_parameters():
            if name.endswith(embeddings):
                continue
            if len(p.shape) > 1:
                functional.assign(p, functional.normal(0, 0.02, p.shape))
            elif name.endswith("bias"):
                functional.assign(p, 0.0)

    def causal_mask(self, seq):
        """(seq, seq) additive mask: 0 where key <= query, -1e9 above the diagonal."""
        if self._causal_mask_cache is None:
            full = np.triu(np.full((self.max_len, self.max_len), _MASKED, np.float32), k=1)
            self._causal_mask_cache = _mark_causal(from_numpy(full))
        mask = self._causal_mask_cache
        if seq != self.max_len:
            mask = _mark_causal(mask.narrow(0, 0, seq).narrow(1, 0, seq))
        return mask

    def forward(self, x, mask=None):
        seq = x.shape[1]
        if seq > self.max_len:
            raise ValueError(f"sequence length {seq} > max_len {self.max_len}")
        positions = from_numpy(np.arange(seq, dtype=np.uint32)[None, :], dtype=np.uint32)
        h = self.tok_emb(x) + self.pos_emb(positions)
        mask = self.causal_mask(seq) if mask is None else mask
        for block in self.blocks:
            h = block(h, mask)
        return self.head(self.ln_f(h))

    def generate(self, prompt, max_new_tokens=64, temperature=1.0, top_k=None, stop_token=None,
                 rng=None):
        """Extend a (batch, seq) or (seq,) prompt by up to ``max_new_tokens``
        sampled ids (never beyond ``max_len`` in total), stopping early once
        every row emits ``stop_token``; returns all ids as uint32.  Runs in
        inference mode (no dropout, no graph) and restores the caller's mode."""
        ids = prompt.numpy() if isinstance(prompt, Tensor) else np.asarray(prompt)
        ids = np.array(ids, dtype=np.uint32, ndmin=2, copy=True)
        if ids.ndim != 2:
            raise ValueError(f"prompt must be 1D or 2D, got shape {ids.shape}")
        if ids.shape[1] == 0:
            raise ValueError("prompt must contain at least one token")
        if ids.shape[1] > self.max_len:
            raise ValueError(f"prompt length {ids.shape[1]} > max_len {self.max_len}")
        if temperature < 0:
            raise ValueError("temperature must be non-negative")
        rng = rng if rng is not None else np.random.default_rng()
        budget = min(int(max_new_tokens), self.max_len - ids.shape[1])
        saved_mode, context.MODE = context.MODE, 1
        try:
            for _ in range(budget):
                logits = self.forward(from_numpy(ids, dtype=np.uint32)).numpy()
                nxt = _sample_rows(logits[:, -1, :].astype(np.float64), temperature, top_k,
                                   rng).astype(np.uint32)
                ids = np.concatenate([ids, nxt[:, None]], axis=1)
                if stop_token is not None and bool(np.all(nxt == stop_token)):
                    break
        finally:
            context.MODE = saved_mode
        return ids


__all__ = ["GPT2", "GPT2Block"]
