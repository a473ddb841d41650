"""Differentiable loss, dropout and embedding (reference src/wxx/autograd/layers.py:6-71)."""

from .. import functional
from .function import Function


class CrossEntropyLoss(Function):
    """Per-row softmax cross-entropy; the logits gradient is the fused
    dlogits scaled by ``g``.  Rows up to 65536 defer dlogits to the backward
    (one pass writing the scaled gradient; the forward keeps each row's max
    and exp-sum), longer rows keep cceloss's eager dlogits."""

    def forward(self, tensor1, tensor2):
        deferred = functional.cceloss_stats(tensor1, tensor2) if any(self.needs_input_grad) \
            else None
        if deferred is not None:
            loss, stats, logits, targets = deferred
            loss.requires_grad = True
            return self.attach(loss, stats=stats, logits=logits, targets=targets, grad=None)
        loss, grad = functional.cceloss(tensor1, tensor2)
        loss.requires_grad = any(self.needs_input_grad)
        return self.attach(loss, grad=grad, stats=None)

    def backward(self, g):
        # one gradient: the Function is built with the logits only
        # (CrossEntropyLoss(prediction), reference nn/loss.py:28)
        if self.stats is not None:
            out = functional.cceloss_grad(self.logits, self.targets, self.stats, g)
            self.stats = self.logits = self.targets = None
            return out
        grad, self.grad = self.grad, None
        return functional.pointwise(grad, g, 2)


class Dropout(Function):
    def forward(self, tensor1, p=0.2):
        # at p == 0 the output shares the input's storage (no copy); the
        # engine never writes into activations or gradients in place
        out, seed = functional.dropout(tensor1, p, share_at_zero=True)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, p=p, seed=seed)

    def backward(self, g):
        if not any(self.needs_input_grad):
            return None
        return functional.dropoutdx(g, self.p, self.seed, share_at_zero=True)


class Embedding(Function):
    def forward(self, tensor1, tensor2, n_token, embed_dim, vocab_size):
        out = functional.embed(tensor1, tensor2, n_token, embed_dim)
        out.requires_grad = tensor1.requires_grad or tensor2.requires_grad
        return self.attach(out, ids=tensor1, n_token=n_token, embed_dim=embed_dim,
                           vocab_size=vocab_size)

    def backward(self, g):
        if not any(self.needs_input_grad):
            return None, None
        ids, self.ids = self.ids, None
        return None, functional.embeddx(g, ids, self.n_token, self.embed_dim, self.vocab_size)


class FusedAttention(Function):
    """Per head softmax(q k^T / sqrt(d) [+ causal mask]), dropout, times v, as
    one Function over the (B, S, D) projections: the reference's head
    permutes, score matmul, scale, mask add, softmax, dropout and value
    matmul (nn/module.py:460-495).  Inputs: q, k, v."""

    def forward(self, q, k, v, n_heads, causal, p=None):
        # p None: inference (the reference's Dropout is the identity and draws
        # no seed); otherwise one seed per call, drawn even at p == 0
        seed = 0 if p is None else functional.attention_ops.draw_seed()
        p = 0.0 if p is None else float(p)
        out, lse = functional.fused_attention(q, k, v, n_heads, causal, p, seed)
        out.requires_grad = any(t.requires_grad for t in (q, k, v))
        # the output is kept through a second tensor over its storage, so the
        # output does not reference its creator through the saved state
        saved_out = functional.layers._same_values(out) if out.requires_grad else None
        return self.attach(out, q=q, k=k, v=v, o=saved_out, lse=lse, seed=seed,
                           n_heads=n_heads, causal=causal, p=p)

    def backward(self, g):
        if not any(self.needs_input_grad):
            return None, None, None
        grads = functional.fused_attention_backward(self.q, self.k, self.v, self.o, g, self.lse,
                                                    self.n_heads, self.causal, self.p, self.seed)
        self.q = self.k = self.v = self.o = self.lse = None
        return tuple(d if need else None for d, need in zip(grads, self.needs_input_grad))
