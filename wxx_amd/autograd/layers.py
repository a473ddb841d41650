"""Differentiable loss, dropout and embedding (reference src/wxx/autograd/layers.py:6-71)."""

from .. import functional
from .function import Function


class CrossEntropyLoss(Function):
    """Per-row softmax cross-entropy; backward scales the fused dlogits by ``g``."""

    def forward(self, tensor1, tensor2):
        loss, grad = functional.cceloss(tensor1, tensor2)
        loss.requires_grad = any(self.needs_input_grad)
        return self.attach(loss, grad=grad)

    def backward(self, g):
        # one gradient: the Function is built with the logits only
        # (CrossEntropyLoss(prediction), reference nn/loss.py:28)
        grad, self.grad = self.grad, None
        return functional.pointwise(grad, g, 2)


class Dropout(Function):
    def forward(self, tensor1, p=0.2):
        out, seed = functional.dropout(tensor1, p)
        out.requires_grad = tensor1.requires_grad
        return self.attach(out, p=p, seed=seed)

    def backward(self, g):
        if not any(self.needs_input_grad):
            return None
        return functional.dropoutdx(g, self.p, self.seed)


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
