"""Differentiable loss, dropout and embedding (reference src/wxx/autograd/layers.py:6-71)."""

from .. import functional
from ..functional._common import empty
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


class swiglu_padded(Function):
    """``w3(silu(x w1) * (x w2))`` over (T, d) rows with the hidden width
    padded to ``hp`` (a multiple of 128) inside the op: zero columns of w1 /
    w2 and zero rows of w3, so the padded activations stay exact zeros and
    every product runs on the direct-to-LDS tiles (a width like Hyena's 682
    is neither a multiple of 64 nor 16-byte aligned per row).  Built as
    ``swiglu_padded(x, w1, w2, w3)``; the parameters and their gradients keep
    their (d, hidden) / (hidden, d) shapes.  The gate silu(a) b and its
    backward are one kernel each (``swiglu_gate``), equal bit for bit to the
    composed sigmoid / product ops and their backwards."""

    # tile codes measured on MI355X for T = 65536, d = 256, hp = 768:
    # 128 x 64 direct-to-LDS tiles for the T-row products (x w1: 247 against
    # 284 us on 128 x 128), 128 x 128 ones over 21 K splits for the weight
    # gradients (250 against 335 us)
    ROWS_TILE = 13
    WGRAD_TILE = 11 + 256 * 21

    def forward(self, x, w1, w2, w3, hp):
        d, hid = w1.shape
        self.shape = list(x.shape)
        x2 = functional.reshape(x, [-1, d])
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        w1p = _pad_cols(w1, hp)
        w2p = _pad_cols(w2, hp)
        w3p = _pad_rows(w3, hp)
        # the direct-to-LDS tiles need 16-byte aligned operands: a view that
        # starts mid-vector takes the automatic choice instead
        t = self.ROWS_TILE if _aligned(x2) else 0
        a = functional.matmul_add(x2, w1p, None, tile=t)
        b = functional.matmul_add(x2, w2p, None, tile=t)
        h = functional.swiglu_gate(a, b)
        y = functional.matmul_add(h, w3p, None, tile=t)
        out = functional.reshape(y, self.shape[:-1] + [w3.shape[1]])
        out.requires_grad = any(v.requires_grad for v in (x, w1, w2, w3))
        return self.attach(out, x2=x2, a=a, b=b, h=h, w1p=w1p, w2p=w2p, w3p=w3p, hid=hid)

    def backward(self, dy):
        x2, a, b, h = self.x2, self.a, self.b, self.h
        w1p, w2p, w3p, hid = self.w1p, self.w2p, self.w3p, self.hid
        self.x2 = self.a = self.b = self.h = None
        self.w1p = self.w2p = self.w3p = None
        dy2 = functional.reshape(dy, [-1, w3p.shape[1]])
        if not dy2.is_contiguous():
            dy2 = dy2.contiguous()
        ok = _aligned(x2, dy2)
        t, tw = (self.ROWS_TILE, self.WGRAD_TILE) if ok else (0, 0)
        dh = functional.matmul_add(dy2, w3p, None, transpose_B=True, tile=t)
        dw3 = None
        if self.needs_input_grad[3]:
            dw3 = functional.contiguous(
                functional.matmul_add(h, dy2, None, transpose_A=True, tile=tw)[:hid])
        da, db = functional.swiglu_gate_backward(dh, a, b)
        dw1 = dw2 = dx = None
        if self.needs_input_grad[1]:
            dw1 = functional.contiguous(
                functional.matmul_add(x2, da, None, transpose_A=True, tile=tw)[:, :hid])
        if self.needs_input_grad[2]:
            dw2 = functional.contiguous(
                functional.matmul_add(x2, db, None, transpose_A=True, tile=tw)[:, :hid])
        if self.needs_input_grad[0]:
            dx = functional.matmul_add(da, w1p, None, transpose_B=True, tile=t)
            dx = functional.matmul_add(db, w2p, dx, transpose_B=True, tile=t)
            dx = functional.reshape(dx, self.shape)
        return dx, dw1, dw2, dw3


def _aligned(*ts):
    return all(t.data_ptr() % 16 == 0 for t in ts)


def _pad_cols(w, width):
    """(r, c) -> (r, width) with zero columns c..width-1 (on the device)."""
    out = empty([w.shape[0], width])
    functional.assign(out, 0.0)
    functional.assign(out[:, :w.shape[1]], w)
    return out


def _pad_rows(w, rows):
    """(r, c) -> (rows, c) with zero rows r..rows-1 (on the device)."""
    out = empty([rows, w.shape[1]])
    functional.assign(out, 0.0)
    functional.assign(out[:w.shape[0]], w)
    return out
