"""Oracle: the reference's training (autograd) paths on the CPU, restated with torch CPU ops.
TEST INFRASTRUCTURE ONLY (imported by tests/; never by the product).

  SparseRecurrent    _SparseRecurrent, CPU branch: y = A h; grad_h = A^T grad_y;   chessfly/brain.py:66-99
                     grad_w[e] = sum_b h[col_e, b] grad_y[row_e, b] by gathers
  literal_grad       ConnectomeRNN.forward under autograd                      chessfly/brain.py:224-229
  constants_grad     ConnectomeRNN._constants under autograd                   chessfly/brain.py:238-252
  cone_grad          ConnectomeRNN.forward_io under autograd (float32 path)    chessfly/brain.py:289-329
  model_grad         FlyChessNet.forward under autograd, layers separately     chessfly/model.py:95-105
  train_loss         the loss of train_step: masked policy cross-entropy plus
                     value cross-entropy (q_ratio 0)                           chessfly/train.py:126-132
  dense_literal      the recurrence with W dense (tests/test_core.py:20-25), the independent check

Parameters are leaf tensors of a `BrainArrays` / `HeadArrays` with requires_grad set by the caller; the
dtype follows the inputs (float64 for the pinning checks, float32 beside the device).
"""

from __future__ import annotations

import dataclasses

import torch
import torch.nn.functional as F

from .forward import BrainArrays, HeadArrays, _crow, edge_weights, norm
from .lightcone import Cone


@dataclasses.dataclass
class Csr:
    """A CSR matrix structure with its row of every non-zero, and the transposed structure on demand."""
    crow: torch.Tensor    # rows + 1
    col: torch.Tensor     # nnz
    row: torch.Tensor     # nnz
    shape: tuple

    def mat(self, w: torch.Tensor) -> torch.Tensor:
        return torch.sparse_csr_tensor(self.crow, self.col, w, self.shape, check_invariants=False)

    def mat_t(self, w: torch.Tensor) -> torch.Tensor:
        if getattr(self, "_t", None) is None:          # the transposed structure, sorted once per matrix
            order = torch.argsort(self.col * self.shape[0] + self.row, stable=True)
            self._t = (order, _crow(self.col[order], self.shape[1]), self.row[order])
        order, crow, col = self._t
        return torch.sparse_csr_tensor(crow, col, w[order], self.shape[::-1], check_invariants=False)


def full_csr(b: BrainArrays) -> Csr:
    cached = getattr(b, "_csr", None)
    if cached is None:
        cached = Csr(_crow(b.post, b.n), b.pre, b.post, (b.n, b.n))
        object.__setattr__(b, "_csr", cached)
    return cached


def sub_csr(op) -> Csr:
    cached = getattr(op, "_csr", None)
    if cached is None:
        t = lambda a: torch.as_tensor(a)
        cached = Csr(t(op.crow), t(op.pre), t(op.post), tuple(op.shape))
        object.__setattr__(op, "_csr", cached)
    return cached


class SparseRecurrent(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, w, op: Csr):
        ctx.save_for_backward(h, w)
        ctx.op = op
        return op.mat(w) @ h

    @staticmethod
    def backward(ctx, grad_y):
        h, w = ctx.saved_tensors
        op = ctx.op
        grad_y = grad_y.contiguous()
        grad_h = op.mat_t(w) @ grad_y if ctx.needs_input_grad[0] else None
        grad_w = (h[op.col] * grad_y[op.row]).sum(1) if ctx.needs_input_grad[1] else None
        return grad_h, grad_w, None


def literal_grad(b: BrainArrays, u: torch.Tensor, steps: int) -> torch.Tensor:
    """h after `steps` updates of lerp(h, clamp(W h + b + u, 0, H), alpha) from h = 0, differentiable."""
    alpha = torch.sigmoid(b.alpha_logit.to(u.dtype)).unsqueeze(1)
    w = edge_weights(b, u.dtype)
    drive = b.bias.to(u.dtype).unsqueeze(1) + u
    op = full_csr(b)
    h = torch.zeros_like(drive)
    for _ in range(steps):
        x = (SparseRecurrent.apply(h, w, op) + drive).clamp(0, b.h_max)
        h = torch.lerp(h, x, alpha)
    return h


def dense_literal(b: BrainArrays, u: torch.Tensor, steps: int) -> torch.Tensor:
    """The same recurrence with W as a dense matrix and (B, N) state (tests/test_core.py:20-25); u (B, N)."""
    w = edge_weights(b, u.dtype)
    mat = torch.zeros(b.n, b.n, dtype=u.dtype).index_put((b.post, b.pre), w, accumulate=True)
    alpha = torch.sigmoid(b.alpha_logit.to(u.dtype))
    h = torch.zeros_like(u)
    for _ in range(steps):
        h = (1 - alpha) * h + alpha * torch.relu(h @ mat.T + b.bias.to(u.dtype) + u).clamp(max=b.h_max)
    return h


def constants_grad(b: BrainArrays, cone: Cone, w: torch.Tensor, alpha: torch.Tensor):
    full = full_csr(b)
    bias = b.bias.to(w.dtype).unsqueeze(1)
    c = torch.zeros(b.n, 1, dtype=w.dtype)
    cs, ks = [c], [None]
    for t in range(1, cone.steps + 1):
        s = SparseRecurrent.apply(c, w, full) if t > 1 else torch.zeros_like(c)
        k = (s + bias)[torch.as_tensor(cone.rows[t])]
        op = cone.ops[t]
        if op is not None:
            k = k - SparseRecurrent.apply(c[torch.as_tensor(cone.rows[t - 1])], w[torch.as_tensor(op.edges)],
                                          sub_csr(op))
        ks.append(k)
        c = torch.lerp(c, (s + bias).clamp(0, b.h_max), alpha)
        cs.append(c)
    return cs, ks


def cone_grad(b: BrainArrays, cone: Cone, u_in: torch.Tensor) -> torch.Tensor:
    """forward_io under autograd: u_in (len(in_idx), B) -> (len(out_idx), B)."""
    t_ = lambda a: torch.as_tensor(a)
    batch = u_in.shape[1]
    w = edge_weights(b, u_in.dtype)
    alpha = torch.sigmoid(b.alpha_logit.to(u_in.dtype)).unsqueeze(1)
    cs, ks = constants_grad(b, cone, w, alpha)
    h = None
    for t in range(1, cone.steps + 1):
        rows, op = t_(cone.rows[t]), cone.ops[t]
        if op is None:
            x = ks[t].expand(-1, batch)
        else:
            x = SparseRecurrent.apply(h, w[t_(op.edges)], sub_csr(op)) + ks[t]
        x = x.index_add(0, t_(cone.u_pos[t]), u_in[t_(cone.u_src[t])]).clamp(0, b.h_max)
        prev = cs[t - 1][rows].expand(-1, batch)
        if len(cone.keep_next[t]):
            prev = prev.index_copy(0, t_(cone.keep_next[t]), h[t_(cone.keep_prev[t])])
        h = torch.lerp(prev, x, alpha[rows])
    out = cs[cone.steps][t_(cone.out_idx)].expand(-1, batch)
    return out.index_copy(0, t_(cone.out_pos), h[t_(cone.out_src)])


def model_grad(heads: HeadArrays, b: BrainArrays, cone: Cone, x: torch.Tensor):
    """FlyChessNet.forward with autograd (eval-mode normaliser): x (B, F) -> logits, wdl."""
    k = heads.n_base
    enc = F.linear(x[:, :k], heads.enc_w[:, :k], heads.enc_b)
    u_in = (enc * heads.input_gain).T.contiguous()
    r = norm(heads, cone_grad(b, cone, u_in).T)
    logits = (F.linear(r, heads.policy_w, heads.policy_b) + F.linear(r, heads.from_w, heads.from_b)[:, heads.move_from]
              + F.linear(r, heads.to_w, heads.to_b)[:, heads.move_to])
    return logits, F.linear(r, heads.value_w, heads.value_b)


def train_loss(logits: torch.Tensor, wdl_logits: torch.Tensor, pi: torch.Tensor, legal: torch.Tensor,
               wdl: torch.Tensor) -> torch.Tensor:
    """policy_loss + value_loss of train_step with q_ratio = 0 (train.py:126-132)."""
    logp = logits.masked_fill(~legal, -1e9).log_softmax(-1)
    return -(pi * logp).sum(-1).mean() + F.cross_entropy(wdl_logits, wdl)
