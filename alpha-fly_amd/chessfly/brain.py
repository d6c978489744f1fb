"""Connectome-constrained rate RNN, evaluated by gfx950 HIP kernels.

    h[t+1] = (1 - alpha) * h[t] + alpha * clamp(W h[t] + b + u, 0, h_max)

Drop-in for chessfly/brain.py of the reference: same classes, constructor arguments, parameters, buffers
and method signatures (ConnectomeRNN.forward / forward_io / light_cone / edge_weights, LightCone and its
attributes).  What runs underneath is libflyeval.so:

* `forward` (chessfly/brain.py:211-223): the literal recurrence over the whole matrix, one fused kernel per
  step (SpMM + bias + input + clamp + lerp), float32.
* `forward_io` (brain.py:282-329): the light cone.  float16 input selects the deviation-from-rest path
  (brain.py:254-280): the resting trajectory and per-row constants are float32 and built once per weight
  version; only the position-dependent deviation is stored, in float16, and accumulated in float32.
  float32 input selects the float32 light-cone path.  Either way one fused kernel per step.
* `light_cone` (brain.py:126-173, 232-236): reach masks, row compaction and sub-matrix extraction on the
  device, integer and bit-exact with the reference's definition.

Training (autograd enabled, brain.py:66-99, 225-229, 238-252, 289-329) runs the reference's float32
recurrence under autograd with its sparse products on the device: `_SparseRecurrent` computes y = A h with
fly_spmm, the state gradient A^T grad_y with fly_spmm over the transposed structure and the per-synapse
gradient sum_b h[pre_e, b] grad_y[post_e, b] with fly_sddmm; the light cone's steps (`_ConeRecurrence`) fuse
those two backward products into one pass over A^T (fly_transposed_backward).  The tensors must live on a HIP
device; nothing here falls back to the CPU.
"""

from __future__ import annotations

import ctypes
import math
import weakref

import torch
from torch import nn

from . import _hip
from .connectome import Connectome


def _crow(sorted_rows: torch.Tensor, n: int) -> torch.Tensor:
    """CSR row pointer of a row-sorted edge list (brain.py:28-31)."""
    crow = torch.zeros(n + 1, dtype=torch.long, device=sorted_rows.device)
    crow[1:] = torch.bincount(sorted_rows, minlength=n).cumsum(0)
    return crow


def _transpose_order(rows: torch.Tensor, cols: torch.Tensor, n_rows: int) -> torch.Tensor:
    """Edge order of the transposed CSR: by column, then row, ties in edge order (brain.py:120, 190)."""
    return torch.argsort(cols * n_rows + rows, stable=True)


def _spmm(crow32, col32, val, n_rows: int, n_cols: int, x: torch.Tensor, out: torch.Tensor | None = None,
          val_ids32: torch.Tensor | None = None) -> torch.Tensor:
    """y (n_rows, B) = A x on the device (fly_spmm); x (n_cols, B) float32.  With `out`, y is added to it; with
    `val_ids32` the values are val[val_ids32[e]]."""
    x = x.contiguous()
    batch = x.shape[1]
    y = torch.empty(n_rows, batch, dtype=torch.float32, device=x.device) if out is None else out
    _hip.check(_hip.load().fly_spmm(crow32.data_ptr(), col32.data_ptr(), val.data_ptr(), _hip.ptr(val_ids32),
                                    val.numel(), n_rows, n_cols, x.data_ptr(), max(batch, 1), batch, y.data_ptr(),
                                    max(batch, 1), int(out is not None), _hip.stream(x.device)), "fly_spmm")
    return y


def _sweep_tables(holder, crow32, col32, n_rows: int, n_cols: int, attr: str = "_sweep"):
    """The banded-sweep tables of a product over one structure (fly_sweep_create, float32 operands), built on first
    use and kept on `holder` (as `attr`) with the row pointer they belong to; None when the structure does not sweep
    (too few or too short rows)."""
    cached = getattr(holder, attr, None)
    if cached is not None and cached[0] is crow32:
        return cached[1]
    tables = _hip.sweep_create(crow32, col32, n_rows, n_cols)
    setattr(holder, attr, (crow32, tables))
    return tables


def _spmm_swept(col32, val, tables, n_rows: int, x: torch.Tensor, records: torch.Tensor | None = None) -> torch.Tensor:
    """y (n_rows, B) = A x as a banded sweep (fly_spmm_swept) from {column, weight} records (`records`, or built from
    col32 and val); x (n_cols, B) float32, contiguous and 16-byte aligned, with B a multiple of 4."""
    batch = x.shape[1]
    y = torch.empty(n_rows, batch, dtype=torch.float32, device=x.device)
    if records is None:
        records = torch.stack((col32, val.contiguous().view(torch.int32)), dim=1)
    lib = _hip.load()
    ws = _hip.workspace(lib.fly_spmm_swept_workspace(tables.handle, batch), x.device)
    _hip.check(lib.fly_spmm_swept(tables.handle, records.data_ptr(), col32.numel(), x.data_ptr(), batch, batch,
                                  y.data_ptr(), batch, ws.data_ptr(), ws.numel(), _hip.stream(x.device)),
               "fly_spmm_swept")
    return y


def _spmv_work(crow32, col32, val, n_rows: int, n_cols: int, x: torch.Tensor, work,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """y (n_rows, 1) = A x for one column over a work list (fly_spmv_work): rows split into segments of at most
    256 non-zeros, longest first, so a transposed connectome's heavy rows spread over several waves.  With
    `out`, y is added to it."""
    x = x.contiguous()
    items, splits, n_slots = work
    y = torch.empty(n_rows, 1, dtype=torch.float32, device=x.device) if out is None else out
    partials = torch.empty(n_slots, dtype=torch.float32, device=x.device) if n_slots else None
    _hip.check(_hip.load().fly_spmv_work(crow32.data_ptr(), col32.data_ptr(), val.data_ptr(), val.numel(), n_rows,
                                         n_cols, x.data_ptr(), 1, y.data_ptr(), 1, int(out is not None),
                                         items.data_ptr(), items.shape[0], splits.data_ptr(), splits.shape[0],
                                         _hip.ptr(partials), n_slots, _hip.stream(x.device)), "fly_spmv_work")
    return y


def _sddmm(crow32, col32, n_rows: int, n_cols: int, g: torch.Tensor, x: torch.Tensor, nnz: int,
           out: torch.Tensor | None = None, ids32: torch.Tensor | None = None) -> torch.Tensor:
    """out[e] = sum_b g[row_e, b] x[col_e, b] on the device (fly_sddmm).  With `out` and `ids32` the values are
    added to out[ids32[e]] (a sub-matrix's gradient straight into the whole weight vector)."""
    g, x = g.contiguous(), x.contiguous()
    batch = x.shape[1]
    if out is None:
        out = torch.empty(nnz, dtype=torch.float32, device=x.device)
    if nnz:
        _hip.check(_hip.load().fly_sddmm(crow32.data_ptr(), col32.data_ptr(), n_rows, n_cols, g.data_ptr(),
                                         max(batch, 1), x.data_ptr(), max(batch, 1), batch, out.data_ptr(),
                                         out.numel(), _hip.ptr(ids32), int(ids32 is not None),
                                         _hip.stream(x.device)), "fly_sddmm")
    return out


class _TakeRows(torch.autograd.Function):
    """x[rows] for distinct rows, whose gradient is one index_add_ into a zero tensor instead of the sort
    that the general index backward needs when indices may repeat."""

    @staticmethod
    def forward(ctx, x, rows):
        ctx.save_for_backward(rows)
        ctx.shape = x.shape
        return x.index_select(0, rows)

    @staticmethod
    def backward(ctx, g):
        (rows,) = ctx.saved_tensors
        return g.new_zeros(ctx.shape).index_add_(0, rows, g), None


def _take_rows(x: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    return _TakeRows.apply(x, rows) if torch.is_grad_enabled() and x.requires_grad else x.index_select(0, rows)


def _take(src: torch.Tensor, ids32: torch.Tensor) -> torch.Tensor:
    """src[ids32] for a float32 vector on the device (fly_gather_values)."""
    src = src.contiguous()
    out = torch.empty(ids32.numel(), dtype=torch.float32, device=src.device)
    _hip.check(_hip.load().fly_gather_values(src.data_ptr(), src.numel(), ids32.data_ptr(), ids32.numel(),
                                             out.data_ptr(), _hip.stream(src.device)), "fly_gather_values")
    return out


def _gathered(op, w: torch.Tensor, transposed: bool, via: tuple | None = None) -> torch.Tensor:
    """op's values taken from the whole weight vector w, in CSR order or in the transposed structure's order,
    gathered once per weight tensor: the forward, its backward and the resting trajectory's products share
    them.  `via` = (src, ids32) names the same values as src[ids32]: a sub-matrix's transposed values read
    from w in W^T's order, where its ids rise, instead of from w at random."""
    slot = "_vals_t" if transposed else "_vals"
    cached = getattr(op, slot, None)
    if cached is not None and cached[0]() is w:
        return cached[1]
    if via is not None:
        vals = _take(*via)
        setattr(op, slot, (weakref.ref(w), vals))
        return vals
    if transposed:
        ids32 = op._transposed()[2]                  # the transpose's edge ids (W^T: its order in W)
    else:
        ids = op._edge_ids()
        ids32 = None if ids is None else ids[0]
    vals = w if ids32 is None else _take(w, ids32)
    setattr(op, slot, (weakref.ref(w), vals))
    return vals


def _records(op, w: torch.Tensor, transposed: bool, via: tuple | None = None) -> torch.Tensor:
    """op's {column, value bits} records (nnz, 2) int32 in CSR order or in the transposed structure's order, the
    swept products' operand, with the values taken from the whole weight vector w in one pass
    (fly_gather_records) and kept once per weight tensor, as _gathered keeps the values alone.  `via` = (src,
    ids32) as in _gathered."""
    slot = "_rec_t" if transposed else "_rec"
    cached = getattr(op, slot, None)
    if cached is not None and cached[0]() is w:
        return cached[1]
    if transposed:
        _, col32, t_ids32 = op._transposed()
        src, ids32 = via if via is not None else (w, t_ids32)
    else:
        col32 = op._structure()[1]
        ids = op._edge_ids()
        src, ids32 = w, (None if ids is None else ids[0])
    src = src.contiguous()
    rec = torch.empty(col32.numel(), 2, dtype=torch.int32, device=w.device)
    _hip.check(_hip.load().fly_gather_records(col32.data_ptr(), src.data_ptr(), src.numel(), _hip.ptr(ids32),
                                              col32.numel(), rec.data_ptr(), _hip.stream(w.device)),
               "fly_gather_records")
    setattr(op, slot, (weakref.ref(w), rec))
    return rec


def backward_work(t_crow: torch.Tensor, seg: int = 256):
    """The work list of fly_transposed_backward over the rows of A^T with row pointer t_crow: each row in
    segments of at most `seg` non-zeros (a multiple of 64), longest first, so the heavy-tailed rows of A^T
    (out-degrees) spread over several waves.  Returns (items (n, 4) int32 {row, first non-zero, count, slot},
    splits (m, 4) int32 {row, first slot, slot count, 0}, number of partial slots)."""
    if seg <= 0 or seg % 64:
        raise ValueError("segments are whole blocks of 64 non-zeros")
    dev = t_crow.device
    crow = t_crow.to(torch.int64)
    lens = crow[1:] - crow[:-1]
    nseg = torch.clamp((lens + seg - 1) // seg, min=1)
    rows = torch.repeat_interleave(torch.arange(lens.numel(), device=dev), nseg)
    start = torch.cumsum(nseg, 0) - nseg                 # each row's first item, in row order
    k = torch.arange(rows.numel(), device=dev) - start[rows]
    off = k * seg
    count = torch.clamp(torch.clamp(lens[rows] - off, max=seg), min=0)
    extra = k > 0
    slot = torch.where(extra, torch.cumsum(extra.to(torch.int64), 0) - 1, torch.full_like(k, -1))
    order = torch.argsort(count, descending=True, stable=True)
    items = torch.stack([rows, off, count, slot], 1)[order].to(torch.int32).contiguous()
    split_rows = torch.nonzero(nseg > 1).squeeze(1)
    splits = torch.stack([split_rows, slot[start[split_rows] + 1], nseg[split_rows] - 1,
                          torch.zeros_like(split_rows)], 1).to(torch.int32).contiguous()
    return items, splits, int(extra.sum())


def _product(op, w: torch.Tensor, x: torch.Tensor, transposed: bool = False, out: torch.Tensor | None = None):
    """A x (or A^T x) with A's values from w, gathered once per weight tensor into the structure's order.
    Every product of a training step over one structure shares the gathered copy, so each reads its values as
    a stream; reading w through value ids instead would cost a random line per non-zero in the transposed
    order, on every call."""
    if transposed:
        crow32, col32, _ = op._transposed()
        _, _, n_cols, n_rows = op._structure()
        if x.shape[1] == 1 and (out is None or out.is_contiguous()):
            return _spmv_work(crow32, col32, _gathered(op, w, True), n_rows, n_cols, x, op._backward_work(), out=out)
    else:
        crow32, col32, n_rows, n_cols = op._structure()
        batch = x.shape[1]
        if out is None and x.dtype == torch.float32 and batch >= 4 and batch % 4 == 0:
            tables = _sweep_tables(op, crow32, col32, n_rows, n_cols)
            x = x.contiguous()
            if tables is not None and x.data_ptr() % 16 == 0:
                return _spmm_swept(col32, None, tables, n_rows, x, records=_records(op, w, False))
    return _spmm(crow32, col32, _gathered(op, w, transposed), n_rows, n_cols, x, out=out)


class _ConeRecurrence(torch.autograd.Function):
    """Steps 1..T of the light cone under autograd, float32 (brain.py:313-327): per step the sub-matrix
    product on the device (its values read from the whole edge-weight vector w at the sub-matrix's edge ids),
    then one fused kernel for the constant drive, the input, the clamp and the lerp (fly_train_step_forward).
    The backward runs per step one fused kernel for the gradients of those (fly_train_step_backward), then
    one pass over A_t^T (fly_transposed_backward, from the sub-matrix's longest-first work list) that adds the
    state gradient A_t^T grad_y to the carried rows' share and writes the per-synapse gradient straight into
    dL/dw (chunk-major above 64 columns, so the gathers share one chunk of grad_y in the caches); batches that
    are not a multiple of 4 take fly_spmm and fly_sddmm instead.  The transposed passes work in the transposed
    order of the whole weight vector (rnn's W^T), where every step's ids rise along the pass: they read A_t^T's
    values from w in that order and add into dL/dw kept in that order, which one gather at the end puts back
    in the weight vector's order.  Inputs after u_in and w, per step t: k_t, the previous resting state
    c_{t-1}[R_t] and alpha[R_t] (each (|R_t|, 1)).  Returns h_T, (|R_T|, B)."""

    @staticmethod
    def forward(ctx, cone, h_max, rnn, u_in, w, *flat):
        lib = _hip.load()
        dev = u_in.device
        st = _hip.stream(dev)
        u_in = u_in.contiguous()
        batch = u_in.shape[1]
        ld = max(batch, 1)
        hs, ys = [], []
        h = None
        for t in range(1, cone.steps + 1):
            k, pdef, alpha = flat[3 * (t - 1):3 * t]
            rows, op = cone.row_counts[t], cone.ops[t]
            prev32, usrc32 = cone.step_tables32(t)
            if op is not None:
                y = _product(op, w, h)
            else:
                y = torch.empty(rows, batch, dtype=torch.float32, device=dev)
            hn = torch.empty(rows, batch, dtype=torch.float32, device=dev)
            # operands bound to names: a temporary freed inside the argument list could be reused (and
            # overwritten on the stream) by the next one before the kernel reads it
            k, pdef, alpha = k.contiguous(), pdef.contiguous(), alpha.contiguous()
            _hip.check(lib.fly_train_step_forward(
                rows, batch, y.data_ptr(), ld, int(op is not None), k.data_ptr(),
                pdef.data_ptr(), alpha.data_ptr(),
                _hip.ptr(prev32 if h is not None and h.shape[0] else None), usrc32.data_ptr(), u_in.data_ptr(), ld,
                _hip.ptr(h), ld, float(h_max), hn.data_ptr(), ld, st), "fly_train_step_forward")
            hs.append(hn)
            ys.append(y)
            h = hn
        ctx.cone, ctx.h_max, ctx.rnn = cone, float(h_max), rnn
        ctx.save_for_backward(u_in, w, *hs, *ys, *flat)
        return h

    @staticmethod
    def backward(ctx, grad_h):
        cone = ctx.cone
        T = cone.steps
        saved = ctx.saved_tensors
        u_in, w = saved[0], saved[1]
        hs, ys, flat = saved[2:2 + T], saved[2 + T:2 + 2 * T], saved[2 + 2 * T:]
        lib = _hip.load()
        dev = u_in.device
        st = _hip.stream(dev)
        batch = u_in.shape[1]
        ld = max(batch, 1)
        g = grad_h.contiguous()
        gu = torch.zeros_like(u_in)
        gw = torch.zeros_like(w)
        gw_t = w_pos32 = None                         # dL/dw in W^T's order, for the transposed passes
        grads = [None] * len(flat)
        for t in range(T, 0, -1):
            k, pdef, alpha = flat[3 * (t - 1):3 * t]
            rows, op = cone.row_counts[t], cone.ops[t]
            prev32, usrc32 = cone.step_tables32(t)
            h_prev = hs[t - 2] if t > 1 else None
            gy = torch.empty(rows, batch, dtype=torch.float32, device=dev)
            gk = torch.empty(rows, dtype=torch.float32, device=dev)
            ga = torch.empty_like(gk)
            gpdef = torch.empty_like(gk)
            gh_prev = torch.zeros(cone.row_counts[t - 1], batch, dtype=torch.float32, device=dev) if t > 1 else None
            pdef, alpha = pdef.contiguous(), alpha.contiguous()
            _hip.check(lib.fly_train_step_backward(
                rows, batch, g.data_ptr(), ld, ys[t - 1].data_ptr(), ld, pdef.data_ptr(),
                alpha.data_ptr(), _hip.ptr(prev32 if h_prev is not None and h_prev.shape[0] else None),
                usrc32.data_ptr(), _hip.ptr(h_prev), ld, ctx.h_max, gy.data_ptr(), ld, gk.data_ptr(), ga.data_ptr(),
                gpdef.data_ptr(), gu.data_ptr(), ld, _hip.ptr(gh_prev), ld, st), "fly_train_step_backward")
            grads[3 * (t - 1)] = gk.view_as(k)
            grads[3 * (t - 1) + 1] = gpdef.view_as(pdef)
            grads[3 * (t - 1) + 2] = ga.view_as(alpha)
            if op is not None:
                crow32, col32, n_rows, n_cols = op._structure()
                if batch % 4 == 0:          # one pass over A^T: the state gradient and dL/dw together
                    t_crow32, t_col32, _ = op._transposed()
                    if w_pos32 is None:
                        w_pos32 = ctx.rnn._transposed_positions()
                        w_t = _gathered(ctx.rnn, w, True)     # shared with the resting trajectory's backward
                    wt_ids32 = op._whole_transposed_ids(w_pos32)
                    if gw_t is None:
                        gw_t = torch.zeros_like(w)
                    # A^T's structure as a banded sweep of gy's rows where it suits the sweep (tables built once per
                    # sub-matrix), else the chunk-major pass over the longest-first work list
                    tables_t = _sweep_tables(op, t_crow32, t_col32, n_cols, n_rows, attr="_sweep_t")
                    if tables_t is not None:
                        records = _records(op, w, True, via=(w_t, wt_ids32))
                        ws = _hip.workspace(lib.fly_transposed_backward_swept_workspace(tables_t.handle, batch), dev)
                        _hip.check(lib.fly_transposed_backward_swept(
                            tables_t.handle, records.data_ptr(), t_col32.numel(), wt_ids32.data_ptr(), gy.data_ptr(),
                            ld, h_prev.data_ptr(), ld, batch, gh_prev.data_ptr(), ld, 1, gw_t.data_ptr(), gw_t.numel(),
                            ws.data_ptr(), ws.numel(), st), "fly_transposed_backward_swept")
                    else:
                        vals_t = _gathered(op, w, True, via=(w_t, wt_ids32))
                        items, splits, n_slots = op._backward_work()
                        partials = torch.empty(n_slots, ld, dtype=torch.float32, device=dev) if n_slots else None
                        # more than one 64-column chunk: chunk-major, each chunk's dot products kept in a workspace
                        chunks = (batch + 63) // 64
                        dots = torch.empty(chunks * wt_ids32.numel(), dtype=torch.float32, device=dev) \
                            if chunks > 1 else None
                        _hip.check(lib.fly_transposed_backward(
                            t_crow32.data_ptr(), t_col32.data_ptr(), vals_t.data_ptr(), wt_ids32.data_ptr(),
                            wt_ids32.numel(), n_cols, n_rows, gy.data_ptr(), ld, h_prev.data_ptr(), ld, batch,
                            gh_prev.data_ptr(), ld, 1, gw_t.data_ptr(), gw_t.numel(), items.data_ptr(),
                            items.shape[0], splits.data_ptr(), splits.shape[0], _hip.ptr(partials), n_slots,
                            _hip.ptr(dots), dots.numel() if dots is not None else 0, st), "fly_transposed_backward")
                else:
                    _product(op, w, gy, transposed=True, out=gh_prev)
                    ids32, ids = op._edge_ids()
                    _sddmm(crow32, col32, n_rows, n_cols, gy, h_prev, len(ids), out=gw, ids32=ids32)
            g = gh_prev
        if gw_t is not None:                          # back to the weight vector's order: gw[i] += gw_t[pos[i]]
            gw += _take(gw_t, w_pos32)
        return (None, None, None, gu, gw, *grads)


class _RestingTrajectory(torch.autograd.Function):
    """The resting trajectory and the light cone's constant drives (brain.py:238-252) as one autograd function
    over device kernels, one column.  Per step one pass over W (fly_rest_forward) gives W c_{t-1} + b for
    c_t = lerp(c_{t-1}, clamp(W c_{t-1} + b, 0, H), alpha) and, summed over the edges from outside R_{t-1}, the
    drive k_t = (W c_{t-1} + b - A_t c_{t-1}[R_{t-1}])[R_t] of the step's rows.  The backward runs per step one
    elementwise kernel (fly_rest_backward) and one pass over W and W^T (fly_rest_products_backward) into a
    single dL/dw.  Inputs w (E), bias (n), alpha = sigmoid(alpha_logit) (n, 1); returns k_1..k_T, then
    p_1..p_T = c_{t-1}[R_t] (each (|R_t|, 1)), then c_T[out_idx] (n_out, 1)."""

    @staticmethod
    def forward(ctx, rnn, cone, out_idx, w, bias, alpha):
        ctx.set_materialize_grads(False)
        lib = _hip.load()
        dev = w.device
        st = _hip.stream(dev)
        n, T = rnn.n, cone.steps
        member, _ = cone.rest_tables(n)
        w, bias, alpha = w.contiguous(), bias.contiguous(), alpha.contiguous()
        x2 = c_prev = None
        ks, ps, saved = [], [], []
        for t in range(1, T + 1):
            full = torch.empty(n, device=dev)
            outside = torch.empty(n, device=dev)
            c_next = torch.empty(n, device=dev)
            x2_next = torch.empty(n, 2, device=dev)
            _hip.check(lib.fly_rest_forward(rnn.crow32.data_ptr(), rnn.pre32.data_ptr(), w.data_ptr(), n,
                                            rnn.n_edges, _hip.ptr(x2), bias.data_ptr(), alpha.data_ptr(),
                                            _hip.ptr(c_prev), rnn._h_bound, member[t].data_ptr(),
                                            full.data_ptr(), outside.data_ptr(), c_next.data_ptr(),
                                            x2_next.data_ptr(), st), "fly_rest_forward")
            rows = cone.rows[t]
            ks.append(outside.index_select(0, rows).unsqueeze(1))
            ps.append((c_prev.index_select(0, rows) if c_prev is not None
                       else torch.zeros(rows.numel(), device=dev)).unsqueeze(1))
            saved.append((full, c_prev, x2))
            x2, c_prev = x2_next, c_next
        c_out = c_prev.index_select(0, out_idx).unsqueeze(1)
        ctx.rnn, ctx.cone, ctx.out_idx, ctx.steps_saved = rnn, cone, out_idx, saved
        ctx.save_for_backward(w, alpha)
        return (*ks, *ps, c_out)

    @staticmethod
    def backward(ctx, *grads):
        rnn, cone, out_idx = ctx.rnn, ctx.cone, ctx.out_idx
        w, alpha = ctx.saved_tensors
        lib = _hip.load()
        dev = w.device
        st = _hip.stream(dev)
        n, T = rnn.n, cone.steps
        member, pos = cone.rest_tables(n)
        flat = lambda g: None if g is None else g.reshape(-1).contiguous()
        g_ks, g_ps, g_out = [flat(g) for g in grads[:T]], [flat(g) for g in grads[T:2 * T]], flat(grads[2 * T])
        gw = torch.zeros_like(w)
        gbias = torch.zeros(n, device=dev)
        galpha = torch.zeros(n, device=dev)
        gc = None if g_out is None else torch.zeros(n, device=dev).index_copy_(0, out_idx, g_out)
        t_crow32, t_col32, _ = rnn._transposed()
        vals_t = _gathered(rnn, w, True)
        items, splits, n_slots = rnn._backward_work()
        partials = torch.empty(max(n_slots, 1), device=dev)
        for t in range(T, 0, -1):
            full, c_prev, x2 = ctx.steps_saved[t - 1]
            g2 = torch.empty(n, 2, device=dev)
            gc_prev = torch.empty(n, device=dev)
            gk, gp = g_ks[t - 1], g_ps[t - 1]
            _hip.check(lib.fly_rest_backward(_hip.ptr(gc), pos[t].data_ptr(), _hip.ptr(gk), _hip.ptr(gp),
                                             full.data_ptr(), _hip.ptr(c_prev), alpha.data_ptr(), rnn._h_bound,
                                             n, g2.data_ptr(), gc_prev.data_ptr(), gbias.data_ptr(),
                                             galpha.data_ptr(), st), "fly_rest_backward")
            if x2 is not None:                 # t > 1: the products over W (c_0 = 0 has none)
                _hip.check(lib.fly_rest_products_backward(
                    rnn.crow32.data_ptr(), rnn.pre32.data_ptr(), n, rnn.n_edges, g2.data_ptr(), x2.data_ptr(),
                    gw.data_ptr(), t_crow32.data_ptr(), t_col32.data_ptr(), vals_t.data_ptr(),
                    member[t - 1].data_ptr(), items.data_ptr(), items.shape[0], splits.data_ptr(), splits.shape[0],
                    partials.data_ptr(), n_slots, gc_prev.data_ptr(), st), "fly_rest_products_backward")
            gc = gc_prev
        return None, None, None, gw, gbias, galpha.view_as(alpha)


class _SparseRecurrent(torch.autograd.Function):
    """y = A h for A in CSR, the state (rows, batch) batch-fastest (brain.py:66-99), with A's values taken
    from the whole edge-weight vector w (a _SubMatrix reads w at its edge ids; the whole W is w itself).
    Forward and the state gradient are device SpMMs over A's structure and its transposed structure; the
    per-synapse gradient dL/dw_e = sum_b h[col_e, b] grad_y[row_e, b] is a device SDDMM written straight at
    the edge ids, so no index backward (sort and scatter) over the edges is needed.  float32 only."""

    @staticmethod
    def forward(ctx, h, w, op):
        if h.dtype != torch.float32 or w.dtype != torch.float32:
            raise RuntimeError("training runs in float32: the state and the weights must be float32")
        h = h.contiguous()
        ctx.save_for_backward(h, w)
        ctx.op = op
        return _product(op, w, h)

    @staticmethod
    def backward(ctx, grad_y):
        h, w = ctx.saved_tensors
        op = ctx.op
        grad_h = grad_w = None
        crow32, col32, n_rows, n_cols = op._structure()
        ids = op._edge_ids()
        if ctx.needs_input_grad[0]:
            grad_h = _product(op, w, grad_y.contiguous(), transposed=True)
        if ctx.needs_input_grad[1]:
            if ids is None:
                grad_w = _sddmm(crow32, col32, n_rows, n_cols, grad_y, h, w.numel())
            else:
                grad_w = torch.zeros_like(w)
                _sddmm(crow32, col32, n_rows, n_cols, grad_y, h, len(ids[1]), out=grad_w, ids32=ids[0])
        return grad_h, grad_w, None


def _spmm64(op, w: torch.Tensor, x: torch.Tensor, transposed: bool = False) -> torch.Tensor:
    """A x (or A^T x) in float64 (fly_spmm_f64), A's values read from the whole weight vector w at A's edge ids."""
    if transposed:
        crow32, col32, ids32 = op._transposed()          # A^T's structure, its non-zeros' edge ids
        _, _, n_rows, n_cols = op._structure()
        n_rows, n_cols = n_cols, n_rows
    else:
        crow32, col32, n_rows, n_cols = op._structure()
        ids = op._edge_ids()
        ids32 = None if ids is None else ids[0]
    x = x.contiguous()
    batch = x.shape[1]
    y = torch.empty(n_rows, batch, dtype=torch.float64, device=x.device)
    _hip.check(_hip.load().fly_spmm_f64(crow32.data_ptr(), col32.data_ptr(), col32.numel(), w.data_ptr(),
                                        _hip.ptr(ids32), w.numel(), n_rows, n_cols, x.data_ptr(), max(batch, 1),
                                        batch, y.data_ptr(), max(batch, 1), 0, _hip.stream(x.device)), "fly_spmm_f64")
    return y


class _SparseRecurrent64(torch.autograd.Function):
    """y = A h in float64 for networks converted to float64 (brain.py:66-99 in float64): the product over A's
    structure, the state gradient over its transposed structure (fly_spmm_f64) and dL/dw at A's edge ids
    (fly_sddmm_f64), every sum in CSR order."""

    @staticmethod
    def forward(ctx, h, w, op):
        h = h.contiguous()
        ctx.save_for_backward(h, w)
        ctx.op = op
        return _spmm64(op, w, h)

    @staticmethod
    def backward(ctx, grad_y):
        h, w = ctx.saved_tensors
        op = ctx.op
        g = grad_y.contiguous()
        grad_h = grad_w = None
        if ctx.needs_input_grad[0]:
            grad_h = _spmm64(op, w, g, transposed=True)
        if ctx.needs_input_grad[1]:
            crow32, col32, n_rows, n_cols = op._structure()
            ids = op._edge_ids()
            batch = h.shape[1]
            grad_w = torch.zeros_like(w)
            _hip.check(_hip.load().fly_sddmm_f64(crow32.data_ptr(), col32.data_ptr(), col32.numel(), n_rows, n_cols,
                                                 g.data_ptr(), max(batch, 1), h.data_ptr(), max(batch, 1), batch,
                                                 grad_w.data_ptr(), grad_w.numel(),
                                                 _hip.ptr(None if ids is None else ids[0]), 0,
                                                 _hip.stream(h.device)), "fly_sddmm_f64")
        return grad_h, grad_w, None


class _SubMatrix:
    """Rows x columns of W as its own CSR (brain.py:102-123), read back from the device cone on first use:
    `edges` (global edge ids in W's order), `post` / `pre` (local row / column), `crow`, `shape`."""

    def __init__(self, cone: "LightCone", t: int, n_rows: int, n_cols: int, nnz: int):
        self._cone, self._t, self._nnz = cone, t, nnz
        self._tr = self._tw = None
        self.shape = (n_rows, n_cols)
        self._data = None

    def _load(self):
        if self._data is None:
            dev = self._cone.device
            crow = torch.empty(self.shape[0] + 1, dtype=torch.int32, device=dev)
            col = torch.empty(self._nnz, dtype=torch.int32, device=dev)
            edge = torch.empty(self._nnz, dtype=torch.int32, device=dev)
            self._cone._step_export(self._t, crow=crow, col=col, edge=edge)
            crow64 = crow.long()
            rows = torch.repeat_interleave(torch.arange(self.shape[0], device=dev), crow64[1:] - crow64[:-1])
            self._data = (edge.long(), rows, col.long(), crow64, crow, col, edge)
        return self._data

    def _edge_ids(self):
        """(int32, int64) ids of the sub-matrix's edges in the whole weight vector."""
        d = self._load()
        return d[6], d[0]

    def _structure(self):
        d = self._load()
        return d[4], d[5], self.shape[0], self.shape[1]

    def _transposed(self):
        """CSR of A^T (brain.py:120-121): order, int32 row pointer and columns, built on first use."""
        if getattr(self, "_tr", None) is None:
            post, pre = self.post, self.pre
            order = _transpose_order(post, pre, self.shape[0])
            t_crow = _crow(pre[order], self.shape[1])
            t_col = post[order]
            self._tr = (order, t_crow, t_col, t_crow.to(torch.int32), t_col.to(torch.int32),
                        self.edges[order].to(torch.int32))
        return self._tr[3], self._tr[4], self._tr[5]

    def _backward_work(self):
        """The transposed backward's work list (backward_work), built on first use."""
        if getattr(self, "_tw", None) is None:
            self._transposed()
            self._tw = backward_work(self._tr[3])
        return self._tw

    def _whole_transposed_ids(self, w_pos32: torch.Tensor) -> torch.Tensor:
        """int32: each non-zero of A^T (in its order) as a position in the transposed order of the whole
        weight vector, from w_pos32 = each edge's position in that order.  Rows and columns keep their
        relative order in the sub-matrix, so A^T's order is a subsequence of W^T's and these ids rise along
        the transposed backward.  Cached per w_pos32."""
        cached = getattr(self, "_wt_ids", None)
        if cached is None or cached[0]() is not w_pos32:
            ids = w_pos32[self._transposed()[2].long()]
            self._wt_ids = cached = (weakref.ref(w_pos32), ids)
        return cached[1]

    @property
    def t_order(self) -> torch.Tensor:
        self._transposed()
        return self._tr[0]

    @property
    def t_crow(self) -> torch.Tensor:
        self._transposed()
        return self._tr[1]

    @property
    def t_col(self) -> torch.Tensor:
        self._transposed()
        return self._tr[2]

    def csr_t(self, w: torch.Tensor) -> torch.Tensor:
        return torch.sparse_csr_tensor(self.t_crow, self.t_col, w[self.t_order], self.shape[::-1],
                                       check_invariants=False)

    @property
    def edges(self) -> torch.Tensor:
        return self._load()[0]

    @property
    def post(self) -> torch.Tensor:
        return self._load()[1]

    @property
    def pre(self) -> torch.Tensor:
        return self._load()[2]

    @property
    def crow(self) -> torch.Tensor:
        return self._load()[3]

    def csr(self, w: torch.Tensor) -> torch.Tensor:
        return torch.sparse_csr_tensor(self.crow, self.pre, w, self.shape, check_invariants=False)


class LightCone:
    """Which rows of the state each step computes (brain.py:126-173), built on the device.

    V_1 = inputs and V_t = V_{t-1} plus the postsynaptic partners of V_{t-1} (within t-1 synapses of an
    input); D_T = outputs and D_t = D_{t+1} plus the presynaptic partners of D_{t+1} (within T-t synapses of
    an output); R_t = sorted(V_t & D_t), R_0 empty.  Attributes match the reference: steps, rows, ops,
    keep_next, keep_prev, carried, prev_row, u_pos, u_src, out_pos, out_src, out_idx, edge_visits (int64
    tensors on the device; `carried` is a (|R_t|, 1) bool column).  The per-step index lists are read back
    from the device cone the first time they are used.
    """

    def __init__(self, rnn: "ConnectomeRNN", in_idx: torch.Tensor, out_idx: torch.Tensor, steps: int,
                 prune: bool = True):
        _hip.require_device(rnn.pre, "LightCone")
        lib = _hip.load()
        self.device = rnn.pre.device
        self.steps = int(steps)
        self.pruned = bool(prune)
        self.out_idx = out_idx
        in32 = in_idx.to(device=self.device, dtype=torch.int32).contiguous()
        out32 = out_idx.to(device=self.device, dtype=torch.int32).contiguous()
        handle = ctypes.c_void_p()
        _hip.check(lib.fly_cone_create(rnn.n, rnn.n_edges, rnn.crow32.data_ptr(), rnn.pre32.data_ptr(),
                                       in32.data_ptr(), in32.numel(), out32.data_ptr(), out32.numel(), self.steps,
                                       0 if prune else _hip.CONE_UNPRUNED, _hip.stream(self.device),
                                       ctypes.byref(handle)), "fly_cone_create")
        self._handle = handle
        T = self.steps
        rows = (ctypes.c_int64 * (T + 1))()
        nnz = (ctypes.c_int64 * (T + 1))()
        has_op = (ctypes.c_int32 * (T + 1))()
        _hip.check(lib.fly_cone_sizes(handle, rows, nnz, has_op), "fly_cone_sizes")
        self.row_counts = [int(r) for r in rows]
        self.nnz = [int(x) for x in nnz]
        self.has_op = [bool(x) for x in has_op]
        self.edge_visits = sum(self.nnz)
        self.n_out = int(out32.numel())
        self._rows = None
        self._steps_idx = None
        self._outs = None
        self._rest = None
        self.ops = [None] + [_SubMatrix(self, t, self.row_counts[t], self.row_counts[t - 1], self.nnz[t])
                             if self.has_op[t] else None for t in range(1, T + 1)]

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._handle

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            try:
                _hip.load().fly_cone_destroy(h)
            except Exception:
                pass
            self._handle = None

    def _step_export(self, t: int, crow=None, col=None, edge=None, prev=None, usrc=None) -> None:
        lib = _hip.load()
        _hip.check(lib.fly_cone_step(self._handle, t, _hip.ptr(crow), _hip.ptr(col), _hip.ptr(edge), _hip.ptr(prev),
                                     _hip.ptr(usrc), _hip.stream(self.device)), "fly_cone_step")

    @property
    def rows(self) -> list:
        if self._rows is None:
            lib = _hip.load()
            out = []
            for t in range(self.steps + 1):
                r = torch.empty(self.row_counts[t], dtype=torch.int32, device=self.device)
                _hip.check(lib.fly_cone_rows(self._handle, t, r.data_ptr(), _hip.stream(self.device)), "fly_cone_rows")
                out.append(r.long())
            self._rows = out
        return self._rows

    def _per_step(self):
        if self._steps_idx is None:
            keep_next, keep_prev, carried, prev_row, u_pos, u_src = ([None] for _ in range(6))
            tables32 = [None]
            for t in range(1, self.steps + 1):
                nr = self.row_counts[t]
                prev = torch.empty(nr, dtype=torch.int32, device=self.device)
                usrc = torch.empty(nr, dtype=torch.int32, device=self.device)
                self._step_export(t, prev=prev, usrc=usrc)
                tables32.append((prev, usrc))
                prev, usrc = prev.long(), usrc.long()
                is_carried = prev >= 0
                keep_next.append(torch.nonzero(is_carried).squeeze(1))
                keep_prev.append(prev[is_carried])
                carried.append(is_carried.unsqueeze(1))
                prev_row.append(prev.clamp_min(0))
                fed = usrc >= 0
                u_pos.append(torch.nonzero(fed).squeeze(1))
                u_src.append(usrc[fed])
            self._steps_idx = (keep_next, keep_prev, carried, prev_row, u_pos, u_src, tables32)
        return self._steps_idx

    def step_tables32(self, t: int):
        """(prev, usrc) of step t as int32 device tensors: the row of R_{t-1} each row of R_t carries (-1: none)
        and the row of the input it is fed from (-1: none)."""
        return self._per_step()[6][t]

    keep_next = property(lambda self: self._per_step()[0])
    keep_prev = property(lambda self: self._per_step()[1])
    carried = property(lambda self: self._per_step()[2])
    prev_row = property(lambda self: self._per_step()[3])
    u_pos = property(lambda self: self._per_step()[4])
    u_src = property(lambda self: self._per_step()[5])

    def _outputs(self):
        if self._outs is None:
            src = torch.empty(self.n_out, dtype=torch.int32, device=self.device)
            if self.n_out:
                _hip.check(_hip.load().fly_cone_outputs(self._handle, src.data_ptr(), _hip.stream(self.device)),
                           "fly_cone_outputs")
            src = src.long()
            hit = src >= 0
            self._outs = (torch.nonzero(hit).squeeze(1), src[hit])
        return self._outs

    out_pos = property(lambda self: self._outputs()[0])
    out_src = property(lambda self: self._outputs()[1])

    def rest_tables(self, n: int):
        """Per step t = 0..T, R_t as a uint8 mask over the n neurons and each neuron's place in R_t (int32, -1
        outside): the resting trajectory's kernels read them (built on first use)."""
        if self._rest is None:
            member, pos = [], []
            for t in range(self.steps + 1):
                r = self.rows[t]
                m = torch.zeros(n, dtype=torch.uint8, device=self.device)
                p = torch.full((n,), -1, dtype=torch.int32, device=self.device)
                if r.numel():
                    m[r] = 1
                    p[r] = torch.arange(r.numel(), dtype=torch.int32, device=self.device)
                member.append(m)
                pos.append(p)
            self._rest = (member, pos)
        return self._rest


class _Plan:
    """Owner of a device weight-set plan (fly_plan)."""

    def __init__(self, handle: ctypes.c_void_p, key):
        self.handle, self.key = handle, key

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                _hip.load().fly_plan_destroy(h)
            except Exception:
                pass
            self.handle = None


class ConnectomeRNN(nn.Module):
    def __init__(self, conn: Connectome, alpha_init: float = 0.5, bias_init: float = 0.0,
                 global_scale: float = 1.0, h_max: float | None = 10.0):
        """global_scale multiplies the normalised connectome weights; activity is clamped to [0, h_max], or only
        below at 0 when h_max is None (brain.py:176-199, 221).  The wiring is rebuilt from the connectome, never
        stored in checkpoints."""
        super().__init__()
        self.n = conn.n_neurons
        self.n_edges = conn.n_edges
        self.h_max = None if h_max is None else float(h_max)
        # the upper bound the kernels clamp to: h_max, or +inf (no upper clamp) for None
        self._h_bound = math.inf if h_max is None else float(h_max)
        self.register_buffer("pre", conn.pre, persistent=False)      # (post, pre) order = CSR order of W
        self.register_buffer("post", conn.post, persistent=False)
        self.register_buffer("sign", conn.sign, persistent=False)
        self.register_buffer("w0", conn.weight * global_scale, persistent=False)
        self.register_buffer("crow", _crow(conn.post, self.n), persistent=False)
        # int32 copies of the CSR structure for the device library
        self.register_buffer("crow32", self.crow.to(torch.int32), persistent=False)
        self.register_buffer("pre32", conn.pre.to(torch.int32), persistent=False)
        # CSR of W^T, for the state gradient of training (brain.py:190-193)
        t_order = _transpose_order(conn.post, conn.pre, self.n)
        self.register_buffer("t_order", t_order, persistent=False)
        self.register_buffer("t_crow", _crow(conn.pre[t_order], self.n), persistent=False)
        self.register_buffer("t_col", conn.post[t_order], persistent=False)
        self.register_buffer("t_crow32", self.t_crow.to(torch.int32), persistent=False)
        self.register_buffer("t_col32", self.t_col.to(torch.int32), persistent=False)
        self.log_gain = nn.Parameter(torch.zeros(conn.n_edges))
        self.bias = nn.Parameter(torch.full((self.n,), float(bias_init)))
        a = torch.full((self.n,), float(alpha_init))
        self.alpha_logit = nn.Parameter(torch.log(a / (1 - a)))
        self._cone = None
        self._plans: dict = {}

    # ---- weights -----------------------------------------------------------------------------------
    def _param_key(self):
        return tuple((p._version, p.data_ptr()) for p in (self.log_gain, self.bias, self.alpha_logit))

    def _is_f64(self) -> bool:
        """A network converted to float64 (the reference's .double() test modules): it runs through the float64
        products, in float64, under autograd or not."""
        return self.log_gain.dtype == torch.float64

    def _check_params_f64(self, what: str) -> None:
        for name in ("log_gain", "bias", "alpha_logit", "sign", "w0"):
            t = getattr(self, name)
            _hip.require_device(t, what)
            if t.dtype != torch.float64:
                raise RuntimeError(f"{what}: a float64 network needs every parameter in float64; {name} is {t.dtype}")

    def _forward64(self, u: torch.Tensor, steps: int) -> torch.Tensor:
        """The literal recurrence of a float64 network (brain.py:211-229 in float64).  Under autograd u stays as it
        is; without, u becomes u + bias in place, as the reference's inference path leaves it."""
        self._check_params_f64("ConnectomeRNN.forward")
        if u.dtype != torch.float64 or u.dim() != 2 or u.shape[0] != self.n:
            raise RuntimeError(f"ConnectomeRNN.forward: a float64 network takes float64 u ({self.n}, B), got "
                               f"{u.dtype} {tuple(u.shape)}")
        alpha = torch.sigmoid(self.alpha_logit).unsqueeze(1)
        w = self.edge_weights()
        drive = self.bias.unsqueeze(1) + u if torch.is_grad_enabled() else u.add_(self.bias.unsqueeze(1))
        h = torch.zeros_like(drive)
        for _ in range(steps):
            x = (_SparseRecurrent64.apply(h, w, self) + drive).clamp(0, self.h_max)
            h = torch.lerp(h, x, alpha)
        return h

    def _forward_io64(self, u_in: torch.Tensor, cone: "LightCone", out_idx: torch.Tensor, steps: int) -> torch.Tensor:
        """forward_io of a float64 network (brain.py:238-252 and 289-329 in float64), under autograd or not: the
        resting trajectory c_t and the constant drives k_t of the light cone's rows, then per step the sub-matrix
        product plus k_t and the input, clamped, from the resting state or the carried row."""
        self._check_params_f64("ConnectomeRNN.forward_io")
        if u_in.dtype != torch.float64:
            raise RuntimeError(f"forward_io: a float64 network takes float64 u_in, got {u_in.dtype}")
        batch = u_in.shape[1]
        w = self.edge_weights()
        alpha = torch.sigmoid(self.alpha_logit).unsqueeze(1)
        bias = self.bias.unsqueeze(1)
        c = torch.zeros(self.n, 1, dtype=torch.float64, device=u_in.device)
        cs, ks = [c], [None]
        for t in range(1, steps + 1):
            full = (_SparseRecurrent64.apply(c, w, self) if t > 1 else torch.zeros_like(c)) + bias
            k = full.index_select(0, cone.rows[t])
            op = cone.ops[t]
            if op is not None:     # the drive from outside R_{t-1}: the full sum less the sub-matrix's share
                k = k - _SparseRecurrent64.apply(c.index_select(0, cone.rows[t - 1]), w, op)
            ks.append(k)
            c = torch.lerp(c, full.clamp(0, self.h_max), alpha)
            cs.append(c)
        h = None
        for t in range(1, steps + 1):
            rows, op = cone.rows[t], cone.ops[t]
            x = ks[t].expand(-1, batch) if op is None else _SparseRecurrent64.apply(h, w, op) + ks[t]
            x = x.index_add(0, cone.u_pos[t], u_in.index_select(0, cone.u_src[t])).clamp(0, self.h_max)
            p = cs[t - 1].index_select(0, rows).expand(-1, batch)
            if cone.keep_next[t].numel():
                p = p.index_copy(0, cone.keep_next[t], h.index_select(0, cone.keep_prev[t]))
            h = torch.lerp(p, x, alpha.index_select(0, rows))
        out = cs[steps].index_select(0, out_idx.to(u_in.device)).expand(-1, batch)
        return out.index_copy(0, cone.out_pos, h.index_select(0, cone.out_src))

    def _check_params(self, what: str) -> None:
        for name in ("log_gain", "bias", "alpha_logit", "sign", "w0"):
            t = getattr(self, name)
            _hip.require_device(t, what)
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise RuntimeError(f"{what}: {name} must be a contiguous float32 tensor, got {t.dtype}")

    def edge_weights(self) -> torch.Tensor:
        """sign * w0 * exp(log_gain) per edge, in CSR order (brain.py:201-202).  Under autograd, the
        differentiable expression; otherwise one device kernel."""
        if (torch.is_grad_enabled() and self.log_gain.requires_grad) or self._is_f64():
            return self.sign * self.w0 * torch.exp(self.log_gain)
        self._check_params("edge_weights")
        w = torch.empty_like(self.w0)
        dev = self.w0.device
        _hip.check(_hip.load().fly_edge_weights(self.sign.data_ptr(), self.w0.data_ptr(), self.log_gain.data_ptr(),
                                                self.n_edges, w.data_ptr(), _hip.stream(dev)), "fly_edge_weights")
        return w

    def csr(self, w: torch.Tensor) -> torch.Tensor:
        return torch.sparse_csr_tensor(self.crow, self.pre, w, (self.n, self.n), check_invariants=False)

    def csr_t(self, w: torch.Tensor) -> torch.Tensor:
        return torch.sparse_csr_tensor(self.t_crow, self.t_col, w[self.t_order], (self.n, self.n),
                                       check_invariants=False)

    def _structure(self):
        return self.crow32, self.pre32, self.n, self.n

    def _transposed(self):
        if getattr(self, "_t_order32", None) is None or self._t_order32.device != self.t_order.device:
            self._t_order32 = self.t_order.to(torch.int32)
        return self.t_crow32, self.t_col32, self._t_order32

    def _transposed_positions(self) -> torch.Tensor:
        """int32 (E,): each edge's position in the transposed order (the inverse of t_order), built on first
        use."""
        cached = getattr(self, "_t_pos32", None)
        if cached is None or cached.device != self.t_order.device:
            pos = torch.empty_like(self.t_order)
            pos[self.t_order] = torch.arange(self.t_order.numel(), device=self.t_order.device)
            self._t_pos32 = cached = pos.to(torch.int32)
        return cached

    def _edge_ids(self):
        return None

    def _backward_work(self):
        """The work list of products over W^T (backward_work), built on first use for the current structure."""
        t_crow32 = self._transposed()[0]
        cached = getattr(self, "_t_work", None)
        if cached is None or cached[0] is not t_crow32:
            self._t_work = (t_crow32, backward_work(t_crow32))
        return self._t_work[1]

    # ---- plans (everything that depends on the weights only; rebuilt when a parameter changes) -------
    def _plan(self, key_extra, build):
        key = self._param_key() + (key_extra,)
        plan = self._plans.get(key_extra)
        if plan is None or plan.key != key:
            self._plans.pop(key_extra, None)          # free the stale plan before building the new one
            handle = ctypes.c_void_p()
            with torch.no_grad():
                build(handle)
            plan = _Plan(handle, key)
            self._plans[key_extra] = plan
        return plan

    def _full_sweep(self):
        """The banded-sweep tables of the whole matrix (float32 states), built once per structure: every literal
        plan (each weight version) shares them.  None when the matrix does not sweep."""
        cached = getattr(self, "_full_sweep_tables", None)
        if cached is None or cached[0] is not self.crow32:
            self._full_sweep_tables = (self.crow32, _hip.sweep_create(self.crow32, self.pre32, self.n, self.n))
        return self._full_sweep_tables[1]

    def _full_plan(self, half: bool = False) -> _Plan:
        """The literal recurrence's plan for this weight version; `half`: its weights rounded to float16, as the
        reference's float16 forward rounds them (w.to(u.dtype), brain.py:215)."""
        def build(handle):
            w = self.edge_weights()
            if half:
                w = w.half().float()
            sweep = self._full_sweep()
            _hip.check(_hip.load().fly_plan_create_full(self.n, self.n_edges, self.crow32.data_ptr(),
                                                        self.pre32.data_ptr(), w.data_ptr(),
                                                        self.alpha_logit.data_ptr(), self._h_bound,
                                                        sweep.handle if sweep is not None else None,
                                                        _hip.stream(w.device), ctypes.byref(handle)),
                       "fly_plan_create_full")
        return self._plan(("full16",) if half else ("full",), build)

    def _cone_plan(self, cone: LightCone, mode: int) -> _Plan:
        def build(handle):
            w = self.edge_weights()
            _hip.check(_hip.load().fly_plan_create(cone.handle, self.crow32.data_ptr(), self.pre32.data_ptr(),
                                                   w.data_ptr(), self.bias.data_ptr(), self.alpha_logit.data_ptr(),
                                                   self._h_bound, mode, _hip.stream(w.device), ctypes.byref(handle)),
                       "fly_plan_create")
        return self._plan(("cone", mode, id(cone)), build)

    # ---- the literal recurrence ----------------------------------------------------------------------
    def forward(self, u: torch.Tensor, steps: int) -> torch.Tensor:
        """u: (N, B) contiguous constant external drive.  Returns the state after `steps` updates, (N, B).
        As in the reference's inference path, u is updated in place to u + bias (brain.py:218).  The recurrence
        runs in u's dtype (brain.py:215-216): float32; float64 (the float32 weights widen exactly); float16 (the
        weights and bias rounded to float16, a float16 state, its sums in float32).  A network converted to float64
        (.double()) runs in float64 through its float64 products, with or without autograd."""
        assert u.is_contiguous()
        _hip.require_device(u, "ConnectomeRNN.forward")
        if self._is_f64():
            return self._forward64(u, steps)
        self._check_params("ConnectomeRNN.forward")
        if torch.is_grad_enabled():
            return self._forward_autograd(u, steps)
        if u.dtype not in (torch.float16, torch.float32, torch.float64) or u.dim() != 2 or u.shape[0] != self.n:
            raise RuntimeError(f"ConnectomeRNN.forward: u must be float16, float32 or float64 ({self.n}, B), got "
                               f"{u.dtype} {tuple(u.shape)}")
        lib = _hip.load()
        batch = u.shape[1]
        h = torch.empty_like(u)
        # the recurrence runs in u's dtype (brain.py:215-216): float64 widens the float32 weights exactly; float16
        # rounds them to float16 and carries a float16 state, summed in float32
        name = {torch.float16: "fly_forward_literal_f16", torch.float32: "fly_forward_literal",
                torch.float64: "fly_forward_literal_f64"}[u.dtype]
        plan = self._full_plan(half=u.dtype == torch.float16)
        ws = _hip.workspace(getattr(lib, name + "_workspace")(plan.handle, batch), u.device)
        _hip.check(getattr(lib, name)(plan.handle, u.data_ptr(), batch, self.bias.data_ptr(), batch, int(steps),
                                      h.data_ptr(), batch, ws.data_ptr(), ws.numel(), _hip.stream(u.device)), name)
        return h

    def _forward_autograd(self, u: torch.Tensor, steps: int) -> torch.Tensor:
        """The literal recurrence under autograd, float32 (brain.py:225-229); u is not modified."""
        if u.dtype != torch.float32:
            raise RuntimeError(f"ConnectomeRNN.forward under autograd runs in float32, got {u.dtype}")
        alpha = torch.sigmoid(self.alpha_logit).unsqueeze(1)
        w = self.edge_weights()
        drive = self.bias.unsqueeze(1) + u
        h = torch.zeros_like(drive)
        for _ in range(steps):
            x = (_SparseRecurrent.apply(h, w, self) + drive).clamp(0, self.h_max)
            h = torch.lerp(h, x, alpha)
        return h

    def _forward_io_autograd(self, u_in: torch.Tensor, cone: LightCone, out_idx: torch.Tensor,
                             steps: int) -> torch.Tensor:
        """forward_io under autograd, float32 (brain.py:289-329): rows outside R_t follow the resting
        trajectory, rows of R_t take the sub-matrix product plus their constant drive and input."""
        if u_in.dtype != torch.float32:
            raise RuntimeError(f"forward_io under autograd runs in float32, got {u_in.dtype}")
        batch = u_in.shape[1]
        w = self.edge_weights()
        alpha = torch.sigmoid(self.alpha_logit).unsqueeze(1)
        rest = _RestingTrajectory.apply(self, cone, out_idx, w, self.bias, alpha)
        flat = []
        for t in range(1, steps + 1):
            flat += [rest[t - 1], rest[steps + t - 1], _take_rows(alpha, cone.rows[t])]
        h = _ConeRecurrence.apply(cone, self._h_bound, self, u_in, w, *flat)
        out = rest[2 * steps].expand(-1, batch)
        return out.index_copy(0, cone.out_pos, _take_rows(h, cone.out_src))

    # ---- the same function through the light cone ------------------------------------------------
    def light_cone(self, in_idx: torch.Tensor, out_idx: torch.Tensor, steps: int, prune: bool = True) -> LightCone:
        """The rows each step computes (cached by the index tensors, like brain.py:232-236).  prune=False
        computes every neuron at every step: the same function without the light cone."""
        key = (steps, in_idx.data_ptr(), out_idx.data_ptr(), str(self.pre.device), bool(prune))
        if self._cone is None or self._cone[0] != key:
            self._cone = None                         # release the old cone (and its plans) first
            self._plans = {k: v for k, v in self._plans.items() if k[0] in ("full", "full16")}
            self._cone = (key, LightCone(self, in_idx, out_idx, steps, prune))
        return self._cone[1]

    def forward_io(self, u_in: torch.Tensor, in_idx: torch.Tensor, out_idx: torch.Tensor, steps: int) -> torch.Tensor:
        """u_in: (len(in_idx), B) drive of the input neurons.  Returns the output neurons after `steps`
        updates, (len(out_idx), B): forward(u, steps)[out_idx] with u zero outside in_idx.  float16 u_in
        takes the deviation path and returns float32; float32 u_in takes the float32 path; float64 u_in runs the
        light cone in float64 over the float32 cache (brain.py:295-329 in u_in's dtype) and returns float64.
        Under autograd the float32 light cone runs differentiably (training).  A network converted to float64 runs
        the light cone in float64, with or without autograd."""
        _hip.require_device(u_in, "ConnectomeRNN.forward_io")
        if self._is_f64():
            if u_in.dim() != 2 or u_in.shape[0] != len(in_idx):
                raise RuntimeError(f"forward_io: u_in must be (len(in_idx), B), got {tuple(u_in.shape)}")
            return self._forward_io64(u_in, self.light_cone(in_idx, out_idx, steps), out_idx, steps)
        self._check_params("ConnectomeRNN.forward_io")
        if torch.is_grad_enabled():
            if u_in.dim() != 2 or u_in.shape[0] != len(in_idx):
                raise RuntimeError(f"forward_io: u_in must be (len(in_idx), B), got {tuple(u_in.shape)}")
            cone = self.light_cone(in_idx, out_idx, steps)
            return self._forward_io_autograd(u_in, cone, out_idx, steps)
        if u_in.dtype == torch.float16:
            mode = _hip.MODE_DEVIATION_F16
        elif u_in.dtype in (torch.float32, torch.float64):
            mode = _hip.MODE_F32
        else:
            raise RuntimeError(f"forward_io: u_in must be float16, float32 or float64, got {u_in.dtype}")
        if u_in.dim() != 2 or u_in.shape[0] != len(in_idx):
            raise RuntimeError(f"forward_io: u_in must be (len(in_idx), B), got {tuple(u_in.shape)}")
        cone = self.light_cone(in_idx, out_idx, steps)
        plan = self._cone_plan(cone, mode)
        batch = u_in.shape[1]
        if u_in.stride(1) != 1 or (batch > 1 and u_in.stride(0) < batch):
            u_in = u_in.contiguous()
        f64 = u_in.dtype == torch.float64
        out = torch.empty(len(out_idx), batch, dtype=torch.float64 if f64 else torch.float32, device=u_in.device)
        lib = _hip.load()
        size = lib.fly_forward_io_f64_workspace if f64 else lib.fly_forward_io_workspace
        run = lib.fly_forward_io_f64 if f64 else lib.fly_forward_io
        ws = _hip.workspace(size(plan.handle, batch), u_in.device)
        ldu = u_in.stride(0) if u_in.shape[0] > 1 else batch
        _hip.check(run(plan.handle, u_in.data_ptr(), ldu, batch, out.data_ptr(), batch, ws.data_ptr(), ws.numel(),
                       _hip.stream(u_in.device)), "fly_forward_io_f64" if f64 else "fly_forward_io")
        return out

    def resting_outputs(self, in_idx: torch.Tensor, out_idx: torch.Tensor, steps: int) -> torch.Tensor:
        """c_T[out_idx]: the outputs of a network that sees no position (float32)."""
        cone = self.light_cone(in_idx, out_idx, steps)
        plan = self._cone_plan(cone, _hip.MODE_DEVIATION_F16)
        out = torch.empty(len(out_idx), dtype=torch.float32, device=self.pre.device)
        _hip.check(_hip.load().fly_plan_resting(plan.handle, out.data_ptr(), _hip.stream(out.device)),
                   "fly_plan_resting")
        return out
