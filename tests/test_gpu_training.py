"""GPU tests of the training path: the device sparse products (fly_spmm, fly_sddmm, through the C ABI and
through _SparseRecurrent) and the gradients of ConnectomeRNN.forward / forward_io / FlyChessNet.forward
under autograd, against the CPU training oracle (float64)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import brain_arrays, random_params, tiny_connectome

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _close(got: torch.Tensor, ref: torch.Tensor, rel: float, what: str) -> None:
    """max |got - ref| within rel * max |ref| (float32 device arithmetic against a float64 oracle)."""
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    scale = float(ref.abs().max()) if ref.numel() else 0.0
    err = float((got - ref).abs().max()) if ref.numel() else 0.0
    assert err <= rel * scale + 1e-30, f"{what}: max error {err:.3e} against max {scale:.3e}"


def _random_csr(rows: int, cols: int, nnz: int, seed: int):
    """Row-sorted non-zeros with empty rows, columns never used and repeated (row, column) pairs."""
    rng = np.random.default_rng(seed)
    r = np.sort(rng.integers(0, max(rows - 2, 1), nnz))          # the last rows stay empty
    c = rng.integers(0, max(cols - 1, 1), nnz)                   # the last column is never read
    c[1::7] = c[::7][:len(c[1::7])]
    r[1::7] = r[::7][:len(r[1::7])]                               # repeats of the previous pair
    order = np.lexsort((c, r))
    r, c = r[order], c[order]
    crow = np.zeros(rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=rows), out=crow[1:])
    return crow, r, c, rng.normal(0, 1, nnz)


def _heavy_csr(rows: int, cols: int, seed: int):
    """Lognormal row lengths (like a transposed connectome) with rows of 700 and 1500 non-zeros, one of them in a
    last, partial group of 8 rows, and empty rows."""
    rng = np.random.default_rng(seed)
    counts = np.minimum(rng.lognormal(np.log(20), 1.2, rows).astype(np.int64), 400)
    counts[5], counts[rows - 3], counts[rows - 1] = 1500, 700, 0
    counts[40:48] = 0
    r = np.repeat(np.arange(rows), counts)
    c = rng.integers(0, max(cols - 1, 1), len(r))
    order = np.lexsort((c, r))
    r, c = r[order], c[order]
    crow = np.zeros(rows + 1, np.int64)
    np.cumsum(counts, out=crow[1:])
    return crow, r, c, rng.normal(0, 1, len(r))


@pytest.mark.parametrize("batch,ld_pad,heavy", [(1, 0, False), (3, 0, False), (5, 3, False), (64, 0, False),
                                                (256, 0, False), (130, 2, False), (1, 0, True), (1, 3, True),
                                                (64, 0, True)])
def test_spmm_and_sddmm_match_float64(batch, ld_pad, heavy):
    """y = A x and out[e] = sum_b g[row_e, b] x[col_e, b] against float64, on 4-byte and 16-byte lanes; the
    heavy-tailed matrices take the batch-1 kernels' whole-wave path for rows past 256 non-zeros."""
    from chessfly import _hip
    lib = _hip.load()
    rows, cols = 701, 500
    crow, r, c, val = _heavy_csr(rows, cols, batch) if heavy else _random_csr(rows, cols, 9000, batch)
    nnz = len(r)
    rng = np.random.default_rng(batch + 1)
    x = rng.normal(0, 1, (cols, batch + ld_pad))
    g = rng.normal(0, 1, (rows, batch + ld_pad))
    dense = np.zeros((rows, cols))
    np.add.at(dense, (r, c), val)
    d32 = lambda a, dt=torch.int32: torch.as_tensor(np.ascontiguousarray(a), device=DEV).to(dt)
    crow_d, col_d, val_d = d32(crow), d32(c), d32(val, torch.float32)
    x_d, g_d = d32(x, torch.float32), d32(g, torch.float32)
    ld = batch + ld_pad
    y = torch.full((rows, ld), 7.0, device=DEV)
    st = _hip.stream(torch.device(DEV))
    _hip.check(lib.fly_spmm(crow_d.data_ptr(), col_d.data_ptr(), val_d.data_ptr(), None, 0, rows, cols,
                            x_d.data_ptr(), ld, batch, y.data_ptr(), ld, 0, st), "fly_spmm")
    ref = dense @ x[:, :batch]
    _close(y[:, :batch], torch.as_tensor(ref), 1e-5, "spmm")
    y2 = y.clone()
    # values through an index into a larger vector, accumulating
    perm = torch.randperm(3 * nnz, device=DEV)[:nnz]
    big = torch.zeros(3 * nnz, device=DEV)
    big[perm] = val_d
    perm32 = perm.to(torch.int32)
    _hip.check(lib.fly_spmm(crow_d.data_ptr(), col_d.data_ptr(), big.data_ptr(), perm32.data_ptr(),
                            big.numel(), rows, cols, x_d.data_ptr(), ld, batch, y2.data_ptr(), ld, 1, st),
               "fly_spmm accumulate")
    _close(y2[:, :batch], torch.as_tensor(2 * ref), 1e-5, "spmm accumulate through value ids")
    if ld_pad:
        assert bool((y[:, batch:] == 7.0).all())                # padding columns are not written
    out = torch.empty(nnz, device=DEV)
    _hip.check(lib.fly_sddmm(crow_d.data_ptr(), col_d.data_ptr(), rows, cols, g_d.data_ptr(), ld, x_d.data_ptr(), ld,
                             batch, out.data_ptr(), out.numel(), None, 0, st), "fly_sddmm")
    ref_w = (g[r, :batch] * x[c, :batch]).sum(1)
    _close(out, torch.as_tensor(ref_w), 1e-5, "sddmm")
    # scattered into a larger vector by distinct ids, accumulating
    ids = torch.randperm(2 * nnz, device=DEV)[:nnz].to(torch.int32)
    big = torch.ones(2 * nnz, device=DEV)
    _hip.check(lib.fly_sddmm(crow_d.data_ptr(), col_d.data_ptr(), rows, cols, g_d.data_ptr(), ld, x_d.data_ptr(), ld,
                             batch, big.data_ptr(), big.numel(), ids.data_ptr(), 1, st), "fly_sddmm ids")
    want = torch.ones(2 * nnz, dtype=torch.float64)
    want[ids.long().cpu()] += torch.as_tensor(ref_w)
    _close(big, want, 1e-5, "sddmm scattered")


@pytest.mark.parametrize("batch,heavy,seg,chunked", [
    (4, False, None, False), (64, False, None, False), (200, False, None, False), (256, False, None, False),
    (64, False, 64, False), (256, True, None, False), (256, True, 256, False), (4, True, 64, False),
    (200, True, 128, False),
    (4, False, None, True), (200, False, None, True), (256, True, None, True), (256, True, 256, True),
    (64, False, 64, True), (200, True, 128, True), (328, True, 64, True)])
def test_transposed_backward_matches_float64(batch, heavy, seg, chunked):
    """fly_transposed_backward: grad_h (+)= A^T g and gw[ids[e]] += sum_b g[row_e, b] h[col_e, b] in one pass,
    against float64, on a matrix with rows of A^T longer than one block of 64 non-zeros and empty ones; with a
    work list (seg: segment length) long rows run as several segments whose shares meet in slot order.  Chunked:
    the chunk-major pass with its dots workspace (a ragged last chunk at 200 and 328 columns)."""
    from chessfly import _hip
    from chessfly.brain import backward_work
    lib = _hip.load()
    rows, cols = 400, 300
    if heavy:                                                   # lognormal rows of A^T, up to 1500 non-zeros
        t_crow_h, rt, ct, val = _heavy_csr(cols, rows, batch + 7)
        r, c = ct, rt
        nnz = len(r)
    else:                                                       # ~100 non-zeros per row of A^T
        nnz = 30000
        crow, r, c, val = _random_csr(rows, cols, nnz, batch + 7)
    order = np.lexsort((r, c))                                  # A^T in CSR: by column, then row
    t_crow = np.zeros(cols + 1, np.int64)
    np.cumsum(np.bincount(c, minlength=cols), out=t_crow[1:])
    rng = np.random.default_rng(batch)
    g = rng.normal(0, 1, (rows, batch))
    h = rng.normal(0, 1, (cols, batch))
    gh0 = rng.normal(0, 1, (cols, batch))
    ids = rng.permutation(2 * nnz)[:nnz]                         # each non-zero's slot in a longer vector
    gw0 = rng.normal(0, 1, 2 * nnz)
    d = lambda a, dt=torch.float32: torch.as_tensor(np.ascontiguousarray(a), device=DEV).to(dt)
    # every operand bound to a name that lives across the call (a temporary freed in the argument list
    # could be handed to the next one and overwritten before the kernel reads it)
    t_crow_d, t_col_d, t_val_d, t_ids_d = d(t_crow, torch.int32), d(r[order], torch.int32), d(val[order]), \
        d(ids[order], torch.int32)
    g_d, h_d, gh, gw = d(g), d(h), d(gh0), d(gw0)
    st = _hip.stream(torch.device(DEV))
    items = splits = partials = None
    n_items = n_splits = n_slots = 0
    if seg is not None:
        items, splits, n_slots = backward_work(t_crow_d, seg)
        n_items, n_splits = items.shape[0], splits.shape[0]
        partials = torch.full((n_slots, batch), float("nan"), device=DEV)   # every slot is written before use
        assert n_slots > 0 or not heavy
    # every (chunk, non-zero) dot is written before k_dots_to_gw reads it
    dots = torch.full(((batch + 63) // 64 * nnz,), float("nan"), device=DEV) if chunked else None
    _hip.check(lib.fly_transposed_backward(t_crow_d.data_ptr(), t_col_d.data_ptr(), t_val_d.data_ptr(),
                                           t_ids_d.data_ptr(), nnz, cols, rows, g_d.data_ptr(), batch, h_d.data_ptr(),
                                           batch, batch, gh.data_ptr(), batch, 1, gw.data_ptr(), gw.numel(),
                                           _hip.ptr(items), n_items, _hip.ptr(splits), n_splits, _hip.ptr(partials),
                                           n_slots, _hip.ptr(dots), dots.numel() if chunked else 0, st),
               "fly_transposed_backward")
    dense = np.zeros((rows, cols))
    np.add.at(dense, (r, c), val)
    _close(gh, torch.as_tensor(gh0 + dense.T @ g), 1e-5, "grad_h")
    want = gw0.copy()
    want[ids] += (g[r] * h[c]).sum(1)
    _close(gw, torch.as_tensor(want), 1e-5, "dL/dw")


@pytest.mark.parametrize("heavy,seg,accumulate", [(True, 256, 0), (True, 64, 1), (False, 64, 0), (False, 256, 1)])
def test_one_column_product_over_a_work_list_matches_float64(heavy, seg, accumulate):
    """fly_spmv_work: y (+)= A x for one column from backward_work's longest-first items, long rows as several
    segments whose partial sums are added in slot order, against float64; empty rows get 0 (or keep y)."""
    from chessfly import _hip
    from chessfly.brain import backward_work
    lib = _hip.load()
    rows, cols = 601, 450
    crow, r, c, val = _heavy_csr(rows, cols, seg + accumulate) if heavy else _random_csr(rows, cols, 20000, seg)
    nnz = len(r)
    rng = np.random.default_rng(seg)
    x = rng.normal(0, 1, (cols, 1))
    y0 = rng.normal(0, 1, (rows, 1))
    d = lambda a, dt=torch.float32: torch.as_tensor(np.ascontiguousarray(a), device=DEV).to(dt)
    crow_d, col_d, val_d, x_d, y = d(crow, torch.int32), d(c, torch.int32), d(val), d(x), d(y0)
    items, splits, n_slots = backward_work(crow_d, seg)
    assert n_slots > 0 or not heavy
    partials = torch.full((max(n_slots, 1),), float("nan"), device=DEV)   # every slot is written before use
    st = _hip.stream(torch.device(DEV))
    _hip.check(lib.fly_spmv_work(crow_d.data_ptr(), col_d.data_ptr(), val_d.data_ptr(), nnz, rows, cols,
                                 x_d.data_ptr(), 1, y.data_ptr(), 1, accumulate, items.data_ptr(), items.shape[0],
                                 splits.data_ptr(), splits.shape[0], partials.data_ptr(), n_slots, st),
               "fly_spmv_work")
    dense = np.zeros((rows, cols))
    np.add.at(dense, (r, c), val)
    want = dense @ x + (y0 if accumulate else 0.0)
    _close(y, torch.as_tensor(want), 1e-5, "spmv over the work list")


@pytest.mark.parametrize("batch", [4, 68, 256])
@pytest.mark.parametrize("hubs", [False, True])
def test_swept_forward_product_matches_float64(batch, hubs):
    """fly_spmm_swept (the forward product as a banded sweep, training batches that are multiples of 4) against
    float64 and fly_spmm, on a random CSR matrix that suits the sweep (70,000 rows of ~40 non-zeros over 40,000
    source rows), plain and with hub rows (longer than 3 x the mean + 10), which the tables split into pieces whose
    sums meet in k_sweep_finish; an inf in a source row reaches only the rows that read it."""
    from chessfly import _hip, brain
    rng = np.random.default_rng(batch)
    n_rows, n_cols = 70_000, 40_000
    lens = rng.poisson(40, n_rows)
    if hubs:
        lens[[5, 123, 69_999]] = [4 * int(lens.mean()) + 200, 2500, 900]
    crow = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    col = np.concatenate([np.sort(rng.integers(0, n_cols, n)) for n in lens]).astype(np.int32)
    val = rng.standard_normal(len(col)).astype(np.float32)
    x = rng.standard_normal((n_cols, batch)).astype(np.float32)
    crow32, col32 = torch.as_tensor(crow, device=DEV), torch.as_tensor(col, device=DEV)
    val_d, x_d = torch.as_tensor(val, device=DEV), torch.as_tensor(x, device=DEV)

    class Holder:
        pass

    holder = Holder()
    tables = brain._sweep_tables(holder, crow32, col32, n_rows, n_cols)
    assert tables is not None
    assert brain._sweep_tables(holder, crow32, col32, n_rows, n_cols) is tables     # built once per structure
    info = _hip.sweep_info(tables.handle)
    assert (info["split_rows"] == 3) == hubs and (info["pieces"] > 0) == hubs, info
    y = brain._spmm_swept(col32, val_d, tables, n_rows, x_d)
    y_ref = brain._spmm(crow32, col32, val_d, n_rows, n_cols, x_d)
    torch.cuda.synchronize()
    rows = np.repeat(np.arange(n_rows), lens)
    exact = np.zeros((n_rows, batch))
    np.add.at(exact, rows, val[:, None].astype(np.float64) * x[col].astype(np.float64))
    scale = np.abs(exact).max()
    err, err_ref = np.abs(y.cpu().numpy() - exact).max() / scale, np.abs(y_ref.cpu().numpy() - exact).max() / scale
    print(f"B={batch}, hubs {hubs} ({info}): swept {err:.2e}, fly_spmm {err_ref:.2e} of the largest |y|", flush=True)
    assert err < 1e-5 and err_ref < 1e-5
    # Tables for 128 workgroups with paired passes: each wave owns over 24 rows and walks two slots per pass.
    _hip.set_tuning("sweep_grid", 128)
    _hip.set_tuning("sweep_paired", 1)
    try:
        paired = _hip.sweep_create(crow32, col32, n_rows, n_cols)
    finally:
        _hip.set_tuning("sweep_grid", 0)
        _hip.set_tuning("sweep_paired", 0)
    assert _hip.sweep_info(paired.handle)["rows_per_wave"] > 24
    y2 = brain._spmm_swept(col32, val_d, paired, n_rows, x_d).cpu().numpy()
    assert np.abs(y2 - exact).max() / scale < 1e-5
    # an inf in one source row: the rows that read it are inf or NaN, every other row stays finite (a paired pass
    # changes only the owning row's sums when the operand is the caller's)
    src = int(col[crow[123]]) if hubs else int(col[0])
    x_inf = x_d.clone()
    x_inf[src] = float("inf")
    reads = np.zeros(n_rows, bool)
    reads[rows[col == src]] = True
    for tb in (tables, paired):
        y_inf = brain._spmm_swept(col32, val_d, tb, n_rows, x_inf).cpu().numpy()
        assert np.isfinite(y_inf[~reads]).all(), "a row that never reads the inf source is not finite"
        assert not np.isfinite(y_inf[reads]).any()


@pytest.mark.parametrize("batch", [4, 68, 200, 256])
@pytest.mark.parametrize("shape", ["by size", "by size with hubs", "forced, small and heavy-tailed"])
def test_swept_transposed_backward_matches_float64(batch, shape):
    """fly_transposed_backward_swept (the backward over A^T as a banded sweep of gy's rows): gh (+)= A^T gy and
    gw[ids[e]] += sum_b gy[i_e, b] h[j_e, b], against float64.  A^T with 70,000 rows of ~40 non-zeros over 40,000
    rows of gy (the size rule sweeps it), plain and with hub rows split into pieces; and a 300-row A^T with rows of
    up to 1,500 non-zeros and empty ones, swept by force on 4 workgroups (spread slots, several passes per wave).
    Batches end inside a 32-column chunk (68, 200); the workspace starts as NaN, so a dot left unwritten would show;
    a second call gives the same bits."""
    from chessfly import _hip
    lib = _hip.load()
    rng = np.random.default_rng([batch, len(shape)])
    if shape == "forced, small and heavy-tailed":
        n_t, n_g = 300, 400                                     # rows of A^T (= rows of h), rows of gy
        t_crow_h, rt, ct, val = _heavy_csr(n_t, n_g, batch + 11)
        t_crow = np.asarray(t_crow_h, np.int64)
        t_col = np.asarray(ct, np.int64)
        val = np.asarray(val, np.float32)
        keys = {"swept": 1, "sweep_grid": 4}
    else:
        n_t, n_g = 70_000, 40_000
        lens = rng.poisson(40, n_t)
        if shape == "by size with hubs":
            lens[[3, 4_321, 69_999]] = [3000, 900, 4 * int(lens.mean()) + 200]
        t_crow = np.concatenate([[0], np.cumsum(lens)])
        t_col = np.concatenate([np.sort(rng.integers(0, n_g, n)) for n in lens])
        val = rng.standard_normal(len(t_col)).astype(np.float32)
        keys = {}
    nnz = len(t_col)
    rows_t = np.repeat(np.arange(n_t), np.diff(t_crow))          # each non-zero's row of A^T
    gy = rng.standard_normal((n_g, batch)).astype(np.float32)
    h = rng.standard_normal((n_t, batch)).astype(np.float32)
    gh0 = rng.standard_normal((n_t, batch)).astype(np.float32)
    ids = rng.permutation(2 * nnz)[:nnz].astype(np.int32)        # each non-zero's slot in a longer vector
    gw0 = rng.standard_normal(2 * nnz).astype(np.float32)
    d = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=DEV)
    t_crow_d, t_col_d, val_d, ids_d = d(t_crow.astype(np.int32)), d(t_col.astype(np.int32)), d(val), d(ids)
    gy_d, h_d = d(gy), d(h)
    for k, v in keys.items():
        _hip.set_tuning(k, v)
    try:
        tables = _hip.sweep_create(t_crow_d, t_col_d, n_t, n_g)
    finally:
        for k in keys:
            _hip.set_tuning(k, 0)
    assert tables is not None, "the structure did not sweep"
    info = _hip.sweep_info(tables.handle)
    records = torch.stack((t_col_d, val_d.view(torch.int32)), dim=1)
    st = _hip.stream(torch.device(DEV))
    outs = []
    for _ in range(2):
        gh, gw = d(gh0), d(gw0)
        ws = _hip.workspace(lib.fly_transposed_backward_swept_workspace(tables.handle, batch), torch.device(DEV))
        ws.fill_(255)                                            # NaN floats
        _hip.check(lib.fly_transposed_backward_swept(tables.handle, records.data_ptr(), nnz, ids_d.data_ptr(),
                                                     gy_d.data_ptr(), batch, h_d.data_ptr(), batch, batch,
                                                     gh.data_ptr(), batch, 1, gw.data_ptr(), gw.numel(),
                                                     ws.data_ptr(), ws.numel(), st), "fly_transposed_backward_swept")
        torch.cuda.synchronize()
        outs.append((gh.cpu(), gw.cpu()))
    want_gh = gh0.astype(np.float64).copy()
    np.add.at(want_gh, rows_t, val[:, None].astype(np.float64) * gy[t_col].astype(np.float64))
    want_gw = gw0.astype(np.float64).copy()
    want_gw[ids] += (gy[t_col].astype(np.float64) * h[rows_t].astype(np.float64)).sum(1)
    print(f"{shape} B={batch}: {info}", flush=True)
    _close(outs[0][0], torch.as_tensor(want_gh), 1e-5, "grad_h")
    _close(outs[0][1], torch.as_tensor(want_gw), 1e-5, "dL/dw")
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), "not deterministic"


def _rnn64_pair(conn, seed: int, h_max=10.0, scale: float = 3.0):
    """A network converted to float64 (as the reference's tests convert theirs, tests/test_core.py:29, 312) with
    parameters that float32 cannot hold, and the oracle's arrays of the same float64 values."""
    from chessfly.brain import ConnectomeRNN
    lg, bias, al = random_params(conn, seed)
    rng = np.random.default_rng(seed + 1000)
    lg, bias, al = (a.astype(np.float64) + rng.normal(0, 1e-3, a.shape) for a in (lg, bias, al))
    rnn = ConnectomeRNN(conn, global_scale=scale, h_max=h_max).double().to(DEV)
    with torch.no_grad():
        rnn.log_gain.copy_(torch.as_tensor(lg))
        rnn.bias.copy_(torch.as_tensor(bias))
        rnn.alpha_logit.copy_(torch.as_tensor(al))
    b = brain_arrays(conn, scale, lg, bias, al, h_max=h_max, dtype=torch.double)
    b.w0 = rnn.w0.cpu()                                        # the network's own float64 weights
    for name in ("log_gain", "bias", "alpha_logit"):
        setattr(b, name, getattr(b, name).clone().requires_grad_(True))
    return rnn, b


@pytest.mark.parametrize("h_max", [10.0, None])
def test_float64_network_literal_recurrence_and_gradients(h_max):
    """A float64 network (ConnectomeRNN(...).double(), tests/test_core.py:28-44): the literal recurrence under
    autograd runs in float64 on the device (fly_spmm_f64, fly_sddmm_f64), state and gradients of u, log_gain, bias and
    alpha_logit against the oracle's float64 recurrence to 1e-10; without autograd the same state, with u left as
    u + bias (brain.py:218)."""
    from oracle import training as T
    conn = tiny_connectome(200, 3000, seed=1)
    rnn, b = _rnn64_pair(conn, 4, h_max=h_max)
    assert rnn.log_gain.dtype == torch.float64
    rng = np.random.default_rng(5)
    u = rng.random((conn.n_neurons, 6)) * (3.0 if h_max is None else 1.0)
    target = rng.random((conn.n_neurons, 6))
    u_d = torch.tensor(u, device=DEV, requires_grad=True)
    out = rnn(u_d, 5)
    assert out.dtype == torch.float64
    ((out - torch.as_tensor(target, device=DEV)) ** 2).sum().backward()
    u_r = torch.tensor(u, requires_grad=True)
    ref = T.literal_grad(b, u_r, 5)
    ((ref - torch.as_tensor(target)) ** 2).sum().backward()
    _close(out, ref, 1e-10, "state")
    for got, want, name in zip(_device_grads(rnn, u_d), (u_r.grad, b.log_gain.grad, b.bias.grad, b.alpha_logit.grad),
                               ("u", "log_gain", "bias", "alpha_logit")):
        assert float(want.abs().max()) > 0, name
        _close(got, want, 1e-10, name)
    u2 = torch.tensor(u, device=DEV)
    with torch.no_grad():
        h = rnn(u2, 5)
    _close(h, ref, 1e-10, "state without autograd")
    assert torch.equal(u2.cpu(), torch.as_tensor(u) + b.bias.detach()[:, None]), "u + bias in place"


@pytest.mark.parametrize("steps", [1, 2, 4, 6])
def test_float64_network_light_cone_equals_the_literal_recurrence(steps):
    """A float64 network's forward_io (tests/test_core.py:309-338): outputs and the gradients of u_in, log_gain, bias
    and alpha_logit equal the literal recurrence's at the output rows (to 1e-9) and the oracle's float64 light cone
    (oracle.training.cone_grad); without autograd the same outputs."""
    from oracle import training as T
    from oracle.lightcone import light_cone
    conn = tiny_connectome(120, 700, seed=3)
    rnn, b = _rnn64_pair(conn, 6)
    in_idx, out_idx = torch.arange(0, 9, device=DEV), torch.arange(100, 120, device=DEV)
    rng = np.random.default_rng(steps)
    u_in = rng.normal(0, 1, (9, 5))
    target = torch.as_tensor(rng.normal(0, 1, (20, 5)), device=DEV)
    results = []
    for mode in ("literal", "cone"):
        rnn.zero_grad()
        u_d = torch.tensor(u_in, device=DEV, requires_grad=True)
        if mode == "literal":
            u = torch.zeros(conn.n_neurons, 5, dtype=torch.float64, device=DEV).index_add(0, in_idx, u_d)
            out = rnn(u.contiguous(), steps)[out_idx]
        else:
            out = rnn.forward_io(u_d, in_idx, out_idx, steps)
        ((out - target) ** 2).sum().backward()
        results.append([out.detach()] + [g if g is not None else torch.zeros_like(p)
                                         for g, p in zip(_device_grads(rnn, u_d), (u_d, rnn.log_gain, rnn.bias,
                                                                                    rnn.alpha_logit))])
    names = ("out", "u_in", "log_gain", "bias", "alpha_logit")
    for lit, cone_r, name in zip(results[0], results[1], names):
        _close(cone_r, lit, 1e-9, f"{name}: light cone against the literal recurrence")
    assert steps == 1 or float(results[1][2].abs().max()) > 0
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.arange(9), np.arange(100, 120), steps)
    u_r = torch.tensor(u_in, requires_grad=True)
    ref = T.cone_grad(b, cone, u_r)
    ((ref - target.cpu()) ** 2).sum().backward()
    wants = (ref.detach(), u_r.grad, b.log_gain.grad, b.bias.grad, b.alpha_logit.grad)
    for got, want, name in zip(results[1], wants, names):
        want = torch.zeros_like(got.cpu()) if want is None else want     # one step never reaches W
        _close(got, want, 1e-10, f"{name}: against the oracle")
    with torch.no_grad():
        _close(rnn.forward_io(torch.tensor(u_in, device=DEV), in_idx, out_idx, steps), results[1][0], 1e-12,
               "forward_io without autograd")


def test_gather_values_reads_the_weight_vector_at_int32_ids():
    """fly_gather_values: out[i] = w[ids[i]] (a sub-matrix's values in its own or its transpose's order), ids past
    the vector (and negative ones) read 0, bit for bit."""
    from chessfly import _hip
    lib = _hip.load()
    g = torch.Generator(device=DEV).manual_seed(4)
    w = torch.randn(100_003, device=DEV, generator=g)
    ids = torch.randint(0, w.numel(), (300_001,), device=DEV, generator=g, dtype=torch.int32)
    ids[::97] = w.numel()
    ids[5::101] = -3
    out = torch.full((ids.numel(),), float("nan"), device=DEV)
    _hip.check(lib.fly_gather_values(w.data_ptr(), w.numel(), ids.data_ptr(), ids.numel(), out.data_ptr(),
                                     _hip.stream(torch.device(DEV))), "fly_gather_values")
    ok = (ids >= 0) & (ids < w.numel())
    want = torch.where(ok, w[ids.clamp(0, w.numel() - 1).long()], torch.zeros(()).to(DEV))
    assert torch.equal(out, want)


def _rnn_pair(conn, seed: int, scale: float = 3.0):
    from chessfly.brain import ConnectomeRNN
    lg, bias, al = random_params(conn, seed)
    rnn = ConnectomeRNN(conn, global_scale=scale).to(DEV)
    with torch.no_grad():
        rnn.log_gain.copy_(torch.as_tensor(lg))
        rnn.bias.copy_(torch.as_tensor(bias))
        rnn.alpha_logit.copy_(torch.as_tensor(al))
    b = brain_arrays(conn, scale, lg, bias, al, dtype=torch.double)
    for name in ("log_gain", "bias", "alpha_logit"):
        setattr(b, name, getattr(b, name).clone().requires_grad_(True))
    return rnn, b


def _device_grads(rnn, *extra):
    return [t.grad for t in (*extra, rnn.log_gain, rnn.bias, rnn.alpha_logit)]


def test_forward_gradients_match_the_oracle():
    """ConnectomeRNN.forward under autograd: the state and the gradients of u, log_gain, bias and alpha_logit
    (chessfly/brain.py:224-229 with _SparseRecurrent, 66-99)."""
    from oracle import training as T
    conn = tiny_connectome(200, 3000, seed=1)
    rnn, b = _rnn_pair(conn, 2)
    rng = np.random.default_rng(3)
    u = rng.random((conn.n_neurons, 16))
    target = rng.random((conn.n_neurons, 16))
    u_d = torch.tensor(u, dtype=torch.float32, device=DEV, requires_grad=True)
    out = rnn(u_d, 4)
    ((out - torch.as_tensor(target, dtype=torch.float32, device=DEV)) ** 2).sum().backward()
    u_r = torch.tensor(u, requires_grad=True)
    ref = T.literal_grad(b, u_r, 4)
    ((ref - torch.as_tensor(target)) ** 2).sum().backward()
    _close(out, ref, 2e-6, "state")
    for got, want, name in zip(_device_grads(rnn, u_d), (u_r.grad, b.log_gain.grad, b.bias.grad, b.alpha_logit.grad),
                               ("u", "log_gain", "bias", "alpha_logit")):
        _close(got, want, 5e-5, name)
    assert float(rnn.log_gain.grad.abs().sum()) > 0


@pytest.mark.parametrize("steps", [1, 2, 4, 6])
def test_forward_io_gradients_match_the_oracle_and_the_full_recurrence(steps):
    """forward_io under autograd (the light cone, chessfly/brain.py:289-329) against the oracle, and against
    forward()[out_idx] on the device: the same function with every gradient."""
    from oracle import training as T
    from oracle.lightcone import light_cone
    conn = tiny_connectome(120, 700, seed=3)
    rnn, b = _rnn_pair(conn, 4)
    in_idx, out_idx = torch.arange(0, 9, device=DEV), torch.arange(100, 120, device=DEV)
    rng = np.random.default_rng(steps)
    u_in = rng.normal(0, 1, (9, 5))
    target = torch.as_tensor(rng.normal(0, 1, (20, 5)))
    results = []
    for mode in ("full", "cone"):
        rnn.zero_grad()
        u_d = torch.tensor(u_in, dtype=torch.float32, device=DEV, requires_grad=True)
        if mode == "full":
            u = torch.zeros(conn.n_neurons, 5, device=DEV).index_add(0, in_idx, u_d)
            out = rnn(u.contiguous(), steps)[out_idx]
        else:
            out = rnn.forward_io(u_d, in_idx, out_idx, steps)
        ((out - target.float().to(DEV)) ** 2).sum().backward()
        results.append([out.detach()] + [g.clone() if g is not None else None for g in _device_grads(rnn, u_d)])
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.arange(9), np.arange(100, 120), steps)
    u_r = torch.tensor(u_in, requires_grad=True)
    ref = T.cone_grad(b, cone, u_r)
    ((ref - target) ** 2).sum().backward()
    refs = [ref.detach(), u_r.grad, b.log_gain.grad, b.bias.grad, b.alpha_logit.grad]
    names = ("out", "u_in", "log_gain", "bias", "alpha_logit")
    for got_full, got_cone, want, name in zip(results[0], results[1], refs, names):
        if want is None:                                      # one step never uses W
            assert got_cone is None or float(got_cone.abs().max()) == 0.0
            continue
        _close(got_cone, want, 5e-5, f"cone {name}")
        _close(got_full, want, 5e-5, f"full {name}")


@pytest.mark.parametrize("batch", [8, 200])
@pytest.mark.parametrize("swept", [False, True])
def test_cone_gradients_over_the_transposed_pass_match_the_oracle_and_repeat_exactly(batch, swept):
    """forward_io under autograd at batches that take the one pass over A^T (multiples of 4): one chunk (8
    boards) and chunk-major with a ragged last chunk (200), on a 3,000-neuron synthetic graph whose longest rows
    of A^T (out-degrees up to 870) run as several work-list segments.  Gradients against the oracle in float64
    (chessfly/brain.py:289-329), and a second run from the same state gives the same bits: partial rows meet
    in slot order, the chunks' dots add in order, and dL/dw returns from W^T's order by a gather.  `swept`: the
    sweep forced onto the graph's structures (4 workgroups), so the forward products and the passes over A^T run
    as banded sweeps, with the long rows of A^T split into pieces."""
    from chessfly import _hip
    from chessfly.synthetic import GraphSpec, synthetic_connectome
    from oracle import training as T
    from oracle.lightcone import light_cone
    conn = synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=5))
    rnn, b = _rnn_pair(conn, 6)
    in_idx, out_idx = torch.arange(0, 300, device=DEV), torch.arange(2900, 3000, device=DEV)
    rng = np.random.default_rng(batch)
    u_in = rng.normal(0, 1, (300, batch))
    target = torch.as_tensor(rng.normal(0, 1, (100, batch)))
    runs = []
    keys = {"swept": 1, "sweep_grid": 4} if swept else {}
    for k, v in keys.items():
        _hip.set_tuning(k, v)
    try:
        for _ in range(2):
            rnn.zero_grad()
            u_d = torch.tensor(u_in, dtype=torch.float32, device=DEV, requires_grad=True)
            out = rnn.forward_io(u_d, in_idx, out_idx, 6)
            ((out - target.float().to(DEV)) ** 2).sum().backward()
            runs.append([out.detach().clone()] + [g.clone() for g in _device_grads(rnn, u_d)])
    finally:
        for k in keys:
            _hip.set_tuning(k, 0)
    if swept:
        dcone = rnn.light_cone(in_idx, out_idx, 6)
        ops = [op for op in dcone.ops if op is not None]
        assert any(getattr(op, "_sweep_t", (None, None))[1] is not None for op in ops), "no pass over A^T swept"
    names = ("out", "u_in", "log_gain", "bias", "alpha_logit")
    for first, second, name in zip(runs[0], runs[1], names):
        assert torch.equal(first, second), f"{name} differs between two identical runs"
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), np.arange(300), np.arange(2900, 3000), 6)
    u_r = torch.tensor(u_in, requires_grad=True)
    ref = T.cone_grad(b, cone, u_r)
    ((ref - target) ** 2).sum().backward()
    refs = (ref.detach(), u_r.grad, b.log_gain.grad, b.bias.grad, b.alpha_logit.grad)
    for got, want, name in zip(runs[0], refs, names):
        assert float(want.abs().max()) > 0, name
        _close(got, want, 1e-4, name)


def test_train_step_gradients_match_the_oracle():
    """One train_step loss (chessfly/train.py:126-132) through FlyChessNet under autograd on a 3,000-neuron
    synthetic graph: every parameter's gradient against the oracle in float64."""
    from chessfly.encoding import N_BASE, N_MOVES
    from chessfly.model import FlyChessNet, ModelConfig
    from chessfly.synthetic import GraphSpec, synthetic_boards, synthetic_connectome
    from oracle import training as T
    from oracle.forward import HeadArrays
    from oracle.lightcone import light_cone
    spec = GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=5)
    conn = synthetic_connectome(spec)
    torch.manual_seed(0)
    net = FlyChessNet(conn, ModelConfig(steps=4)).to(DEV).eval()
    with torch.no_grad():
        for p in net.parameters():
            p.add_(torch.randn_like(p) * 0.05)
    batch = 12
    x = torch.as_tensor(synthetic_boards(batch, seed=3), dtype=torch.float32)
    rng = np.random.default_rng(0)
    legal = torch.as_tensor(rng.random((batch, N_MOVES)) < 0.01)
    legal[:, 0] = True
    pi = torch.where(legal, torch.as_tensor(rng.random((batch, N_MOVES))), torch.zeros(()))
    pi = pi / pi.sum(1, keepdim=True)
    wdl = torch.as_tensor(rng.integers(0, 3, batch))
    net.zero_grad()
    logits, wdl_logits = net(x.to(DEV))
    T.train_loss(logits, wdl_logits, pi.float().to(DEV), legal.to(DEV), wdl.to(DEV)).backward()

    brain = net.brain
    d = lambda t: t.detach().double().cpu().clone().requires_grad_(True)
    b = brain_arrays(conn, net.cfg.weight_scale, brain.log_gain.detach().cpu(), brain.bias.detach().cpu(),
                     brain.alpha_logit.detach().cpu(), dtype=torch.double)
    for name in ("log_gain", "bias", "alpha_logit"):
        setattr(b, name, getattr(b, name).clone().requires_grad_(True))
    hp = HeadArrays(d(net.encoder.weight), d(net.encoder.bias), net.cfg.input_gain, N_BASE, d(net.policy.weight),
                    d(net.policy.bias), d(net.policy_from.weight), d(net.policy_from.bias), d(net.policy_to.weight),
                    d(net.policy_to.bias), d(net.value.weight), d(net.value.bias), net.move_from.cpu(),
                    net.move_to.cpu(), net.norm.mean.double().cpu(), net.norm.var.double().cpu())
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), net.in_idx.cpu().numpy(),
                      net.out_idx.cpu().numpy(), net.cfg.steps)
    rl, rw = T.model_grad(hp, b, cone, x.double())
    T.train_loss(rl, rw, pi.double(), legal, wdl).backward()
    _close(logits, rl, 1e-5, "logits")
    pairs = [(net.encoder.weight.grad[:, :N_BASE], hp.enc_w.grad[:, :N_BASE], "encoder.weight"),
             (net.encoder.bias.grad, hp.enc_b.grad, "encoder.bias"),
             (brain.log_gain.grad, b.log_gain.grad, "brain.log_gain"), (brain.bias.grad, b.bias.grad, "brain.bias"),
             (brain.alpha_logit.grad, b.alpha_logit.grad, "brain.alpha_logit"),
             (net.policy.weight.grad, hp.policy_w.grad, "policy.weight"),
             (net.policy_from.weight.grad, hp.from_w.grad, "policy_from.weight"),
             (net.policy_to.bias.grad, hp.to_b.grad, "policy_to.bias"),
             (net.value.weight.grad, hp.value_w.grad, "value.weight")]
    for got, want, name in pairs:
        assert float(want.abs().max()) > 0, name
        _close(got, want, 2e-4, name)
    assert float(net.encoder.weight.grad[:, N_BASE:].abs().sum()) == 0   # attack planes off: no gradient


def test_training_head_square_maps_equal_the_indexing_exactly():
    """The training forward adds the from/to-square heads as f @ one-hot maps (model.py:104-110 index them):
    bit-identical on the device to f[:, move_from] and f[:, move_to]."""
    from chessfly.model import FlyChessNet, ModelConfig
    from chessfly.synthetic import GraphSpec, synthetic_connectome
    conn = synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=5))
    net = FlyChessNet(conn, ModelConfig(steps=4)).to(DEV)
    f = torch.randn(37, 64, device=DEV, generator=torch.Generator(device=DEV).manual_seed(1)) * 100
    assert torch.equal(f @ net.move_from_onehot, f[:, net.move_from])
    assert torch.equal(f @ net.move_to_onehot, f[:, net.move_to])


def test_training_mode_without_autograd_updates_the_normaliser_and_matches_eval():
    """Training mode with autograd off (the reference's self-play-time calls between steps) runs the fused
    recurrence, then the normaliser updates its running statistics as RunningNorm does."""
    from chessfly.model import FlyChessNet, ModelConfig
    from chessfly.synthetic import GraphSpec, synthetic_boards, synthetic_connectome
    conn = synthetic_connectome(GraphSpec(n=3000, edges=120_000, n_sensory=300, n_output=100, seed=6))
    net = FlyChessNet(conn, ModelConfig(steps=4)).to(DEV)
    with torch.no_grad():                       # the zero-initialised heads would hide the normaliser
        for layer in (net.policy, net.value):
            layer.weight.normal_(0, 0.1)
    x = torch.as_tensor(synthetic_boards(16, seed=2), dtype=torch.float32, device=DEV)
    net.train()
    with torch.no_grad():
        logits_train, _ = net(x)
    assert bool(net.norm.initialised) and float(net.norm.mean.abs().sum()) > 0
    net.eval()
    with torch.no_grad():
        logits_eval, _ = net(x)
    _close(logits_eval, logits_train, 2e-3, "eval after the first training-mode call")


@pytest.mark.parametrize("batch", [4, 68])
def test_full_scale_train_step_gradients_match_the_oracle(full_net, batch):
    """The train_step loss on the full 166,700-neuron synthetic network (6 steps): every parameter's gradient
    against the oracle in float64.  4 positions take the one-chunk pass over A^T; 68 take the chunk-major pass
    with a ragged second chunk.  Only gradients are computed; the shared network's parameters are not
    changed."""
    from chessfly.encoding import N_BASE, N_MOVES
    from chessfly.synthetic import synthetic_boards
    from oracle import training as T
    from oracle.forward import HeadArrays
    from oracle.lightcone import light_cone
    net, conn = full_net
    x = torch.as_tensor(synthetic_boards(batch, seed=11), dtype=torch.float32)
    rng = np.random.default_rng(1)
    legal = torch.as_tensor(rng.random((batch, N_MOVES)) < 0.01)
    legal[:, 0] = True
    pi = torch.where(legal, torch.as_tensor(rng.random((batch, N_MOVES))), torch.zeros(()))
    pi = pi / pi.sum(1, keepdim=True)
    wdl = torch.as_tensor(rng.integers(0, 3, batch))
    net.zero_grad(set_to_none=True)
    try:
        logits, wdl_logits = net(x.to(DEV))
        T.train_loss(logits, wdl_logits, pi.float().to(DEV), legal.to(DEV), wdl.to(DEV)).backward()
        got = {"log_gain": net.brain.log_gain.grad.cpu(), "bias": net.brain.bias.grad.cpu(),
               "alpha_logit": net.brain.alpha_logit.grad.cpu(), "encoder": net.encoder.weight.grad[:, :N_BASE].cpu(),
               "policy": net.policy.weight.grad.cpu(), "value": net.value.weight.grad.cpu()}
        logits = logits.detach().cpu()
    finally:
        net.zero_grad(set_to_none=True)
    brain = net.brain
    d = lambda t: t.detach().double().cpu().clone().requires_grad_(True)
    b = brain_arrays(conn, net.cfg.weight_scale, brain.log_gain.detach().cpu(), brain.bias.detach().cpu(),
                     brain.alpha_logit.detach().cpu(), dtype=torch.double)
    for name in ("log_gain", "bias", "alpha_logit"):
        setattr(b, name, getattr(b, name).clone().requires_grad_(True))
    hp = HeadArrays(d(net.encoder.weight), d(net.encoder.bias), net.cfg.input_gain, N_BASE, d(net.policy.weight),
                    d(net.policy.bias), d(net.policy_from.weight), d(net.policy_from.bias), d(net.policy_to.weight),
                    d(net.policy_to.bias), d(net.value.weight), d(net.value.bias), net.move_from.cpu(),
                    net.move_to.cpu(), net.norm.mean.double().cpu(), net.norm.var.double().cpu())
    cone = light_cone(conn.n_neurons, conn.pre.numpy(), conn.post.numpy(), net.in_idx.cpu().numpy(),
                      net.out_idx.cpu().numpy(), net.cfg.steps)
    rl, rw = T.model_grad(hp, b, cone, x.double())
    T.train_loss(rl, rw, pi.double(), legal, wdl).backward()
    _close(logits, rl, 1e-4, "logits")
    want = {"log_gain": b.log_gain.grad, "bias": b.bias.grad, "alpha_logit": b.alpha_logit.grad,
            "encoder": hp.enc_w.grad[:, :N_BASE], "policy": hp.policy_w.grad, "value": hp.value_w.grad}
    for name in got:
        assert float(want[name].abs().max()) > 0, name
        _close(got[name], want[name], 1e-3, name)
