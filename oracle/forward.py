"""Oracle: the reference's forward evaluator on the CPU, restated with torch CPU ops.
TEST INFRASTRUCTURE ONLY (imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline).

It mirrors the reference's CPU code path op for op (sparse CSR matmul, index_add, clamp, torch.lerp), so
it is also the CPU baseline the GPU evaluator is timed beside:

  literal          ConnectomeRNN.forward, no-grad branch            chessfly/brain.py:211-223
                   (literal_step: one update, brain.py:219-220)
  constants        ConnectomeRNN._constants                         chessfly/brain.py:238-252
  cone_f32         ConnectomeRNN.forward_io, float32 CPU branch      chessfly/brain.py:282-329 (295-329)
                   (f32_step: one step of it, brain.py:313-327)
  cone_half        ConnectomeRNN._forward_io_half                   chessfly/brain.py:254-280, with the
                   per-weight-version constants (deviation_constants, brain.py:257-270) and one step
                   (deviation_step, brain.py:273-277 and 53-58) apart, and
                   float16 storage points (s, u, lo/hi/e/a, A_t values, d) and float16 arithmetic of the
                   fused deviation update (brain.py:53-58) emulated on the CPU
  model_forward    FlyChessNet.forward                               chessfly/model.py:95-105
  norm             RunningNorm.forward in eval mode                  chessfly/model.py:51-58
  expected_value   FlyChessNet.expected_value                        chessfly/model.py:107-110

Inputs are plain tensors in `BrainArrays` / `HeadArrays`, never the product's modules.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import torch

from .lightcone import Cone


@dataclasses.dataclass
class BrainArrays:
    n: int
    pre: torch.Tensor          # (E,) int64, (post, pre)-sorted
    post: torch.Tensor         # (E,) int64
    sign: torch.Tensor         # (E,) float32
    w0: torch.Tensor           # (E,) float32: syn / sum_in(post) * global_scale
    log_gain: torch.Tensor     # (E,)
    bias: torch.Tensor         # (N,)
    alpha_logit: torch.Tensor  # (N,)
    h_max: float = 10.0


@dataclasses.dataclass
class HeadArrays:
    enc_w: torch.Tensor        # (n_in, F)
    enc_b: torch.Tensor        # (n_in,)
    input_gain: float
    n_base: int
    policy_w: torch.Tensor     # (M, n_out)
    policy_b: torch.Tensor
    from_w: torch.Tensor       # (64, n_out)
    from_b: torch.Tensor
    to_w: torch.Tensor
    to_b: torch.Tensor
    value_w: torch.Tensor      # (3, n_out)
    value_b: torch.Tensor
    move_from: torch.Tensor    # (M,) int64
    move_to: torch.Tensor
    norm_mean: torch.Tensor    # (n_out,)
    norm_var: torch.Tensor
    norm_eps: float = 1e-8
    norm_clip: float = 8.0


def normalised_weight(n: int, post: torch.Tensor, syn: torch.Tensor) -> torch.Tensor:
    """syn / total input of the postsynaptic neuron, the total clamped below at 1 (connectome.py:70-74)."""
    total = torch.zeros(n, dtype=syn.dtype).index_add_(0, post, syn)
    return syn / total[post].clamp_min(1.0)


def edge_weights(b: BrainArrays, dtype=torch.float32) -> torch.Tensor:
    """sign * w0 * exp(log_gain) (brain.py:201-202)."""
    return (b.sign.to(dtype) * b.w0.to(dtype)) * torch.exp(b.log_gain.to(dtype))


def _crow(rows: torch.Tensor, n: int) -> torch.Tensor:
    crow = torch.zeros(n + 1, dtype=torch.long)
    crow[1:] = torch.bincount(rows, minlength=n).cumsum(0)
    return crow


def full_matrix(b: BrainArrays, w: torch.Tensor) -> torch.Tensor:
    return torch.sparse_csr_tensor(_crow(b.post, b.n), b.pre, w, (b.n, b.n), check_invariants=False)


def _sub(op, w: torch.Tensor) -> torch.Tensor:
    return torch.sparse_csr_tensor(torch.as_tensor(op.crow), torch.as_tensor(op.pre), w[torch.as_tensor(op.edges)],
                                   op.shape, check_invariants=False)


def literal_step(b: BrainArrays, mat: torch.Tensor, alpha: torch.Tensor, h: torch.Tensor,
                 drive: torch.Tensor) -> torch.Tensor:
    """One update of the literal recurrence, h' = lerp(h, clamp(W h + drive, 0, H), alpha), with drive = u + b
    (brain.py:219-220)."""
    x = (mat @ h).add_(drive).clamp_(0, b.h_max)
    return torch.lerp(h, x, alpha)


def literal_operands(b: BrainArrays, dtype):
    """W as a sparse CSR tensor and alpha (N, 1), in dtype, as the literal recurrence uses them (brain.py:215-216):
    computed in the parameters' own dtype, then converted to the state's (float32 parameters widen exactly into a
    float64 recurrence)."""
    pdt = b.alpha_logit.dtype
    alpha = torch.sigmoid(b.alpha_logit).to(dtype).unsqueeze(1)
    return full_matrix(b, edge_weights(b, pdt).to(dtype)), alpha


def literal_f16_operands(b: BrainArrays):
    """The operands of the reference's float16 literal recurrence (brain.py:213-216 with u float16): the weights and
    alpha computed in the parameters' dtype and rounded to float16, widened exactly to float64, so a float64
    recurrence over them is the exact function of what the float16 path computes with."""
    pdt = b.alpha_logit.dtype
    alpha = torch.sigmoid(b.alpha_logit).half().double().unsqueeze(1)
    return full_matrix(b, edge_weights(b, pdt).half().double()), alpha


def literal(b: BrainArrays, u: torch.Tensor, steps: int) -> torch.Tensor:
    """Literal recurrence h <- lerp(h, clamp(W h + b + u, 0, H), alpha) from h = 0; u (N, B)."""
    dtype = u.dtype
    mat, alpha = literal_operands(b, dtype)
    drive = u + b.bias.to(dtype).unsqueeze(1)
    h = torch.zeros_like(drive)
    for _ in range(steps):
        h = literal_step(b, mat, alpha, h, drive)
    return h


def constants(b: BrainArrays, cone: Cone, w: torch.Tensor, alpha: torch.Tensor, dtype):
    """Resting trajectory c_0..c_T (c_0 = 0) and per-step drive
    k_t = (W c_{t-1} + b)[R_t] - A_t c_{t-1}[R_{t-1}] (brain.py:238-252)."""
    mat = full_matrix(b, w)
    bias = b.bias.to(w.dtype).unsqueeze(1)
    c = torch.zeros(b.n, 1, dtype=w.dtype)
    cs, ks = [c], [None]
    for t in range(1, cone.steps + 1):
        s = mat @ c if t > 1 else torch.zeros_like(c)
        rows = torch.as_tensor(cone.rows[t])
        k = (s + bias)[rows]
        op = cone.ops[t]
        if op is not None:
            k = k - _sub(op, w) @ c[torch.as_tensor(cone.rows[t - 1])]
        ks.append(k.to(dtype))
        c = torch.lerp(c, (s + bias).clamp(0, b.h_max), alpha)
        cs.append(c)
    return [x.to(dtype) for x in cs], ks


def prepare_f32(b: BrainArrays, cone: Cone, dtype=torch.float32, weights_dtype=None) -> dict:
    """Everything the float32 light cone caches per weight version (brain.py:295-306): the resting
    trajectory, the per-step drive k_t, the sub-matrices and alpha, in `dtype` (float32 or float64).
    weights_dtype is the parameters' dtype the reference computes the cache in before its .to(dtype)
    (brain.py:299-303): `dtype` by default (the reference's tests on a .double() network), float32 for
    float64 inputs to a float32 network."""
    wdt = weights_dtype or (torch.float64 if dtype == torch.float64 else torch.float32)
    w = edge_weights(b, wdt)
    alpha = torch.sigmoid(b.alpha_logit.to(wdt)).unsqueeze(1)
    cs, ks = constants(b, cone, w, alpha, dtype)
    mats = [None] + [_sub(op, w.to(dtype)) if op is not None else None for op in cone.ops[1:]]
    idx = lambda a: torch.as_tensor(a)
    lists = {name: [None] + [idx(v) for v in getattr(cone, name)[1:]]
             for name in ("u_pos", "u_src", "keep_next", "keep_prev")}
    rows = [idx(r) for r in cone.rows]
    return {"cs": cs, "ks": ks, "mats": mats, "alpha": alpha.to(dtype), "rows": rows, "h_max": b.h_max,
            "out_idx": idx(cone.out_idx), "out_pos": idx(cone.out_pos), "out_src": idx(cone.out_src), **lists}


def f32_step(prep: dict, t: int, h: torch.Tensor | None, u_in: torch.Tensor) -> torch.Tensor:
    """Step t of the float32 light cone (brain.py:313-327, CPU branch): the state of R_t from the state of
    R_{t-1} (None at t = 1) and the input drive u_in (len(in_idx), B)."""
    batch = u_in.shape[1]
    cs, ks, mats, alpha = prep["cs"], prep["ks"], prep["mats"], prep["alpha"]
    rows = prep["rows"][t]
    if mats[t] is None:
        x = ks[t].expand(-1, batch)
    else:
        x = (mats[t] @ h).add_(ks[t])
    x = x.index_add(0, prep["u_pos"][t], u_in[prep["u_src"][t]])
    x = x.clamp(0, prep["h_max"])
    prev = cs[t - 1][rows].expand(-1, batch)
    if len(prep["keep_next"][t]):
        prev = prev.index_copy(0, prep["keep_next"][t], h[prep["keep_prev"][t]])
    return torch.lerp(prev, x, alpha[rows])


def run_f32(prep: dict, steps: int, u_in: torch.Tensor, states: list | None = None) -> torch.Tensor:
    """The per-position part of the float32 light-cone forward_io (brain.py:307-329, CPU branch).  `states`, if
    given, collects h_1..h_T (the state of R_t after each step)."""
    batch = u_in.shape[1]
    cs = prep["cs"]
    h = None
    for t in range(1, steps + 1):
        h = f32_step(prep, t, h, u_in)
        if states is not None:
            states.append(h)
    out = cs[steps][prep["out_idx"]].expand(-1, batch)
    return out.index_copy(0, prep["out_pos"], h[prep["out_src"]])


def cone_f32(b: BrainArrays, cone: Cone, u_in: torch.Tensor, steps: int) -> torch.Tensor:
    """Light-cone forward_io in u_in's dtype (float32 or float64): (len(in_idx), B) -> (len(out_idx), B)."""
    assert steps == cone.steps
    return run_f32(prepare_f32(b, cone, u_in.dtype), steps, u_in)


def _h(x: torch.Tensor) -> torch.Tensor:
    """Round to float16 and back: one float16 storage point or one float16 arithmetic result."""
    return x.to(torch.float16).to(torch.float32)


def deviation_constants(b: BrainArrays, cone: Cone, half: bool = True) -> dict:
    """What the deviation path caches per weight version (brain.py:257-270): from the exact resting trajectory,
    k_full_t = (t > 1 ? W c_{t-1} : 0) + b and c_t = lerp(c_{t-1}, clamp(k_full_t, 0, H), alpha); per step
    lo = -k, hi = H - k, e = k - clamp(k, 0, H), a = alpha[R_t] with k = k_full_t[R_t], the carried flags and A_t;
    and c_T[out_idx].  half=True rounds lo/hi/e/a and A_t's values to float16 (the reference's storage);
    half=False keeps everything float64."""
    dt = torch.float32 if half else torch.float64
    r = _h if half else (lambda v: v)
    w = edge_weights(b, dt)
    alpha = torch.sigmoid(b.alpha_logit.to(dt)).unsqueeze(1)
    mat = full_matrix(b, w)
    bias = b.bias.to(dt).unsqueeze(1)
    c = torch.zeros(b.n, 1, dtype=dt)
    per_step = [None]
    for t in range(1, cone.steps + 1):
        k_full = (mat @ c if t > 1 else torch.zeros_like(c)) + bias
        k = k_full[torch.as_tensor(cone.rows[t])]
        xc = k.clamp(0, b.h_max)
        op = cone.ops[t]
        sub = None
        if op is not None:
            sub = torch.sparse_csr_tensor(torch.as_tensor(op.crow), torch.as_tensor(op.pre),
                                          r(w[torch.as_tensor(op.edges)]), op.shape, check_invariants=False)
        per_step.append((r(-k), r(b.h_max - k), r(k - xc), r(alpha[torch.as_tensor(cone.rows[t])]),
                         torch.as_tensor(cone.carried[t]).unsqueeze(1), sub))
        c = torch.lerp(c, k_full.clamp(0, b.h_max), alpha)
    return {"per_step": per_step, "c_out": c[torch.as_tensor(cone.out_idx)], "half": half, "dtype": dt}


def deviation_step(consts: dict, cone: Cone, t: int, d: torch.Tensor | None, u: torch.Tensor) -> torch.Tensor:
    """Step t of the deviation path (brain.py:273-277 with FUSED_DEVIATION, brain.py:53-58): s = A_t d_{t-1}
    plus the input on input rows, x = clamp(s, lo, hi) + e, p = carried ? d_{t-1} : 0, d_t = p + a (x - p).
    d is the deviation of R_{t-1} (None at t = 1), u the input drive (len(in_idx), B) in the path's storage."""
    r = _h if consts["half"] else (lambda v: v)
    dt = consts["dtype"]
    batch = u.shape[1]
    lo, hi, e, a, carried, sub = consts["per_step"][t]
    s = r(sub @ d) if sub is not None else torch.zeros(len(cone.rows[t]), batch, dtype=dt)
    pos = torch.as_tensor(cone.u_pos[t])
    s = s.clone()
    s[pos] = r(s[pos] + u[torch.as_tensor(cone.u_src[t])])
    x = r(torch.minimum(torch.maximum(s, lo), hi) + e)
    p = torch.where(carried, d[torch.as_tensor(cone.prev_row[t])], torch.zeros_like(s)) if d is not None \
        else torch.zeros_like(s)
    return r(p + r(a * r(x - p)))


def cone_half(b: BrainArrays, cone: Cone, u_in: torch.Tensor, steps: int, half: bool = True,
              states: list | None = None) -> torch.Tensor:
    """Deviation-from-rest forward_io (brain.py:254-280): deviation_constants, then deviation_step for t = 1..T;
    the result is c_T[out_idx] + d_T at out_pos.

    half=True emulates the reference's float16 storage in float32: lo/hi/e/a, the sub-matrix values, s, the
    input and d are rounded to float16, s accumulates in float32, and every operation of the fused update is
    rounded to float16 (c10::Half arithmetic).  half=False runs the same algebra in float64 with no
    rounding, where it must equal the float64 light cone exactly up to summation order.  `states`, if given,
    collects d_1..d_T.
    """
    assert steps == cone.steps
    batch = u_in.shape[1]
    consts = deviation_constants(b, cone, half)
    r = _h if half else (lambda v: v)
    u = r(u_in.to(consts["dtype"]))
    d = None
    for t in range(1, steps + 1):
        d = deviation_step(consts, cone, t, d, u)
        if states is not None:
            states.append(d)
    out = consts["c_out"].expand(-1, batch).clone()
    pos = torch.as_tensor(cone.out_pos)
    out[pos] += d[torch.as_tensor(cone.out_src)]
    return out


def norm(hp: HeadArrays, r: torch.Tensor) -> torch.Tensor:
    """Eval-mode RunningNorm: clamp((r - mean) / sqrt(var + eps), -clip, clip) (model.py:51-58)."""
    return ((r - hp.norm_mean.to(r.dtype)) / (hp.norm_var.to(r.dtype) + hp.norm_eps).sqrt()).clamp(-hp.norm_clip,
                                                                                                  hp.norm_clip)


def encode_input(hp: HeadArrays, x: torch.Tensor, dtype) -> torch.Tensor:
    """u_in = ((x[:, :n_base] W[:, :n_base]^T + b) * input_gain) in `dtype`, transposed to (n_in, B) (model.py:101-102)."""
    wdt = torch.float64 if x.dtype == torch.float64 else torch.float32
    enc = torch.nn.functional.linear(x[:, :hp.n_base].to(wdt), hp.enc_w[:, :hp.n_base].to(wdt), hp.enc_b.to(wdt))
    return (enc * hp.input_gain).to(dtype).T.contiguous()


def heads(hp: HeadArrays, r: torch.Tensor):
    """Policy logits with the from/to-square terms, and WDL logits (model.py:104-105)."""
    f = torch.nn.functional.linear
    dt = r.dtype
    logits = (f(r, hp.policy_w.to(dt), hp.policy_b.to(dt))
              + f(r, hp.from_w.to(dt), hp.from_b.to(dt))[:, hp.move_from]
              + f(r, hp.to_w.to(dt), hp.to_b.to(dt))[:, hp.move_to])
    return logits, f(r, hp.value_w.to(dt), hp.value_b.to(dt))


def model_forward(b: BrainArrays, hp: HeadArrays, cone: Cone, x: torch.Tensor, mode: str = "f32", prep=None):
    """FlyChessNet.forward: mode "f32" is the float32 path, "f16" the deviation path, "f64" everything in
    float64 (for pinning against the brute force).  `prep` (from prepare_f32) skips the per-weight-version
    constants of the float32 path, as the reference caches them."""
    if mode == "f64":
        u_in = encode_input(hp, x.to(torch.float64), torch.float64)
        out = cone_f32(b, cone, u_in, cone.steps)
        return heads(hp, norm(hp, out.T))
    dtype = torch.float16 if mode == "f16" else torch.float32
    u_in = encode_input(hp, x.to(torch.float32), dtype)
    if mode == "f16":
        out = cone_half(b, cone, u_in, cone.steps)
    else:
        out = run_f32(prep if prep is not None else prepare_f32(b, cone, dtype), cone.steps, u_in)
    return heads(hp, norm(hp, out.T.float()))


def expected_value(wdl: torch.Tensor) -> torch.Tensor:
    """P(win) - P(loss) of the softmax over the WDL logits (model.py:107-110)."""
    p = wdl.softmax(-1)
    return p[..., 0] - p[..., 2]


def as_numpy(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()
