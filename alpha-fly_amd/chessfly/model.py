"""Policy/value network whose only hidden computation is the fly connectome, evaluated on gfx950.

    board features --linear--> sensory neurons --`steps` recurrent updates--> output neurons
                   --RunningNorm--> move logits (+ from/to-square terms), WDL logits

Drop-in for chessfly/model.py of the reference (ModelConfig, RunningNorm, FlyChessNet, Evaluator,
load_weights): same constructor, parameters, state_dict keys and forward signature.  In evaluation (eval
mode, autograd off) FlyChessNet.forward runs as one call into libflyeval.so (fly_model_forward): the encoder
GEMM on the matrix cores, the light-cone recurrence (float16 deviation path when `infer_dtype` is float16,
float32 otherwise), and the head GEMMs whose operand loader gathers the output neurons and applies the
eval-mode normaliser in place.  In training it runs the same layers separately, differentiably, with the
recurrence's sparse products on the device (ConnectomeRNN.forward_io under autograd).
"""

from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch
from torch import nn

from . import _hip
from .brain import ConnectomeRNN
from .connectome import Connectome
from .encoding import N_BASE, N_FEATURES, N_MOVES, move_squares

READOUT_SUPERCLASSES = ("descending_neuron",)   # plus every efferent neuron (model.py:23)


@dataclasses.dataclass
class ModelConfig:
    """chessfly/model.py:26-34."""
    steps: int = 4
    min_syn: int = 3
    shuffled: bool = False       # control: degree-preserving rewired connectome
    attack_planes: bool = False  # feed the attack-plane features (columns N_BASE..N_FEATURES)
    input_gain: float = 5.0
    weight_scale: float = 2.0
    bias_init: float = 0.1


class RunningNorm(nn.Module):
    """Per-neuron standardisation with running statistics (chessfly/model.py:37-58).  In eval mode it is
    clamp((r - mean) / sqrt(var + eps), -clip, clip); FlyChessNet.forward applies it inside the head kernel.
    Calling the module directly keeps the reference's behaviour, statistics update in training mode included."""

    def __init__(self, n: int, momentum: float = 0.05, eps: float = 1e-8, clip: float = 8.0):
        super().__init__()
        self.momentum, self.eps, self.clip = momentum, eps, clip
        self.register_buffer("mean", torch.zeros(n))
        self.register_buffer("var", torch.ones(n))
        self.register_buffer("initialised", torch.tensor(False))

    def forward(self, r: torch.Tensor) -> torch.Tensor:
        if self.training and r.shape[0] > 1:
            with torch.no_grad():
                # the first batch's weight 1, then the momentum, chosen on the device: reading the flag on
                # the host would wait for the whole forward and leave the GPU idle while the backward queues
                m = torch.where(self.initialised, self.momentum, 1.0)
                self.mean.lerp_(r.mean(0), m)
                self.var.lerp_(r.var(0), m)
                self.initialised.fill_(True)
        return ((r - self.mean) / (self.var + self.eps).sqrt()).clamp(-self.clip, self.clip)


class FlyChessNet(nn.Module):
    def __init__(self, conn: Connectome, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        # float16 selects the deviation-from-rest path (the only float16 inference the reference trusts,
        # chessfly/model.py:65-72); float32 selects the float32 light cone.
        self.infer_dtype = torch.float16
        # The reference always evaluates through the light cone; False computes every neuron at every step
        # (the same function, pruning off) for measurement.
        self.light_cone_pruning = True
        if cfg.shuffled:
            conn = conn.shuffled()
        self.brain = ConnectomeRNN(conn, bias_init=cfg.bias_init, global_scale=cfg.weight_scale)
        self.register_buffer("in_idx", conn.nodes("afferent"), persistent=False)
        out = torch.cat([conn.nodes("efferent"), conn.nodes_of_superclass(*READOUT_SUPERCLASSES)]).unique()
        self.register_buffer("out_idx", out, persistent=False)
        self.encoder = nn.Linear(N_FEATURES, len(self.in_idx))
        self.norm = RunningNorm(len(out))
        self.policy = nn.Linear(len(out), N_MOVES)
        self.value = nn.Linear(len(out), 3)
        self.policy_from, self.policy_to = nn.Linear(len(out), 64), nn.Linear(len(out), 64)
        frm, to = move_squares()
        self.register_buffer("move_from", torch.as_tensor(frm), persistent=False)
        self.register_buffer("move_to", torch.as_tensor(to), persistent=False)
        self.register_buffer("move_from32", torch.as_tensor(frm.astype(np.int32)), persistent=False)
        self.register_buffer("move_to32", torch.as_tensor(to.astype(np.int32)), persistent=False)
        # (64, N_MOVES) one-hot maps of each move's from and to square: f[:, move_from] as f @ onehot, exact in
        # the forward (one value times 1 plus zeros per output), and in the backward a product instead of the
        # index backward's radix sort of 4,168 repeated indices
        for name, sq in (("move_from_onehot", frm), ("move_to_onehot", to)):
            onehot = torch.zeros(64, len(sq))
            onehot[torch.as_tensor(sq), torch.arange(len(sq))] = 1.0
            self.register_buffer(name, onehot, persistent=False)
        for layer in (self.policy_from, self.policy_to):
            nn.init.zeros_(layer.weight)
            nn.init.zeros_(layer.bias)
        nn.init.zeros_(self.policy.weight)
        nn.init.zeros_(self.value.weight)

    def _dense_tensors(self):
        return (self.encoder.weight, self.encoder.bias, self.norm.mean, self.norm.var, self.policy.weight,
                self.policy.bias, self.policy_from.weight, self.policy_from.bias, self.policy_to.weight,
                self.policy_to.bias, self.value.weight, self.value.bias)

    def _dense(self, k: int) -> _hip.Handle:
        """The encoder and head weights split for the matrix cores, rebuilt when any of them changes."""
        tensors = self._dense_tensors()
        key = (k,) + tuple((t._version, t.data_ptr()) for t in tensors)
        cached = getattr(self, "_dense_cache", None)
        if cached is not None and cached.key == key:
            return cached
        self._dense_cache = None
        for t in tensors:
            _hip.require_device(t, "FlyChessNet.forward")
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise RuntimeError("FlyChessNet.forward: encoder, head and normaliser tensors must be contiguous float32")
        enc_w, enc_b = tensors[0], tensors[1]
        head = _hip.HeadDesc(len(self.out_idx), N_MOVES, self.norm.mean.data_ptr(), self.norm.var.data_ptr(),
                             float(self.norm.eps), float(self.norm.clip), *[t.data_ptr() for t in tensors[4:]],
                             self.move_from32.data_ptr(), self.move_to32.data_ptr())
        handle = ctypes.c_void_p()
        _hip.check(_hip.load().fly_dense_create(ctypes.byref(head), enc_w.data_ptr(), enc_w.stride(0), k,
                                                enc_b.data_ptr(), enc_w.shape[0], _hip.stream(enc_w.device),
                                                ctypes.byref(handle)), "fly_dense_create")
        self._dense_cache = _hip.Handle(handle, "fly_dense_destroy", key)
        return self._dense_cache

    def _forward_layers(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """The forward as separate differentiable layers (chessfly/model.py:95-105): training, or any call
        with autograd enabled.  Under autograd the recurrence is float32 (its sparse products on the device);
        without it, in training mode, the recurrence is the fused device forward_io in infer_dtype and the
        normaliser updates its running statistics."""
        dtype = torch.float32 if torch.is_grad_enabled() else self.infer_dtype
        if x.dtype != torch.float32:
            x = x.float()
        if self.cfg.attack_planes:
            enc = self.encoder(x)
        else:                                   # the attack planes are never seen and their weights get no gradient
            enc = nn.functional.linear(x[:, :N_BASE], self.encoder.weight[:, :N_BASE], self.encoder.bias)
        u_in = (enc * self.cfg.input_gain).to(dtype).T.contiguous()
        r = self.norm(self.brain.forward_io(u_in, self.in_idx, self.out_idx, self.cfg.steps).T.float())
        logits = self.policy(r) + self.policy_from(r) @ self.move_from_onehot + self.policy_to(r) @ self.move_to_onehot
        return logits, self.value(r)

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """x: (B, >= N_BASE) -> policy logits (B, N_MOVES), WDL logits (B, 3), both float32.  Half-precision
        boards (what the search sends) are read as they are: widening them to float32 is exact.  Evaluation
        (eval mode, no autograd) is one fused device call; training goes through the layers."""
        _hip.require_device(x, "FlyChessNet.forward")
        if torch.is_grad_enabled() or self.training:
            return self._forward_layers(x)
        dtype = self.infer_dtype
        if dtype not in (torch.float16, torch.float32):
            raise RuntimeError(f"infer_dtype must be float16 or float32, got {dtype}")
        k = N_FEATURES if self.cfg.attack_planes else N_BASE
        if x.dim() != 2 or x.shape[1] < k:
            raise RuntimeError(f"FlyChessNet.forward: x must be (B, >= {k}), got {tuple(x.shape)}")
        if x.dtype not in (torch.float32, torch.float16):
            x = x.float()
        if x.stride(1) != 1:
            x = x.contiguous()
        brain = self.brain
        brain._check_params("FlyChessNet.forward")
        cone = brain.light_cone(self.in_idx, self.out_idx, self.cfg.steps, prune=self.light_cone_pruning)
        mode = _hip.MODE_DEVIATION_F16 if dtype == torch.float16 else _hip.MODE_F32
        plan = brain._cone_plan(cone, mode)
        dense = self._dense(k)
        batch = x.shape[0]
        logits = torch.empty(batch, N_MOVES, dtype=torch.float32, device=x.device)
        wdl = torch.empty(batch, 3, dtype=torch.float32, device=x.device)
        lib = _hip.load()
        ws = _hip.workspace(lib.fly_model_workspace(plan.handle, dense.handle, batch), x.device)
        ldx = x.stride(0) if batch > 1 else x.shape[1]
        x_f16 = int(x.dtype == torch.float16)
        _hip.check(lib.fly_model_forward(plan.handle, dense.handle, x.data_ptr(), x_f16, ldx, batch,
                                         float(self.cfg.input_gain), logits.data_ptr(), wdl.data_ptr(), ws.data_ptr(),
                                         ws.numel(), _hip.stream(x.device)), "fly_model_forward")
        return logits, wdl

    @staticmethod
    def expected_value(wdl_logits: torch.Tensor) -> torch.Tensor:
        """P(win) - P(loss) under the softmax of the WDL logits (model.py:107-110)."""
        p = wdl_logits.softmax(-1)
        return p[..., 0] - p[..., 2]


def _upload(a: np.ndarray, device) -> torch.Tensor:
    """Host array -> device tensor through pinned memory, so the copy is queued on the stream and `submit`
    returns before it has run.  torch's pinned-block cache keeps the block until the copy has finished."""
    host = torch.empty(a.shape, dtype=torch.from_numpy(a[:0]).dtype, pin_memory=True)
    host.numpy()[...] = a
    return host.to(device, non_blocking=True)


# Workgroups of the answers' download (fly_evaluator_download).  With another batch in flight the copy shares the
# GPU with that batch's forward, and its stores to host memory stall the CUs that issue them: 4 workgroups measured
# best (B = 1120, lazy answers, two batches in flight: 6.846 ms per batch against 6.793 for the bare forward; 16
# workgroups 6.943, the runtime's copy on every CU 7.036).  Alone, the copy only has to be fast: 64 workgroups.
DOWNLOAD_SHARED, DOWNLOAD_ALONE = 4, 64


class _Submitted:
    """A batch in flight: the pinned host buffers the device copies its answers into, and the event
    recorded after the last copy.  The copies run on `down` after the compute stream's work so far, as a
    download kernel of `workgroups` workgroups (fly_evaluator_download)."""

    def __init__(self, device_outputs, compute, down, workgroups: int, on_done=None):
        self._on_done = on_done
        self._down, self.done = down, None
        down.wait_stream(compute)
        self.host = [torch.empty(t.shape, dtype=t.dtype, pin_memory=True) for t in device_outputs]
        lib = _hip.load()
        with torch.cuda.stream(down):
            for h, t in zip(self.host, device_outputs):
                _hip.check(lib.fly_evaluator_download(t.data_ptr(), h.data_ptr(), t.numel() * t.element_size(),
                                                      workgroups, down.cuda_stream), "fly_evaluator_download")
                t.record_stream(down)          # the allocator keeps t until this copy has read it
        self.done = torch.cuda.Event()
        self.done.record(down)

    def _finish(self):
        if self._on_done is not None:
            self._on_done()
            self._on_done = None

    def __del__(self):
        # torch's pinned-block cache does not see the download kernel's writes: a batch dropped unread keeps its
        # host buffers until the kernel is done, so no later batch is handed a block still being written
        try:
            if self.done is not None:
                self.done.synchronize()
            else:                       # a download failed to queue: wait for any that were queued before it
                self._down.synchronize()
        except Exception:
            pass
        self._finish()

    def wait(self):
        self.done.synchronize()
        self._finish()
        policy, values, bad = self.host
        if int(bad[0]):
            raise IndexError("Evaluator: a legal-move index lies outside the (batch, N_MOVES) policy")
        return policy.numpy(), values.numpy()        # views that keep their pinned block alive


class Evaluator:
    """The `evaluate` callable of the search: numpy in, numpy out (chessfly/model.py:113-135).  `submit`
    queues the upload, the forward and the download and returns before the GPU finishes; `result` waits for
    it.  One kernel (fly_evaluator_outputs) computes the expected values and either rounds the whole policy to
    half precision (lazy search) or gathers the legal moves' logits (eager search), so only the requested
    bytes cross back to the host.

    Uploads and downloads run on two copy streams of their own, ordered with the compute stream (the
    device's current stream) by events: with two batches in flight, as the search's workers keep them
    (workers.py:118-167), batch i+1's boards go up and batch i's answers come down while the GPU computes.
    A batch submitted while another is in flight downloads its answers on a few CUs (DOWNLOAD_SHARED), so
    the forward it overlaps keeps the rest of the GPU."""

    def __init__(self, net: FlyChessNet, device):
        self.net, self.device = net, device
        self._up = self._down = None
        self._in_flight = 0          # batches submitted and not yet read

    def _streams(self):
        if self._up is None:
            self._up = torch.cuda.Stream(device=self.device)      # default priority
            self._down = torch.cuda.Stream(device=self.device)
        return self._up, self._down

    @torch.no_grad()
    def submit(self, x, rows, cols):
        self.net.eval()
        x = np.ascontiguousarray(x)
        if x.dtype not in (np.float16, np.float32):
            x = x.astype(np.float32)
        up, down = self._streams()
        compute = torch.cuda.current_stream(self.device)
        r = c = None
        n_legal = 0
        with torch.cuda.stream(up):
            xd = _upload(x, self.device)
            if rows is not None:
                rows = np.ascontiguousarray(rows, dtype=np.int64)
                cols = np.ascontiguousarray(cols, dtype=np.int64)
                if rows.shape != cols.shape or rows.ndim != 1:
                    raise IndexError(f"Evaluator: rows {rows.shape} and cols {cols.shape} must be equal 1-d shapes")
                n_legal = len(rows)
                if n_legal:
                    r, c = _upload(rows, self.device), _upload(cols, self.device)
        compute.wait_stream(up)
        for t in (xd, r, c):
            if t is not None:
                t.record_stream(compute)       # allocated on the upload stream, read on the compute stream
        logits, wdl = self.net(xd)
        batch, n_moves = logits.shape
        device = logits.device
        values = torch.empty(batch, dtype=torch.float32, device=device)
        bad = torch.empty(1, dtype=torch.int32, device=device)
        if rows is None:                      # lazy search: the whole policy vector, half precision
            policy = torch.empty(batch, n_moves, dtype=torch.float16, device=device)
            out16, legal = policy.data_ptr(), None
        else:
            if not n_legal:                   # non-null pointers still select the legal-move form
                r = c = torch.zeros(1, dtype=torch.int64, device=device)
            policy = torch.empty(n_legal, dtype=torch.float32, device=device)
            out16, legal = None, policy.data_ptr()
        _hip.check(_hip.load().fly_evaluator_outputs(logits.data_ptr(), wdl.data_ptr(), batch, n_moves, _hip.ptr(r),
                                                     _hip.ptr(c), n_legal, out16, legal, values.data_ptr(),
                                                     bad.data_ptr(), compute.cuda_stream), "fly_evaluator_outputs")
        shared = self._in_flight > 0        # another batch still computes: keep the download to a few CUs
        self._in_flight += 1
        return _Submitted((policy, values, bad), compute, down, DOWNLOAD_SHARED if shared else DOWNLOAD_ALONE,
                          self._landed)

    def _landed(self):
        self._in_flight -= 1

    @staticmethod
    def result(handle):
        return handle.wait()

    def __call__(self, x, rows, cols):
        return self.result(self.submit(x, rows, cols))


NEW_HEADS = ("policy_from.", "policy_to.")


def load_net(path, data_dir: str = "data", device="cuda", conn: Connectome | None = None) -> FlyChessNet:
    """The network of a checkpoint or snapshot, ready to evaluate (chessfly/model.py:154-161): a dict with
    "config" (ModelConfig fields) and "model" (the state dict), read with torch.load(weights_only=True).  The
    wiring is `conn`, which is required: the reference parses the MaleCNS release from data_dir here, and this
    package has no reader for it (the release is a network download).  `data_dir` stays for the signature."""
    if conn is None:
        raise ValueError("load_net needs the connectome the checkpoint was trained on (conn=...): this package "
                         "does not read the MaleCNS release")
    ck = torch.load(path, map_location="cpu", weights_only=True)
    cfg = ModelConfig(**ck["config"])
    net = FlyChessNet(conn, cfg)
    load_weights(net, ck["model"])
    return net.to(device).eval()


def load_weights(net: FlyChessNet, state: dict) -> None:
    """Load a state dict (chessfly/model.py:141-151): an encoder saved before the attack planes is padded
    with zero columns, and the zero-initialised from/to heads may be missing; nothing else may be."""
    state = dict(state)
    w = state.get("encoder.weight")
    if w is not None and w.shape[1] < net.encoder.weight.shape[1]:
        pad = w.new_zeros(w.shape[0], net.encoder.weight.shape[1] - w.shape[1])
        state["encoder.weight"] = torch.cat([w, pad], dim=1)
    missing, unexpected = net.load_state_dict(state, strict=False)
    bad = [k for k in missing if not k.startswith(NEW_HEADS)] + list(unexpected)
    if bad:
        raise RuntimeError(f"checkpoint does not match the network: {bad}")
