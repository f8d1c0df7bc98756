"""Training and evaluation engine (trainer.py:1-394) on the gfx950 step executor.

``VNNTrainer`` keeps the reference's functional surface -- ``train_step``, ``train_epoch``,
``evaluate_packed``, ``evaluate_metric``, their ``*_adaptive`` (per-bbox bucket) and
``*_annealed`` (dynamic temperature / Codd mode) variants, ``train_epochs`` and
``_get_adaptive_fns`` / ``_get_annealed_fns`` -- with MI355X execution underneath:

* When ``apply_fn`` is a ``VonNeumannNetwork``'s ``apply`` and the loss is the default MSE, a
  step is the executor's fixed launch sequence (forward -> MSE -> reverse -> AdamW) over
  persistent HBM buffers.  An epoch (the reference's ``lax.scan``) is recorded once into a
  HIP graph and replayed: the first call for a bucket runs eagerly (loading every kernel, the
  analogue of the XLA compile), later calls replay the graph.
* Any other ``apply_fn`` / ``loss_fn`` runs through torch autograd on the same HIP operators,
  with the AdamW update on the AdamW kernel.

Parameters and optimiser state live in one flat device buffer owned by the trainer; the
``params`` / ``opt_state`` it returns are views of that buffer (the next call on the same
trainer updates them in place -- ``clone()`` what must be kept).  Passing any other tensors
copies them in first.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from typing import Callable, NamedTuple

import numpy as np
import torch

from ._lib import NeurocellError, call, ptr, stream_ptr
from .engine import ParamState, StepPlan, TrainState, inv_tau_f32, port_input_shapes
from .params import VNNParams
from .propagator import cropped_bbox

BIT_WEIGHTS_U8 = (128, 64, 32, 16, 8, 4, 2, 1)


# ------------------------------------------------------------------ schedules (optax.*)

class _Schedule:
    """A learning-rate schedule evaluated on the host; ``horizon`` is the step after which it
    is constant (None when unknown)."""
    horizon: int | None = None

    def __call__(self, count: int) -> float:
        raise NotImplementedError


class constant_schedule(_Schedule):
    def __init__(self, value: float):
        self.value, self.horizon = float(value), 0

    def __call__(self, count):
        return self.value


class linear_schedule(_Schedule):
    """optax.linear_schedule: init -> end over ``transition_steps`` (constant ``init_value``
    when ``transition_steps <= 0``)."""

    def __init__(self, init_value, end_value, transition_steps, transition_begin=0):
        self.i, self.e = float(init_value), float(end_value)
        self.n, self.b = int(transition_steps), int(transition_begin)
        self.horizon = max(0, self.b + self.n)

    def __call__(self, count):
        if self.n <= 0:
            return self.i
        c = min(max(count - self.b, 0), self.n)
        return (self.i - self.e) * (1.0 - c / self.n) + self.e


class cosine_decay_schedule(_Schedule):
    """optax.cosine_decay_schedule: init * ((1-alpha) * (0.5(1+cos(pi c/decay)))^exp + alpha)."""

    def __init__(self, init_value, decay_steps, alpha=0.0, exponent=1.0):
        if not decay_steps > 0:
            raise ValueError("The cosine_decay_schedule requires positive decay_steps!")
        self.i, self.n, self.a, self.p = float(init_value), int(decay_steps), float(alpha), \
            float(exponent)
        self.horizon = self.n

    def __call__(self, count):
        c = min(count, self.n)
        cos = 0.5 * (1.0 + math.cos(math.pi * c / self.n))
        return self.i * ((1.0 - self.a) * cos ** self.p + self.a)


class warmup_cosine_decay_schedule(_Schedule):
    """optax.warmup_cosine_decay_schedule (the reference driver's schedule,
    test_vnn_alu_arithmetic.py:172-178): linear warmup init -> peak over ``warmup_steps``, then
    cosine decay to ``end_value`` at ``decay_steps``."""

    def __init__(self, init_value, peak_value, warmup_steps, decay_steps, end_value=0.0,
                 exponent=1.0):
        alpha = 0.0 if peak_value == 0.0 else end_value / peak_value
        self.warm = linear_schedule(init_value, peak_value, warmup_steps)
        self.cos = cosine_decay_schedule(peak_value, decay_steps - warmup_steps, alpha, exponent)
        self.w = int(warmup_steps)
        self.horizon = int(decay_steps)

    def __call__(self, count):
        return self.warm(count) if count < self.w else self.cos(count - self.w)


# ------------------------------------------------------------------ optimiser (optax.adamw)

class AdamWState(NamedTuple):
    """optax ScaleByAdamState analogue: step count (int32 (1,)) and the two moments."""
    count: torch.Tensor
    mu: VNNParams
    nu: VNNParams


class AdamW:
    """optax.adamw(learning_rate, b1, b2, eps, eps_root=0, weight_decay) on the AdamW kernel:
    u = mhat/(sqrt(vhat)+eps) + weight_decay*p, p -= lr(count)*u."""

    def __init__(self, learning_rate, b1=0.9, b2=0.999, eps=1e-8, eps_root=0.0,
                 weight_decay=1e-4):
        if eps_root != 0.0:
            raise NeurocellError("eps_root != 0 is not implemented by the AdamW kernel")
        self.learning_rate = learning_rate
        self.b1, self.b2, self.eps, self.weight_decay = float(b1), float(b2), float(eps), \
            float(weight_decay)

    def init(self, params: VNNParams) -> AdamWState:
        z = lambda t: torch.zeros_like(t, dtype=torch.float32)
        dev = params.cell_params.device
        return AdamWState(torch.zeros(1, dtype=torch.int32, device=dev),
                          VNNParams(z(params.cell_params), z(params.greens_filters)),
                          VNNParams(z(params.cell_params), z(params.greens_filters)))

    def lr_table(self, n: int) -> np.ndarray:
        """The schedule at steps 0..n-1 (fp32)."""
        lr = self.learning_rate
        if not callable(lr):
            return np.array([lr], np.float32)
        return np.array([lr(k) for k in range(int(n))], np.float32)


def adamw(learning_rate, b1=0.9, b2=0.999, eps=1e-8, eps_root=0.0, weight_decay=1e-4) -> AdamW:
    return AdamW(learning_rate, b1, b2, eps, eps_root, weight_decay)


# ------------------------------------------------------------------ reference helpers

def compute_annealed_temperature(epoch: int, total_epochs: int, init_temp: float = 1.0,
                                 final_temp: float = 0.1, schedule: str = "exponential") -> float:
    """trainer.py:23-46."""
    if total_epochs <= 1:
        return float(final_temp)
    progress = min(1.0, max(0.0, float(epoch) / float(total_epochs - 1)))
    if schedule == "exponential":
        return float(init_temp * ((final_temp / init_temp) ** progress))
    if schedule == "cosine":
        cosine_decay = 0.5 * (1.0 + math.cos(math.pi * progress))
        return float(final_temp + (init_temp - final_temp) * cosine_decay)
    if schedule == "linear":
        return float(init_temp + (final_temp - init_temp) * progress)
    raise ValueError(f"Unsupported temperature schedule '{schedule}'; choose from "
                     "('exponential', 'cosine', 'linear').")


def packbits_u8_on_device(bits_u8: torch.Tensor) -> torch.Tensor:
    """trainer.py:49-54: (..., 8) uint8 -> (..., 1) uint8, MSB first, modulo 256."""
    w = torch.tensor(BIT_WEIGHTS_U8, dtype=torch.int32, device=bits_u8.device)
    return ((bits_u8.to(torch.int32) * w).sum(-1) & 0xFF).to(torch.uint8)[..., None]


def _squeeze_like(logits, targets):
    if logits.ndim == 3 and logits.shape[-1] == 1 and targets.ndim == 2:
        return logits.squeeze(-1)
    return logits


def default_mse_loss(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """trainer.py:57-61."""
    logits = _squeeze_like(logits, targets)
    return ((logits - targets) ** 2).mean()


def default_exact_match_metric(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """trainer.py:64-69 (round half to even, as jnp.round)."""
    logits = _squeeze_like(logits, targets)
    return (torch.round(logits) == torch.round(targets)).float().mean()


# ------------------------------------------------------------------ graph replay

class _Replay:
    """Runs ``fn`` eagerly on first use, then records it into a HIP graph that every later use
    replays (the eager run loads each kernel before capture and is a real step)."""

    def __init__(self, fn, use_graph: bool):
        self.fn, self.use_graph = fn, use_graph
        self.graph, self.warm = None, False

    def __call__(self):
        if self.graph is not None:
            self.graph.replay()
            return
        if not self.use_graph or not self.warm:
            self.fn()
            self.warm = True
            return
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.fn()
        self.graph = g
        g.replay()


class _LRU(OrderedDict):
    def __init__(self, cap):
        super().__init__()
        self.cap = cap

    def get_or(self, key, make):
        if key in self:
            self.move_to_end(key)
            return self[key]
        v = self[key] = make()
        while len(self) > self.cap:
            self.popitem(last=False)
        return v


def _is_vnn_apply(fn):
    from .model import VonNeumannNetwork
    owner = getattr(fn, "__self__", None)
    func = getattr(fn, "__func__", None)
    return (isinstance(owner, VonNeumannNetwork)
            and func in (VonNeumannNetwork.apply, VonNeumannNetwork.__call__)), owner


def _flat_batches(x: torch.Tensor, nb: int, B: int) -> torch.Tensor:
    """(nb, B, ...) stacked port inputs -> (nb, B, n_in): ports are concatenated in order,
    which for one stacked array is its row-major flattening."""
    if x.dtype != torch.float32 or not x.is_cuda:
        raise NeurocellError("batches must be float32 device tensors")
    return x.reshape(nb, B, -1).contiguous()


class VNNTrainer:
    """trainer.py:72-394."""

    def __init__(self, apply_fn: Callable, optimizer: AdamW, batch_size: int = 128,
                 loss_fn: Callable | None = None, eval_metric_fn: Callable | None = None,
                 use_graphs: bool = True, max_cached_graphs: int = 8):
        if not isinstance(optimizer, AdamW):
            raise NeurocellError("optimizer must be neurocell.trainer.adamw(...)")
        self.apply_fn = apply_fn
        self.optimizer = optimizer
        self.batch_size = int(batch_size)
        self.custom_loss_fn = loss_fn or default_mse_loss
        self.eval_metric_fn = eval_metric_fn or default_exact_match_metric
        fused, owner = _is_vnn_apply(apply_fn)
        self.model = owner if fused else None
        self.fused = fused and loss_fn is None
        self.use_graphs = bool(use_graphs)
        self._ps: ParamState | None = None
        self._host_count = 0
        self._plans = {}
        self._trainers = {}
        self._runs = _LRU(max_cached_graphs)

        self.train_step = self._bind_step(None, None)
        self.train_epoch = self._bind_epoch(None, None)
        self.evaluate_packed = self._bind_eval_packed(None)
        self.evaluate_metric = self._bind_eval_metric(None)
        self._adaptive_cache = {}
        self._annealed_cache = {}

    # -------------------------------------------------------------- state plumbing
    def _sync(self, params: VNNParams, opt_state: AdamWState) -> ParamState:
        """Makes the trainer's flat buffer hold ``params`` / ``opt_state``."""
        ps = self._ps
        cell, filt = params.cell_params, params.greens_filters
        if ps is None or ps.cell.shape != cell.shape or ps.filt.shape != filt.shape:
            o = self.optimizer
            ps = self._ps = ParamState(cell.detach(), filt.detach(), learning_rate=0.0,
                                       b1=o.b1, b2=o.b2, eps=o.eps, weight_decay=o.weight_decay)
            self._runs.clear()
            self._trainers.clear()
            self._lr_n = 0
            fresh = True
        else:
            fresh = False
        same = lambda a, b: a.data_ptr() == b.data_ptr()
        if not fresh and not (same(cell, ps.cell) and same(filt, ps.filt)):
            ps.cell.copy_(cell.detach())
            ps.filt.copy_(filt.detach())
        mine = (same(opt_state.count, ps.count) and same(opt_state.mu.cell_params, ps.m)
                and same(opt_state.nu.cell_params, ps.v))
        if not mine:
            nc = ps.cell.numel()
            ps.m[:nc].copy_(opt_state.mu.cell_params.reshape(-1))
            ps.m[nc:].copy_(opt_state.mu.greens_filters.reshape(-1))
            ps.v[:nc].copy_(opt_state.nu.cell_params.reshape(-1))
            ps.v[nc:].copy_(opt_state.nu.greens_filters.reshape(-1))
            ps.count.copy_(opt_state.count.reshape(-1).to(torch.int32))
            self._host_count = int(ps.count.item())
        return ps

    def _ensure_lr(self, steps_ahead: int) -> None:
        """The device learning-rate table covers every step up to host_count + steps_ahead;
        a new table invalidates the recorded graphs (they hold its address)."""
        lr = self.optimizer.learning_rate
        if not callable(lr):
            if self._lr_n == 0:
                self._ps.set_learning_rate(float(lr))
                self._lr_n = 1
            return
        need = self._host_count + steps_ahead
        horizon = getattr(lr, "horizon", None)
        if horizon is not None:
            need = min(need, horizon + 1)
        if need <= self._lr_n and self._lr_n > 0:
            return
        n = max(need, 2 * self._lr_n, 1)
        if horizon is not None:
            n = min(n, horizon + 1)
        self._ps.set_learning_rate(torch.from_numpy(self.optimizer.lr_table(n)))
        self._lr_n = n
        self._runs.clear()

    def _outputs(self, ps: ParamState):
        nc = ps.cell.numel()
        m = VNNParams(ps.m[:nc].view(ps.cell.shape), ps.m[nc:].view(ps.filt.shape))
        v = VNNParams(ps.v[:nc].view(ps.cell.shape), ps.v[nc:].view(ps.filt.shape))
        return VNNParams(ps.cell, ps.filt), AdamWState(ps.count, m, v)

    # -------------------------------------------------------------- fused executor
    def _codd(self, codd_mode, temperature):
        m = self.model
        mode, tau, thr = m._resolve(codd_mode, temperature, None)
        return mode, inv_tau_f32(float(tau)), float(thr)

    def _plan(self, B, bbox, training, port_shapes, device):
        m = self.model
        key = (B, bbox, training, tuple(port_shapes), str(device))
        p = self._plans.get(key)
        if p is None:
            p = self._plans[key] = StepPlan(m.topology, B, port_shapes, roi_bbox=bbox,
                                            activate=m.activate,
                                            final_activate=m.final_activate,
                                            hard_pin_io=m.hard_pin_io, training=training,
                                            device=device, gated_filters=m.gated_filters,
                                            sharpen=m.sharpen_filter)
        return p

    def _check_model(self):
        m = self.model
        if not m.norm:
            raise NeurocellError("norm=False is not part of the MI355X path")

    def _fused_train(self, params, opt_state, xb, yb, bbox, codd, nb):
        """nb optimiser steps over (nb, B, ...) batches; returns per-step losses (nb,)."""
        self._check_model()
        B = xb.shape[1]
        ps = self._sync(params, opt_state)
        self._ensure_lr(nb)
        shapes = port_input_shapes(xb[0], self.model.topology)
        plan = self._plan(B, bbox, True, shapes, ps.cell.device)
        x = _flat_batches(xb, nb, B)
        if x.shape[2] != plan.n_in:
            raise NeurocellError(f"batches carry {x.shape[2]} inputs per sample, the ports "
                                 f"take {plan.n_in}")
        if yb.numel() != nb * B * plan.P:
            raise NeurocellError("targets do not match the output port")
        y = yb.reshape(nb, B, plan.P).to(torch.float32).contiguous()
        tkey = (B, bbox, tuple(shapes))
        ts = self._trainers.get(tkey)
        if ts is None:
            ts = self._trainers[tkey] = TrainState(plan, ps)
        if nb == 1:  # single steps go through the static batch buffers: one graph per bucket
            ts.x.copy_(x[0])
            ts.y.copy_(y[0])
            x, y = ts.x[None], ts.y[None]
        mode, it, thr = codd
        key = ("train", tkey, codd, x.data_ptr(), y.data_ptr(), nb, ps.lr.data_ptr())

        def make():
            losses = torch.empty(nb, device=x.device, dtype=torch.float32)

            def fn():
                ts.codd = (mode, it, thr)
                for i in range(nb):
                    ts.launch(x[i], y[i], losses[i:i + 1])
            return _Replay(fn, self.use_graphs), losses, x, y  # x, y kept alive with the graph
        run, losses, _, _ = self._runs.get_or(key, make)
        run()
        self._host_count += nb
        return losses

    def _generic_train(self, params, opt_state, xb, yb, kw, nb):
        ps = self._sync(params, opt_state)
        self._ensure_lr(nb)
        losses = torch.empty(nb, device=ps.cell.device, dtype=torch.float32)
        for i in range(nb):
            cell = ps.cell.detach().requires_grad_(True)
            filt = ps.filt.detach().requires_grad_(True)
            logits = self.apply_fn(VNNParams(cell, filt), xb[i], **kw)
            loss = self.custom_loss_fn(logits, yb[i])
            g_cell, g_filt = torch.autograd.grad(loss, (cell, filt), allow_unused=True)
            ps.g_cell.copy_(g_cell if g_cell is not None else torch.zeros_like(ps.g_cell))
            ps.g_filt.copy_(g_filt if g_filt is not None else torch.zeros_like(ps.g_filt))
            ps.adamw()
            losses[i] = loss.detach()
            self._host_count += 1
        return losses

    def _train(self, params, opt_state, xb, yb, mask_spec, codd_mode, temperature, nb,
               annealed):
        bbox = cropped_bbox(mask_spec, self.model.topology) if self.fused else None
        if self.fused:
            codd = self._codd(codd_mode, temperature)
            losses = self._fused_train(params, opt_state, xb, yb, bbox, codd, nb)
        else:
            kw = {}
            if mask_spec is not None and not mask_spec.is_full_roi or annealed:
                kw["spatial_mask"] = mask_spec
            if annealed:
                kw.update(codd_mode=codd_mode, state_temperature=temperature)
            losses = self._generic_train(params, opt_state, xb, yb, kw, nb)
        new_params, new_state = self._outputs(self._ps)
        return new_params, new_state, losses

    # -------------------------------------------------------------- evaluation
    def _forward_batches(self, params, xb, mask_spec, per_batch):
        """Runs the forward over (nb, B, ...) batches and hands each batch's logits
        (B, out_h, out_w) to ``per_batch(i, logits)`` (launched on the current stream; the
        executor reuses the buffer for the next batch)."""
        nb, B = xb.shape[0], xb.shape[1]
        if self.fused:
            self._check_model()
            bbox = cropped_bbox(mask_spec, self.model.topology)
            shapes = port_input_shapes(xb[0], self.model.topology)
            plan = self._plan(B, bbox, False, shapes, params.cell_params.device)
            x = _flat_batches(xb, nb, B)
            if x.shape[2] != plan.n_in:
                raise NeurocellError(f"batches carry {x.shape[2]} inputs per sample, the "
                                     f"ports take {plan.n_in}")
            mode, it, thr = self._codd(None, None)
            cell = params.cell_params.detach().contiguous()
            filt = params.greens_filters.detach().contiguous()
            oh, ow = self.model.topology.out_port.size
            for i in range(nb):
                plan.forward(cell, filt, x[i], codd_mode=mode, inv_tau=it, active_threshold=thr)
                per_batch(i, plan.out.view(B, oh, ow))
            return
        kw = {} if mask_spec is None or mask_spec.is_full_roi else {"spatial_mask": mask_spec}
        with torch.no_grad():
            for i in range(nb):
                per_batch(i, self.apply_fn(params, xb[i], **kw))

    def _eval_packed(self, params, x_batches, y_packed_batches, mask_spec):
        nb, B = x_batches.shape[0], x_batches.shape[1]
        dev = params.cell_params.device
        y = y_packed_batches.reshape(nb, B).to(device=dev, dtype=torch.uint8).contiguous()
        preds = torch.empty(nb, B, device=dev, dtype=torch.uint8)
        acc = torch.zeros(1, device=dev, dtype=torch.float32)

        def per_batch(i, logits):
            out = logits.reshape(B, -1).contiguous()
            if out.shape[1] != 8:
                raise NeurocellError("evaluate_packed needs 8 output-port cells per sample")
            call("nc_packed_accuracy", stream_ptr(), B, 8, ptr(out), ptr(y[i]), ptr(preds[i]),
                 ptr(acc))
        self._forward_batches(params, x_batches, mask_spec, per_batch)
        return (acc / float(nb))[0], preds[..., None]

    def _eval_metric(self, params, x_batches, y_batches, mask_spec):
        nb, B = x_batches.shape[0], x_batches.shape[1]
        total = torch.zeros((), device=params.cell_params.device, dtype=torch.float32)

        def per_batch(i, logits):
            nonlocal total
            total = total + self.eval_metric_fn(logits.clone(), y_batches[i])
        self._forward_batches(params, x_batches, mask_spec, per_batch)
        return total / float(nb)

    # -------------------------------------------------------------- bound entry points
    def _bind_step(self, mask_spec, annealed_mode):
        def step(params, opt_state, batch_x, batch_y, *temp):
            tau = temp[0] if temp else None
            p, s, losses = self._train(params, opt_state, batch_x[None], batch_y[None],
                                       mask_spec, annealed_mode, tau, 1, annealed_mode is not None)
            return p, s, losses[0]
        return step

    def _bind_epoch(self, mask_spec, annealed_mode):
        def epoch(params, opt_state, x_epoch, y_epoch, *temp):
            tau = temp[0] if temp else None
            nb = x_epoch.shape[0]
            p, s, losses = self._train(params, opt_state, x_epoch, y_epoch, mask_spec,
                                       annealed_mode, tau, nb, annealed_mode is not None)
            return p, s, losses.sum() / float(self.batch_size)
        return epoch

    def _bind_eval_packed(self, mask_spec):
        return lambda params, xb, yb: self._eval_packed(params, xb, yb, mask_spec)

    def _bind_eval_metric(self, mask_spec):
        return lambda params, xb, yb: self._eval_metric(params, xb, yb, mask_spec)

    def _get_adaptive_fns(self, mask_spec):
        """trainer.py:164-248: (train_step, train_epoch, evaluate_packed, evaluate_metric)
        for the mask's bucket, cached by (roi_bbox, is_full_roi)."""
        if mask_spec is None or mask_spec.is_full_roi:
            return self.train_step, self.train_epoch, self.evaluate_packed, self.evaluate_metric
        key = (tuple(mask_spec.roi_bbox), mask_spec.is_full_roi)
        fns = self._adaptive_cache.get(key)
        if fns is None:
            fns = self._adaptive_cache[key] = (
                self._bind_step(mask_spec, None), self._bind_epoch(mask_spec, None),
                self._bind_eval_packed(mask_spec), self._bind_eval_metric(mask_spec))
        return fns

    def train_step_adaptive(self, params, opt_state, batch_x, batch_y, mask_spec):
        return self._get_adaptive_fns(mask_spec)[0](params, opt_state, batch_x, batch_y)

    def train_epoch_adaptive(self, params, opt_state, x_epoch, y_epoch, mask_spec):
        return self._get_adaptive_fns(mask_spec)[1](params, opt_state, x_epoch, y_epoch)

    def evaluate_packed_adaptive(self, params, x_batches, y_packed_batches, mask_spec):
        return self._get_adaptive_fns(mask_spec)[2](params, x_batches, y_packed_batches)

    def evaluate_metric_adaptive(self, params, x_batches, y_batches, mask_spec):
        return self._get_adaptive_fns(mask_spec)[3](params, x_batches, y_batches)

    def _get_annealed_fns(self, codd_mode: str = "annealed", mask_spec=None):
        """trainer.py:260-314: (train_step_ann, train_epoch_ann) taking the temperature as
        their last argument, cached by (codd_mode, bbox)."""
        bbox_key = None if (mask_spec is None or mask_spec.is_full_roi) else \
            (tuple(mask_spec.roi_bbox), mask_spec.is_full_roi)
        key = (codd_mode, bbox_key)
        fns = self._annealed_cache.get(key)
        if fns is None:
            fns = self._annealed_cache[key] = (self._bind_step(mask_spec, codd_mode),
                                               self._bind_epoch(mask_spec, codd_mode))
        return fns

    def train_step_annealed(self, params, opt_state, batch_x, batch_y,
                            state_temperature=1.0, codd_mode: str = "annealed",
                            mask_spec=None):
        step_fn, _ = self._get_annealed_fns(codd_mode=codd_mode, mask_spec=mask_spec)
        return step_fn(params, opt_state, batch_x, batch_y, float(state_temperature))

    def train_epoch_annealed(self, params, opt_state, x_epoch, y_epoch,
                             state_temperature=1.0, codd_mode: str = "annealed",
                             mask_spec=None):
        _, epoch_fn = self._get_annealed_fns(codd_mode=codd_mode, mask_spec=mask_spec)
        return epoch_fn(params, opt_state, x_epoch, y_epoch, float(state_temperature))

    def train_epochs(self, params, opt_state, x_train, y_train, rng, num_epochs: int):
        """trainer.py:358-394: ``num_epochs`` epochs with an on-device shuffle per epoch
        (torch.randperm from ``rng``, an int seed or a device torch.Generator; the permutation
        stream is not JAX's).  Returns (params, opt_state, epoch_losses (num_epochs,))."""
        n = x_train.shape[0]
        steps = n // self.batch_size
        usable = steps * self.batch_size
        dev = x_train.device
        gen = rng if isinstance(rng, torch.Generator) else \
            torch.Generator(device=dev).manual_seed(int(rng))
        x_ep = torch.empty((steps, self.batch_size) + tuple(x_train.shape[1:]), device=dev,
                           dtype=x_train.dtype)
        y_ep = torch.empty((steps, self.batch_size) + tuple(y_train.shape[1:]), device=dev,
                           dtype=y_train.dtype)
        out = torch.empty(int(num_epochs), device=dev, dtype=torch.float32)
        for e in range(int(num_epochs)):
            perm = torch.randperm(n, generator=gen, device=dev)[:usable]
            torch.index_select(x_train, 0, perm, out=x_ep.view((usable,) + x_ep.shape[2:]))
            torch.index_select(y_train, 0, perm, out=y_ep.view((usable,) + y_ep.shape[2:]))
            params, opt_state, loss = self.train_epoch(params, opt_state, x_ep, y_ep)
            out[e] = loss
        return params, opt_state, out
