"""Soma, dendrite and adaptation: the three-state neuron and its torch runtimes.

Public surface of the reference's compartmental module
(src/neurosim_gpu/compartmental.py:1-348): ``DendriticDynamics`` (fields,
validation messages, ``from_time_constants``, ``advance``) and the runtimes
``DendriticMatrixRuntime`` and ``DendriticPELSRuntime`` (constructor
arguments, ``step`` signatures, ``precision`` / ``precision_execution``, the
state attributes a checkpoint carries).  Per neuron n and column b, with
retention factors rho per tick:

    d' = rho_d*d + (1-rho_d)*tanh(j + dendritic_drive)
    u  = (1-c)*j + c*d' - k*a
    s' = clamp(alpha*s + (1-alpha)*gain*tanh(u + drive), 0, 1)
    a' = rho_a*a + (1-rho_a)*s'

Zero coupling and zero adaptation strength give the point model back.  These
runtimes are the portable torch paths; ``native_compartmental`` runs the same
tick as gfx950 kernels.  Reduced precisions are emulated here: fp16 runs the
product in binary16 (``_HalfProduct``), fp8 and NVFP4 round the weights and
the source through their formats and multiply in float32 (``ReducedProduct``).
"""

from __future__ import annotations

from dataclasses import dataclass
import math

import torch

from .dynamics import Dynamics
from .precision import Precision, quantize_dequantize, validate_precision
from .runtime import HybridPELSRuntime, MatrixRuntime, PropagationMode, RuntimeStats
from .topology import SparseTopology

_EXECUTION = {
    "fp32": "torch-csr-input-dtype",
    "fp16": "torch-csr-fp16-forward-fp32-backward",
    "fp8": "torch-csr-fp32-with-fp8-e4m3-qdq-emulation",
    "nvfp4": "torch-csr-fp32-with-nvfp4-e2m1-qdq-emulation",
}


def _in_range(value: torch.Tensor, low: float, high: float, *, high_open: bool) -> bool:
    above = value >= high if high_open else value > high
    return not bool(((value < low) | above).any())


@dataclass(frozen=True)
class DendriticDynamics:
    """A signed dendritic compartment and a slow negative-feedback trace per neuron.

    ``dendrite_decay`` and ``adaptation_decay`` are retention factors per tick
    in [0, 1); ``coupling`` in [0, 1] mixes the synaptic current with the
    dendrite; ``adaptation_strength`` >= 0 scales the feedback.
    """

    soma: Dynamics
    dendrite_decay: torch.Tensor
    adaptation_decay: torch.Tensor
    coupling: torch.Tensor
    adaptation_strength: torch.Tensor

    def __post_init__(self) -> None:
        like = self.soma.alpha
        vectors = {"soma.alpha": like, "soma.gain": self.soma.gain,
                   "dendrite_decay": self.dendrite_decay,
                   "adaptation_decay": self.adaptation_decay, "coupling": self.coupling,
                   "adaptation_strength": self.adaptation_strength}
        rules = (
            (lambda v: v.ndim == 1 and v.shape == like.shape, "must have one value per neuron"),
            (lambda v: v.is_floating_point(), "must be floating point"),
            (lambda v: v.device == like.device and v.dtype == like.dtype,
             "must match soma device and dtype"),
            (lambda v: bool(torch.isfinite(v).all()), "must be finite"),
        )
        for name, value in vectors.items():
            for holds, message in rules:
                if not holds(value):
                    raise ValueError(f"{name} {message}")
        for name in ("dendrite_decay", "adaptation_decay"):
            if not _in_range(vectors[name], 0.0, 1.0, high_open=True):
                raise ValueError(f"{name} must be in [0, 1)")
        if not _in_range(self.coupling, 0.0, 1.0, high_open=False):
            raise ValueError("coupling must be in [0, 1]")
        if bool((self.adaptation_strength < 0).any()):
            raise ValueError("adaptation_strength must be non-negative")

    @classmethod
    def from_time_constants(cls, soma: Dynamics, *, dt: float,
                            tau_dendrite: torch.Tensor | float,
                            tau_adaptation: torch.Tensor | float,
                            coupling: torch.Tensor | float = 0.5,
                            adaptation_strength: torch.Tensor | float = 0.2
                            ) -> "DendriticDynamics":
        """Time constants to retention factors, rho = exp(-dt / tau).

        A scalar becomes a stride-0 view over the N neurons."""
        if not (math.isfinite(dt) and dt > 0):
            raise ValueError("dt must be finite and positive")
        like = soma.alpha

        def vector(value, name: str) -> torch.Tensor:
            out = torch.as_tensor(value, dtype=like.dtype, device=like.device)
            out = out.expand_as(like) if out.ndim == 0 else out
            if out.shape != like.shape:
                raise ValueError(f"{name} must be scalar or have one value per neuron")
            return out

        retention = {}
        for name, tau in (("tau_dendrite", tau_dendrite), ("tau_adaptation", tau_adaptation)):
            tau = vector(tau, name)
            if not bool((torch.isfinite(tau) & (tau > 0)).all()):
                raise ValueError(f"{name} must be finite and positive")
            retention[name] = torch.exp(-dt / tau)
        return cls(soma, retention["tau_dendrite"], retention["tau_adaptation"],
                   vector(coupling, "coupling"), vector(adaptation_strength, "adaptation_strength"))

    def advance(self, state: torch.Tensor, dendritic_state: torch.Tensor,
                adaptation_state: torch.Tensor, synaptic_current: torch.Tensor,
                drive: torch.Tensor | float = 0.0, *,
                dendritic_drive: torch.Tensor | float = 0.0
                ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(s', d', a'): a pure, differentiable tick.  The feedback reads a_t;
        the trace then follows s'.  Each line is one tensor op of the model, in
        the order the fused kernel evaluates it (bitwise agreement)."""
        rho_d, rho_a, c, k = (self.dendrite_decay, self.adaptation_decay, self.coupling,
                              self.adaptation_strength)
        dendrite_input = torch.tanh(synaptic_current + dendritic_drive)
        dendrite = rho_d * dendritic_state + (1.0 - rho_d) * dendrite_input
        soma_current = (1.0 - c) * synaptic_current + c * dendrite - k * adaptation_state
        soma = self.soma.advance(state, soma_current, drive)
        adaptation = rho_a * adaptation_state + (1.0 - rho_a) * soma
        return soma, dendrite, adaptation


def _csr(rowptr: torch.Tensor, col: torch.Tensor, values: torch.Tensor, n: int) -> torch.Tensor:
    return torch.sparse_csr_tensor(rowptr, col, values, size=(n, n), check_invariants=False)


class _HalfProduct(torch.autograd.Function):
    """W @ s computed in binary16 (both operands rounded, fp16 sparse product).

    Derivatives are float32 products with the rounded operands: for the
    weights, grad[b, dst] * s16[b, src] summed over b at each stored edge only
    (a sampled dense-dense product); for the source, the transposed graph
    (the topology's source-major view) applied to the incoming gradient.
    """

    @staticmethod
    def forward(ctx, weight, source, half_matrix, topology):
        rounded = source.to(torch.float16)
        ctx.save_for_backward(half_matrix, rounded)
        ctx.topology = topology
        product = torch.sparse.mm(half_matrix, rounded.transpose(0, 1))
        return product.transpose(0, 1).to(torch.float32)

    @staticmethod
    def backward(ctx, grad):
        half_matrix, rounded = ctx.saved_tensors
        topology = ctx.topology
        wants_weight, wants_source = ctx.needs_input_grad[:2]
        d_weight = d_source = None
        with torch.autocast(device_type=grad.device.type, enabled=False):
            source32 = rounded.to(torch.float32)
            if wants_weight:
                sampled = torch.sparse.sampled_addmm(
                    half_matrix.to(torch.float32), grad.transpose(0, 1).contiguous(),
                    source32.contiguous(), beta=0.0)
                d_weight = sampled.values()
            if wants_source:
                by_source = half_matrix.values().to(torch.float32)[topology.out_weight_index]
                transposed = _csr(topology.out_rowptr, topology.dst, by_source,
                                  topology.n_neurons)
                d_source = torch.sparse.mm(transposed, grad.transpose(0, 1)).transpose(0, 1)
        return d_weight, d_source, None, None


class ReducedProduct:
    """W @ s with the weights stored in ``precision`` (fp16, fp8 or nvfp4).

    fp16 runs the product in binary16; fp8 and NVFP4 round the weights and the
    source through the format and multiply in float32, with straight-through
    gradients.  The rounded matrix is kept per topology weight version while
    the weights are not being trained.
    """

    def __init__(self, topology: SparseTopology, precision: Precision) -> None:
        self.topology, self.precision = topology, precision
        self.clear()

    def clear(self) -> None:
        self._version, self._matrix = None, None

    def _rounded_matrix(self, needs_grad: bool, training_weights: bool) -> torch.Tensor:
        topology = self.topology
        reusable = (not training_weights and self._matrix is not None
                    and self._version == topology.weight_version
                    and not (needs_grad and self._matrix.is_inference()))
        if reusable:
            return self._matrix
        weights = topology.in_weight
        values = (weights.detach().to(torch.float16) if self.precision == "fp16"
                  else quantize_dequantize(weights, self.precision))
        matrix = _csr(topology.in_rowptr, topology.in_col, values, topology.n_neurons)
        if not training_weights:
            self._version, self._matrix = topology.weight_version, matrix
        return matrix

    def __call__(self, source: torch.Tensor) -> torch.Tensor:
        grad_mode = torch.is_grad_enabled()
        training_weights = grad_mode and self.topology.in_weight.requires_grad
        needs_grad = grad_mode and (training_weights or source.requires_grad)
        matrix = self._rounded_matrix(needs_grad, training_weights)
        with torch.autocast(device_type=source.device.type, enabled=False):
            if self.precision == "fp16":
                if needs_grad:
                    return _HalfProduct.apply(self.topology.in_weight, source, matrix,
                                              self.topology)
                half = torch.sparse.mm(matrix, source.to(torch.float16).transpose(0, 1))
                return half.transpose(0, 1).to(torch.float32)
            operand = quantize_dequantize(source, self.precision)
            return torch.sparse.mm(matrix, operand.transpose(0, 1)).transpose(0, 1)


def _checked_precision(precision: str, initial_state: torch.Tensor) -> Precision:
    precision = validate_precision(precision)
    if precision != "fp32" and initial_state.dtype != torch.float32:
        raise ValueError("reduced precision requires FP32 master weights and states")
    if precision == "fp16" and not initial_state.is_cuda:
        raise ValueError("FP16 CSR propagation requires CUDA")
    return precision


def _check_compartment_inputs(topology: SparseTopology, dynamics: DendriticDynamics,
                              initial_state: torch.Tensor) -> None:
    if initial_state.ndim != 2 or initial_state.shape[1] != topology.n_neurons:
        raise ValueError("initial_state must have shape [batch, n_neurons]")
    if dynamics.soma.n_neurons != topology.n_neurons:
        raise ValueError("dynamics and topology neuron counts must match")
    for value in (dynamics.soma.alpha, topology.weight):
        if (value.device, value.dtype) != (initial_state.device, initial_state.dtype):
            raise ValueError("state, topology and dynamics must match device and dtype")
    inside = torch.isfinite(initial_state) & (initial_state >= 0) & (initial_state <= 1)
    if not bool(inside.all()):
        raise ValueError("initial_state must be finite and in [0, 1]")


class _Compartments:
    """What the two torch runtimes share: the dendrite and adaptation traces,
    the reduced-precision product and the compartment advance."""

    state: torch.Tensor
    topology: SparseTopology

    def _setup_compartments(self, topology, dynamics, initial_state, precision) -> None:
        self.precision: Precision = _checked_precision(precision, initial_state)
        _check_compartment_inputs(topology, dynamics, initial_state)
        self.compartment_dynamics = dynamics
        self.dendritic_state = torch.zeros_like(initial_state)
        self.adaptation_state = torch.zeros_like(initial_state)
        self._reduced = (ReducedProduct(topology, self.precision)
                         if self.precision != "fp32" else None)

    @property
    def precision_execution(self) -> str:
        return _EXECUTION[self.precision]

    def _invalidate_precision_cache(self) -> None:
        """Drop products derived from the weights (called after a restore)."""
        if getattr(self, "_reduced", None) is not None:
            self._reduced.clear()

    def _propagate(self, source: torch.Tensor) -> torch.Tensor:
        if self._reduced is None:
            return MatrixRuntime._propagate(self, source)
        return self._reduced(source)

    def _drive_error(self, name: str, value) -> str | None:
        if not isinstance(value, torch.Tensor):
            return None
        if self.precision != "fp32" and (value.dtype, value.device) != (self.state.dtype,
                                                                        self.state.device):
            return f"{name} must match state device and dtype"
        try:
            fits = torch.broadcast_shapes(value.shape, self.state.shape) == self.state.shape
        except RuntimeError:
            fits = False
        return None if fits else f"{name} must broadcast to [batch, n_neurons]"

    def _advance_with(self, current: torch.Tensor, drive, dendritic_drive) -> torch.Tensor:
        """New soma state from ``current``; the traces advance with it.  Drives
        are checked first, so a rejected call changes nothing."""
        for name, value in (("drive", drive), ("dendritic_drive", dendritic_drive)):
            message = self._drive_error(name, value)
            if message is not None:
                raise ValueError(message)
        soma, self.dendritic_state, self.adaptation_state = self.compartment_dynamics.advance(
            self.state, self.dendritic_state, self.adaptation_state, current, drive,
            dendritic_drive=dendritic_drive)
        return soma


class DendriticMatrixRuntime(_Compartments, MatrixRuntime):
    """One CSR product and O(B*N) work per tick, with two extra [B,N] states.

    Both traces start at zero; a checkpoint restores all three states.
    """

    def __init__(self, topology: SparseTopology, dynamics: DendriticDynamics,
                 initial_state: torch.Tensor, *, precision: str = "fp32") -> None:
        self._setup_compartments(topology, dynamics, initial_state, precision)
        MatrixRuntime.__init__(self, topology, dynamics.soma, initial_state)
        self._invalidate_precision_cache()

    def step(self, drive: torch.Tensor | float = 0.0, *,
             dendritic_drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        self.state = self._advance_with(self._propagate(self.state), drive, dendritic_drive)
        return self.state


class DendriticPELSRuntime(_Compartments, HybridPELSRuntime):
    """PELS propagation with every neuron's compartments advanced on every tick.

    theta = 0 reproduces DendriticMatrixRuntime; only the soma emits.  With a
    reduced precision the current is recomputed whole from the emitted state
    each tick (matrix propagation only), and an emitter's emitted value becomes
    its new state rather than the old value plus the delta.
    """

    def __init__(self, topology: SparseTopology, dynamics: DendriticDynamics,
                 initial_state: torch.Tensor, *, theta: float | torch.Tensor,
                 propagation: PropagationMode = "auto", event_edge_fraction: float = 0.12,
                 policy_interval: int = 16, precision: str = "fp32") -> None:
        if _checked_precision(precision, initial_state) != "fp32" and propagation != "matrix":
            raise ValueError("reduced-precision PELS requires propagation='matrix'")
        self._setup_compartments(topology, dynamics, initial_state, precision)
        HybridPELSRuntime.__init__(self, topology, dynamics.soma, initial_state, theta=theta,
                                   propagation=propagation,
                                   event_edge_fraction=event_edge_fraction,
                                   policy_interval=policy_interval)
        self._invalidate_precision_cache()

    def step(self, drive: torch.Tensor | float = 0.0, *,
             dendritic_drive: torch.Tensor | float = 0.0, collect_stats: bool = False):
        self._refresh_current()
        next_state = self._advance_with(self.persistent_current, drive, dendritic_drive)
        if self.precision == "fp32":
            return self._commit(next_state, collect_stats=collect_stats)
        return self._commit_recomputed(next_state, collect_stats)

    def _commit_recomputed(self, next_state: torch.Tensor, collect_stats: bool):
        active = (next_state - self.emitted_state).detach().abs() >= self.theta
        self.emitted_state = torch.where(active, next_state, self.emitted_state)
        self.state = next_state
        self.persistent_current = self._propagate(self.emitted_state).contiguous()
        self._tick += 1
        if not collect_stats:
            return self.state
        sources = torch.nonzero(active, as_tuple=True)[1]
        edges = int(self.topology.out_degree[sources].sum().item()) if sources.numel() else 0
        return self.state, RuntimeStats(path="matrix-precision",
                                        active_neurons=int(active.sum().item()),
                                        active_edges=edges)
