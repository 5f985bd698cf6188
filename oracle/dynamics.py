"""Oracle three-state update (test infrastructure only).

Restates DendriticDynamics.advance (reference compartmental.py:152-183) and
Dynamics.advance_modulated (reference dynamics.py:41-61) with the same torch
CPU tensor ops in the same order, and the parameter construction of
DendriticDynamics.from_time_constants (compartmental.py:110-150).

Pins: closed forms and reference-held traces in tests/test_oracle_dynamics.py
(impulse decay (1-rho_d)*tanh(1)*rho_d**t, test_compartmental.py:73-85;
neutral coupling/strength reproduce the point model exactly, :30-39; the FP64
probe traces of results/compartmental_probe_cpu.json).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Params:
    """Per-neuron vectors in the reference order (native_compartmental.py:20-23)."""

    alpha: torch.Tensor
    gain: torch.Tensor
    dendrite_decay: torch.Tensor
    adaptation_decay: torch.Tensor
    coupling: torch.Tensor
    adaptation_strength: torch.Tensor

    def as_list(self) -> list[torch.Tensor]:
        return [self.alpha, self.gain, self.dendrite_decay, self.adaptation_decay,
                self.coupling, self.adaptation_strength]


def _vector(value, like: torch.Tensor) -> torch.Tensor:
    result = torch.as_tensor(value, dtype=like.dtype, device=like.device)
    if result.ndim == 0:
        result = result.expand_as(like)
    return result


def from_time_constants(alpha, gain, *, dt: float, tau_dendrite, tau_adaptation,
                        coupling=0.5, adaptation_strength=0.2) -> Params:
    """rho = exp(-dt / tau) evaluated as torch does it (compartmental.py:138-142)."""
    alpha = torch.as_tensor(alpha)
    gain = torch.as_tensor(gain)
    rho_d = torch.exp(-dt / _vector(tau_dendrite, alpha))
    rho_a = torch.exp(-dt / _vector(tau_adaptation, alpha))
    return Params(alpha, gain, rho_d, rho_a, _vector(coupling, alpha),
                  _vector(adaptation_strength, alpha))


def advance(p: Params, state, dendrite, adaptation, current, drive=0.0, dendritic_drive=0.0):
    """One update; every line is one tensor op of the reference, same order."""
    new_dendrite = (p.dendrite_decay * dendrite
                    + (1.0 - p.dendrite_decay) * torch.tanh(current + dendritic_drive))
    soma_input = ((1.0 - p.coupling) * current + p.coupling * new_dendrite
                  - p.adaptation_strength * adaptation)
    equilibrium = p.gain * 1.0 * torch.tanh(soma_input + drive + 0.0)
    new_state = torch.clamp(p.alpha * state + (1.0 - p.alpha) * equilibrium, min=0.0, max=1.0)
    new_adaptation = p.adaptation_decay * adaptation + (1.0 - p.adaptation_decay) * new_state
    return new_state, new_dendrite, new_adaptation


def point_advance(alpha, gain, state, current, drive=0.0):
    """The original point-neuron update (dynamics.py:41-61)."""
    equilibrium = gain * 1.0 * torch.tanh(current + drive + 0.0)
    return torch.clamp(alpha * state + (1.0 - alpha) * equilibrium, min=0.0, max=1.0)
