"""Liquid Time-Constant layer with an MI355X-native fused ODE solver (drop-in for ltc.py).

Same public surface as the reference module (ltc.py:109-349):
`TrueLiquidTimeConstant(input_dim, hidden_dim=64, dt=1/30, ode_unfolds=6,
sparsity=0.5, sensory_sparsity=0.5, input_mapping="affine", epsilon=1e-8)`,
`forward(x_seq, h0=None) -> (outputs, (h, h))`, the same parameter and buffer
names (so state_dicts load across), the same RNG consumption order at init (so
a seed builds the same tensors), the eval-mode transform cache, the
`_force_torchscript` switch, the `W_rec` / `fused_euler_step` shims and the
`TemporalLTC` alias.

Dispatch. fp32 tensors on a HIP device go to the fused kernels in
libltc_hip.so. In training mode the whole layer (LayerNorm, affine, softplus
transforms and the ODE loop, and their backward) is one library call each way
(`ltc_cuda.ltc_module_forward`). In eval mode the reference's transform cache
applies (ltc.py:270-288) and the cached boundary tensors go through
`ltc_cuda.ltc_cuda_forward`, as in the reference. If the library is not
loaded, the call raises: on a GPU the fused path is never swapped for another
one behind the caller's back. CPU tensors, non-fp32 tensors and an explicit
`module._force_torchscript = True` use the TorchScript loop below, which is
this module's own CPU implementation of the same equations (the reference
does the same, ltc.py:293-323).
"""

from __future__ import annotations

import logging

import torch
import torch.nn as nn
import torch.nn.functional as F

import ltc_cuda
from ltc_cuda import _HAS_CUDA_KERNELS, ltc_cuda_forward  # noqa: F401  (reference import surface)

logger = logging.getLogger(__name__)


@torch.jit.script
def _ltc_ode_step_jit(
    inputs: torch.Tensor,        # (B, D)
    state: torch.Tensor,         # (B, H)
    w_pos: torch.Tensor,         # (H, H) softplus(w) * sparsity_mask
    w_erev: torch.Tensor,        # (H, H) w_pos * erev
    mu: torch.Tensor,            # (H, H)
    sigma: torch.Tensor,         # (H, H)
    sensory_mu: torch.Tensor,    # (D, H)
    sensory_sigma: torch.Tensor, # (D, H)
    sensory_erev: torch.Tensor,  # (D, H)
    sensory_w_pos: torch.Tensor, # (D, H) softplus(sensory_w) * mask
    cm_t: torch.Tensor,          # (H,)
    gleak_pos: torch.Tensor,     # (H,)
    vleak: torch.Tensor,         # (H,)
    ode_unfolds: int,
    epsilon: float,
) -> torch.Tensor:
    """One time step: sensory conductances, then `ode_unfolds` implicit-Euler updates.

    Reductions run over dim 1: inputs d for the sensory (B, D, H) product and
    presynaptic i for the recurrent (B, H, H) product (ltc.py:42-63).
    """
    gate_s = torch.sigmoid(sensory_sigma * (inputs.unsqueeze(-1) - sensory_mu))
    cond_s = sensory_w_pos * gate_s
    num_sensory = (cond_s * sensory_erev).sum(dim=1)
    den_sensory = cond_s.sum(dim=1)
    v = state
    for _ in range(ode_unfolds):
        gate_r = torch.sigmoid(sigma * (v.unsqueeze(-1) - mu))
        num = (gate_r * w_erev).sum(dim=1) + num_sensory
        den = (w_pos * gate_r).sum(dim=1) + den_sensory
        v = (cm_t * v + gleak_pos * vleak + num) / (cm_t + gleak_pos + den + epsilon)
    return v


@torch.jit.script
def _ltc_forward_loop_jit(
    x_seq: torch.Tensor,         # (B, T, D)
    state: torch.Tensor,         # (B, H)
    w_pos: torch.Tensor,
    w_erev: torch.Tensor,
    mu: torch.Tensor,
    sigma: torch.Tensor,
    sensory_mu: torch.Tensor,
    sensory_sigma: torch.Tensor,
    sensory_erev: torch.Tensor,
    sensory_w_pos: torch.Tensor,
    cm_t: torch.Tensor,
    gleak_pos: torch.Tensor,
    vleak: torch.Tensor,
    ode_unfolds: int,
    epsilon: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Outer loop over T time steps; returns (outputs (B, T, H), final state)."""
    B = x_seq.size(0)
    T = x_seq.size(1)
    H = state.size(1)
    outputs = torch.empty(B, T, H, device=x_seq.device, dtype=x_seq.dtype)
    for t in range(T):
        state = _ltc_ode_step_jit(
            x_seq[:, t, :], state, w_pos, w_erev, mu, sigma,
            sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
            cm_t, gleak_pos, vleak, ode_unfolds, epsilon)
        outputs[:, t, :] = state
    return outputs, state


class TrueLiquidTimeConstant(nn.Module):
    """Liquid Time-Constant network layer (Hasani/Lechner LTC cell, ncps formulation).

    Per-synapse sigmoid-gated conductances with learned mu/sigma, per-synapse
    reversal potentials, leak reversal potential vleak, membrane capacitance
    cm and leak conductance gleak, a sensory synapse pathway from the inputs,
    and `ode_unfolds` implicit-Euler sub-steps per time step. No tanh on the
    state; softplus keeps w, cm, gleak and sensory_w positive.
    """

    def __init__(
        self,
        input_dim: int,
        hidden_dim: int = 64,
        dt: float = 1.0 / 30.0,
        ode_unfolds: int = 6,
        sparsity: float = 0.5,
        sensory_sparsity: float = 0.5,
        input_mapping: str = "affine",
        epsilon: float = 1e-8,
    ):
        super().__init__()
        self.input_dim = input_dim
        self.hidden_dim = hidden_dim
        self.dt = float(dt)
        self.ode_unfolds = int(max(1, ode_unfolds))
        self.sparsity = sparsity
        self.sensory_sparsity = sensory_sparsity
        self.input_mapping = input_mapping
        self.epsilon = epsilon

        H, D = hidden_dim, input_dim
        # The order of RNG draws below is part of the contract: a seed must
        # build the same tensors as the reference (ltc.py:149-172).
        self.w = nn.Parameter(torch.empty(H, H).uniform_(0.001, 1.0))
        self.mu = nn.Parameter(torch.empty(H, H).uniform_(0.3, 0.8))
        self.sigma = nn.Parameter(torch.empty(H, H).uniform_(3.0, 8.0))
        rec_mask, rec_erev = self._create_recurrent_wiring(H, sparsity)
        self.register_buffer("sparsity_mask", rec_mask)
        self.erev = nn.Parameter(rec_erev)

        self.sensory_w = nn.Parameter(torch.empty(D, H).uniform_(0.001, 1.0))
        self.sensory_mu = nn.Parameter(torch.empty(D, H).uniform_(0.3, 0.8))
        self.sensory_sigma = nn.Parameter(torch.empty(D, H).uniform_(3.0, 8.0))
        sens_mask, sens_erev = self._create_sensory_wiring(D, H, sensory_sparsity)
        self.register_buffer("sensory_sparsity_mask", sens_mask)
        self.sensory_erev = nn.Parameter(sens_erev)

        self.gleak = nn.Parameter(torch.empty(H).uniform_(0.001, 1.0))
        self.vleak = nn.Parameter(torch.empty(H).uniform_(-0.2, 0.2))
        self.cm = nn.Parameter(torch.empty(H).uniform_(0.4, 0.6))

        # Input mapping decides which of input_w / input_b are trainable (ltc.py:175-183).
        if input_mapping == "affine":
            self.input_w = nn.Parameter(torch.ones(D))
            self.input_b = nn.Parameter(torch.zeros(D))
        elif input_mapping == "linear":
            self.input_w = nn.Parameter(torch.ones(D))
            self.register_buffer("input_b", torch.zeros(D))
        else:
            self.register_buffer("input_w", torch.ones(D))
            self.register_buffer("input_b", torch.zeros(D))

        self.input_norm = nn.LayerNorm(D)
        # Eval-mode cache of the positivity transforms (ltc.py:188-190).
        self._cached_transforms: dict | None = None

    @staticmethod
    def _wiring(rows: int, hidden_dim: int, sparsity: float):
        """Bernoulli(sparsity) mask with every column non-empty, and +/-1 reversal signs."""
        if sparsity >= 1.0:
            mask = torch.ones(rows, hidden_dim)
        else:
            mask = (torch.rand(rows, hidden_dim) < sparsity).float()
            for col in range(hidden_dim):
                if not mask[:, col].any():
                    pick = torch.randint(0, rows, (1,))
                    mask[pick, col] = 1.0
        sign = torch.where(torch.rand(rows, hidden_dim) < 0.8,
                           torch.ones(rows, hidden_dim), -torch.ones(rows, hidden_dim))
        return mask, sign * mask

    @staticmethod
    def _create_recurrent_wiring(hidden_dim: int, sparsity: float):
        """Recurrent mask (H, H) and reversal potentials, ~80% excitatory (ltc.py:193-211)."""
        return TrueLiquidTimeConstant._wiring(hidden_dim, hidden_dim, sparsity)

    @staticmethod
    def _create_sensory_wiring(input_dim: int, hidden_dim: int, sparsity: float):
        """Sensory mask (D, H) and reversal potentials, ~80% excitatory (ltc.py:214-231)."""
        return TrueLiquidTimeConstant._wiring(input_dim, hidden_dim, sparsity)

    def _transforms(self):
        w_pos = F.softplus(self.w) * self.sparsity_mask
        w_erev = w_pos * self.erev
        cm_t = F.softplus(self.cm) / (self.dt / self.ode_unfolds)
        gleak_pos = F.softplus(self.gleak)
        sensory_w_pos = F.softplus(self.sensory_w) * self.sensory_sparsity_mask
        return w_pos, w_erev, cm_t, gleak_pos, sensory_w_pos

    def forward(
        self,
        x_seq: torch.Tensor,
        h0: tuple[torch.Tensor, torch.Tensor] | None = None,
    ) -> tuple[torch.Tensor, tuple[torch.Tensor, torch.Tensor]]:
        """(B, T, D) inputs -> ((B, T, H) outputs, (h_final, h_final)).

        h0 is an (h, c) pair for LSTM API compatibility; only h is used.
        """
        B, T, D = x_seq.shape
        d = self.__dict__
        force_ts = d.get("_force_torchscript", False)
        on_hip = x_seq.is_cuda and x_seq.dtype == torch.float32 and not force_ts
        if on_hip and d["training"]:
            leaves = self._module_leaves(D)
            if leaves is not None:
                # Whole layer in two library calls: LayerNorm, affine and the
                # positivity transforms run inside the fused kernels. Without h0
                # the library starts from a zero state itself (state None).
                state = None if h0 is None else h0[0]
                if state is not None and state.dtype != x_seq.dtype:
                    state = state.to(x_seq.dtype)
                outputs, state = ltc_cuda.ltc_module_forward(
                    x_seq, state, leaves, d["dt"], d["ode_unfolds"], d["epsilon"],
                    d["_modules"]["input_norm"].__dict__["eps"])
                return outputs, (state, state)

        state = torch.zeros(B, self.hidden_dim, device=x_seq.device, dtype=x_seq.dtype)
        if h0 is not None:
            state = h0[0]
        x_seq = self.input_norm(x_seq)
        if state.dtype != x_seq.dtype:
            state = state.to(x_seq.dtype)
        x_seq = x_seq * self.input_w + self.input_b

        if not self.training and self._cached_transforms is not None:
            c = self._cached_transforms
            w_pos, w_erev, cm_t, gleak_pos, sensory_w_pos = (
                c["w_pos"], c["w_erev"], c["cm_t"], c["gleak_pos"], c["sensory_w_pos"])
        else:
            w_pos, w_erev, cm_t, gleak_pos, sensory_w_pos = self._transforms()
            if not self.training:
                self._cached_transforms = {
                    "w_pos": w_pos, "w_erev": w_erev, "cm_t": cm_t,
                    "gleak_pos": gleak_pos, "sensory_w_pos": sensory_w_pos,
                }

        if on_hip:
            ltc_cuda.require_kernels()
            outputs, state = ltc_cuda.ltc_cuda_forward(
                x_seq, state, w_pos, w_erev, self.mu, self.sigma,
                self.sensory_mu, self.sensory_sigma, self.sensory_erev, sensory_w_pos,
                cm_t, gleak_pos, self.vleak, self.ode_unfolds, self.epsilon)
        else:
            if not getattr(self, "_ts_fallback_warned", False):
                logger.info(
                    "LTC using the TorchScript loop: is_cuda=%s, dtype=%s, force_ts=%s",
                    x_seq.is_cuda, x_seq.dtype, force_ts)
                self._ts_fallback_warned = True
            outputs, state = _ltc_forward_loop_jit(
                x_seq, state, w_pos, w_erev, self.mu, self.sigma,
                self.sensory_mu, self.sensory_sigma, self.sensory_erev, sensory_w_pos,
                cm_t, gleak_pos, self.vleak, self.ode_unfolds, self.epsilon)
        return outputs, (state, state)

    def _module_path_ok(self, D: int) -> bool:
        """Whether the fused module path applies: standard LayerNorm, fp32 leaves, D in range."""
        return self._module_leaves(D) is not None

    def _module_leaves(self, D: int):
        """The 17 leaves of the fused module path in the library's order, or None
        when the path does not apply (a LayerNorm other than nn.LayerNorm over D
        with weight and bias, non-fp32 or host leaves, D out of range). Read
        straight from the registries: nn.Module attribute access costs a
        __getattr__ call per name on this per-step path."""
        d = self.__dict__
        P, Bf = d["_parameters"], d["_buffers"]
        norm = d["_modules"].get("input_norm")
        w = P.get("w")
        if (D > ltc_cuda.MODULE_MAX_D or not isinstance(norm, nn.LayerNorm) or w is None
                or w.dtype != torch.float32 or not w.is_cuda):
            return None
        nd = norm.__dict__
        NP = nd["_parameters"]
        lw, lb = NP.get("weight"), NP.get("bias")
        if lw is None or lb is None or tuple(nd["normalized_shape"]) != (D,):
            return None
        return [w, P["erev"], Bf["sparsity_mask"], P["mu"], P["sigma"],
                P["sensory_w"], P["sensory_erev"], Bf["sensory_sparsity_mask"],
                P["sensory_mu"], P["sensory_sigma"], P["gleak"], P["vleak"], P["cm"],
                P["input_w"] if "input_w" in P else Bf["input_w"],
                P["input_b"] if "input_b" in P else Bf["input_b"], lw, lb]

    def zero_grad(self, set_to_none: bool = True) -> None:
        """nn.Module.zero_grad over the layer's own parameters and its LayerNorm's,
        read straight from their registries: the generic walk over
        named_parameters costs more host time than the rest of a small layer's
        step. Any other module structure takes nn.Module's own walk."""
        d = self.__dict__
        mods = d["_modules"]
        norm = mods.get("input_norm")
        if (len(mods) != 1 or type(norm) is not nn.LayerNorm or norm._modules
                or d.get("_is_replica", False)):
            return super().zero_grad(set_to_none)
        for reg in (d["_parameters"], norm.__dict__["_parameters"]):
            for p in reg.values():
                if p is None or p.grad is None:
                    continue
                if set_to_none:
                    p.grad = None
                else:
                    if p.grad.grad_fn is not None:
                        p.grad.detach_()
                    else:
                        p.grad.requires_grad_(False)
                    p.grad.zero_()

    def train(self, mode: bool = True):
        """Switching to train mode drops the eval-mode transform cache (ltc.py:328-332)."""
        if mode:
            self._cached_transforms = None
        return super().train(mode)

    @property
    def W_rec(self) -> nn.Parameter:
        """Compatibility alias of the recurrent weight parameter (ltc.py:336-339)."""
        return self.w

    def fused_euler_step(self, *args, **kwargs):
        """Removed entry point kept for attribute checks (ltc.py:341-345)."""
        raise NotImplementedError(
            "fused_euler_step is removed. Use _ode_solver(inputs, state) instead."
        )


TemporalLTC = TrueLiquidTimeConstant
