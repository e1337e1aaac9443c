"""Torch restatement of the reference LTC path, used as the CPU oracle.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product never imports
this file. It restates, in this build's own code:

  * the module init and its RNG consumption order    ltc.py:149-231
  * the pre-transforms (LayerNorm, affine, softplus)  ltc.py:249-288
  * one implicit-Euler ODE step with U unfolds        ltc.py:19-65
    (as its two halves, sensory_sums and unfolds, which are also the
    reference's per-step entry points, csrc/ltc_kernels.cu:675-777)
  * the outer T loop                                  ltc.py:68-106
  * the return convention (out, (h, h))               ltc.py:326

Every function works in the dtype of its inputs, so the same code runs as the
float32 oracle (the reference computes in float32) and as a float64 check.
`forward_loop_scripted` is the TorchScript-compiled form that `bench.py` times
as the CPU baseline, mirroring the reference's `torch.jit.script` use.

Pinning (what checks this file, all under tests/):
  * golden vectors written by the reference itself (tests/golden/), for init,
    forward outputs and every parameter gradient;
  * closed-form special cases (no synapses -> geometric approach to vleak,
    sigma = 0 -> affine recurrence, fixed point at vleak, H = D = 1 scalar
    brute force, saturation);
  * float64 gradcheck, and the independent analytic backward in ltc_analytic.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "PARAM_KEYS",
    "init_params",
    "transforms",
    "sensory_sums",
    "unfolds",
    "ode_step",
    "forward_loop",
    "forward_loop_scripted",
    "module_forward",
    "boundary_inputs",
]

# Leaf parameters of the reference module, in registration order (ltc.py:150-186).
PARAM_KEYS = (
    "w", "mu", "sigma", "erev",
    "sensory_w", "sensory_mu", "sensory_sigma", "sensory_erev",
    "gleak", "vleak", "cm",
    "input_w", "input_b",
    "input_norm.weight", "input_norm.bias",
)


def _wiring(rows: int, hidden_dim: int, sparsity: float):
    """Mask + reversal potentials, same RNG calls as ltc.py:193-231.

    With sparsity >= 1 no mask RNG is drawn (ltc.py:195-196, 216-217). Every
    column that ends up empty gets one random row switched on, drawn with
    randint over `rows` (ltc.py:200-203, 221-224). erev is +1 with p=0.8 else
    -1, then multiplied by the mask (ltc.py:206-210, 227-230).
    """
    if sparsity >= 1.0:
        mask = torch.ones(rows, hidden_dim)
    else:
        mask = (torch.rand(rows, hidden_dim) < sparsity).float()
        for col in range(hidden_dim):
            if not mask[:, col].any():
                r = torch.randint(0, rows, (1,))
                mask[r, col] = 1.0
    sign = torch.where(torch.rand(rows, hidden_dim) < 0.8,
                       torch.ones(rows, hidden_dim), -torch.ones(rows, hidden_dim))
    return mask, sign * mask


def init_params(input_dim: int, hidden_dim: int, sparsity: float = 0.5,
                sensory_sparsity: float = 0.5, input_mapping: str = "affine") -> dict:
    """State dict of a freshly built reference module (ltc.py:149-186).

    Consumes the global torch RNG in exactly the reference order: w, mu,
    sigma, recurrent wiring, sensory w/mu/sigma, sensory wiring, gleak, vleak,
    cm. input_w/input_b are ones/zeros and LayerNorm weight/bias are
    ones/zeros, which draw nothing.
    """
    H, D = hidden_dim, input_dim
    p = {}
    p["w"] = torch.empty(H, H).uniform_(0.001, 1.0)
    p["mu"] = torch.empty(H, H).uniform_(0.3, 0.8)
    p["sigma"] = torch.empty(H, H).uniform_(3.0, 8.0)
    p["sparsity_mask"], p["erev"] = _wiring(H, H, sparsity)
    p["sensory_w"] = torch.empty(D, H).uniform_(0.001, 1.0)
    p["sensory_mu"] = torch.empty(D, H).uniform_(0.3, 0.8)
    p["sensory_sigma"] = torch.empty(D, H).uniform_(3.0, 8.0)
    p["sensory_sparsity_mask"], p["sensory_erev"] = _wiring(D, H, sensory_sparsity)
    p["gleak"] = torch.empty(H).uniform_(0.001, 1.0)
    p["vleak"] = torch.empty(H).uniform_(-0.2, 0.2)
    p["cm"] = torch.empty(H).uniform_(0.4, 0.6)
    p["input_w"] = torch.ones(D)
    p["input_b"] = torch.zeros(D)
    p["input_norm.weight"] = torch.ones(D)
    p["input_norm.bias"] = torch.zeros(D)
    del input_mapping  # mapping only decides parameter vs buffer, not values
    return p


def transforms(p: dict, dt: float, ode_unfolds: int):
    """Positivity transforms of ltc.py:279-283, returned in that order."""
    w_pos = F.softplus(p["w"]) * p["sparsity_mask"]
    w_erev = w_pos * p["erev"]
    cm_t = F.softplus(p["cm"]) / (dt / ode_unfolds)
    gleak_pos = F.softplus(p["gleak"])
    sensory_w_pos = F.softplus(p["sensory_w"]) * p["sensory_sparsity_mask"]
    return w_pos, w_erev, cm_t, gleak_pos, sensory_w_pos


def sensory_sums(inputs, sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos):
    """One step's sensory numerator and denominator sums (ltc.py:44-48).

    inputs (B, D); the sums reduce over D (dim 1 of the (B, D, H) product).
    Returns (num_s, den_s), each (B, H). The reference's per-step entry point
    ltc_sensory_fwd computes the same pair (csrc/ltc_kernels.cu:675-713).
    """
    s_act = torch.sigmoid(sensory_sigma * (inputs.unsqueeze(-1) - sensory_mu))
    s_wact = sensory_w_pos * s_act
    return (s_wact * sensory_erev).sum(dim=1), s_wact.sum(dim=1)


def unfolds(state, w_pos, w_erev, mu, sigma, num_s, den_s, cm_t, gleak_pos, vleak,
            ode_unfolds: int, epsilon: float):
    """U implicit-Euler unfolds of one step (ltc.py:50-63).

    The recurrent sums reduce over the presynaptic index i (dim 1 of the
    (B, H, H) product). Returns (v after the last unfold, [pre-state of every
    unfold]); the reference's ltc_ode_unfold_fwd returns the same pair
    (csrc/ltc_kernels.cu:716-777).
    """
    v = state
    pre = []
    for _ in range(ode_unfolds):
        pre.append(v)
        act = torch.sigmoid(sigma * (v.unsqueeze(-1) - mu))
        num = (act * w_erev).sum(dim=1) + num_s
        den = (w_pos * act).sum(dim=1) + den_s
        v = (cm_t * v + gleak_pos * vleak + num) / (cm_t + gleak_pos + den + epsilon)
    return v, pre


def ode_step(inputs, state, w_pos, w_erev, mu, sigma,
             sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
             cm_t, gleak_pos, vleak, ode_unfolds: int, epsilon: float):
    """One time step: sensory reduction, then U implicit-Euler unfolds.

    Follows ltc.py:42-65. inputs (B, D), state (B, H).
    """
    num_s, den_s = sensory_sums(inputs, sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos)
    v, _ = unfolds(state, w_pos, w_erev, mu, sigma, num_s, den_s, cm_t, gleak_pos, vleak,
                   ode_unfolds, epsilon)
    return v


def forward_loop(x_seq, state, w_pos, w_erev, mu, sigma,
                 sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                 cm_t, gleak_pos, vleak, ode_unfolds: int, epsilon: float):
    """Outer T loop of ltc.py:90-106; returns (outputs (B,T,H), final state)."""
    outs = []
    for t in range(x_seq.size(1)):
        state = ode_step(x_seq[:, t, :], state, w_pos, w_erev, mu, sigma,
                         sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                         cm_t, gleak_pos, vleak, ode_unfolds, epsilon)
        outs.append(state)
    if not outs:
        return x_seq.new_empty(x_seq.size(0), 0, state.size(1)), state
    return torch.stack(outs, dim=1), state


@torch.jit.script
def _step_ts(inputs: torch.Tensor, state: torch.Tensor, w_pos: torch.Tensor,
             w_erev: torch.Tensor, mu: torch.Tensor, sigma: torch.Tensor,
             sensory_mu: torch.Tensor, sensory_sigma: torch.Tensor,
             sensory_erev: torch.Tensor, sensory_w_pos: torch.Tensor,
             cm_t: torch.Tensor, gleak_pos: torch.Tensor, vleak: torch.Tensor,
             ode_unfolds: int, epsilon: float) -> torch.Tensor:
    s_act = torch.sigmoid(sensory_sigma * (inputs.unsqueeze(-1) - sensory_mu))
    s_wact = sensory_w_pos * s_act
    num_s = (s_wact * sensory_erev).sum(dim=1)
    den_s = s_wact.sum(dim=1)
    v = state
    for _ in range(ode_unfolds):
        act = torch.sigmoid(sigma * (v.unsqueeze(-1) - mu))
        num = (act * w_erev).sum(dim=1) + num_s
        den = (w_pos * act).sum(dim=1) + den_s
        v = (cm_t * v + gleak_pos * vleak + num) / (cm_t + gleak_pos + den + epsilon)
    return v


@torch.jit.script
def forward_loop_scripted(x_seq: torch.Tensor, state: torch.Tensor,
                          w_pos: torch.Tensor, w_erev: torch.Tensor,
                          mu: torch.Tensor, sigma: torch.Tensor,
                          sensory_mu: torch.Tensor, sensory_sigma: torch.Tensor,
                          sensory_erev: torch.Tensor, sensory_w_pos: torch.Tensor,
                          cm_t: torch.Tensor, gleak_pos: torch.Tensor,
                          vleak: torch.Tensor, ode_unfolds: int,
                          epsilon: float) -> tuple[torch.Tensor, torch.Tensor]:
    """TorchScript form of `forward_loop` (the reference's executor, ltc.py:68)."""
    B = x_seq.size(0)
    T = x_seq.size(1)
    H = state.size(1)
    outputs = torch.empty(B, T, H, device=x_seq.device, dtype=x_seq.dtype)
    for t in range(T):
        state = _step_ts(x_seq[:, t, :], state, w_pos, w_erev, mu, sigma,
                         sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                         cm_t, gleak_pos, vleak, ode_unfolds, epsilon)
        outputs[:, t, :] = state
    return outputs, state


def boundary_inputs(p: dict, x_seq, dt: float, ode_unfolds: int):
    """Module pre-transforms up to the dispatch point (ltc.py:259-283).

    Returns the 13 tensors the reference hands to its fused boundary, in the
    boundary's argument order (ltc.py:301-306), with x already normalised.
    """
    D = x_seq.size(-1)
    xn = F.layer_norm(x_seq, (D,), p["input_norm.weight"], p["input_norm.bias"], 1e-5)
    xn = xn * p["input_w"] + p["input_b"]
    w_pos, w_erev, cm_t, gleak_pos, sensory_w_pos = transforms(p, dt, ode_unfolds)
    return (xn, w_pos, w_erev, p["mu"], p["sigma"],
            p["sensory_mu"], p["sensory_sigma"], p["sensory_erev"], sensory_w_pos,
            cm_t, gleak_pos, p["vleak"])


def module_forward(p: dict, x_seq, h0=None, dt: float = 1.0 / 30.0,
                   ode_unfolds: int = 6, epsilon: float = 1e-8, scripted: bool = False):
    """Whole module forward (ltc.py:249-326): returns (outputs, (h, h))."""
    B = x_seq.size(0)
    H = p["w"].size(0)
    state = torch.zeros(B, H, dtype=x_seq.dtype, device=x_seq.device)
    if h0 is not None:
        state = h0[0]
    (xn, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev, s_wpos,
     cm_t, gleak_pos, vleak) = boundary_inputs(p, x_seq, dt, ode_unfolds)
    if state.dtype != xn.dtype:
        state = state.to(xn.dtype)
    loop = forward_loop_scripted if scripted else forward_loop
    out, h = loop(xn, state, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev, s_wpos,
                  cm_t, gleak_pos, vleak, int(ode_unfolds), float(epsilon))
    return out, (h, h)
