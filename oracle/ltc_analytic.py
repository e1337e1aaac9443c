"""Float64 numpy restatement of the LTC boundary forward and its closed-form backward.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

This is a second, independent derivation of the gradients at the fused
boundary: it does not use autograd. The reference computes the same
quantities in its native backward (csrc/ltc_kernels.cu:627-667 for the
recurrent unfold, :323-338 for the sensory synapses). Tests check it against
torch.autograd through `ltc_oracle.forward_loop` in float64, so a dropped
term, a wrong sign or a transposed index in either derivation shows up.

Conventions (ltc.py:42-63): recurrent matrices are indexed [i, j] with i the
presynaptic neuron (the reduction axis) and j the postsynaptic neuron;
sensory matrices are [d, h] with the reduction over d.
"""

from __future__ import annotations

import numpy as np

__all__ = ["forward", "backward"]


def _sig(z):
    # Two-branch form keeps exp() from overflowing for large |z|.
    out = np.empty_like(z)
    pos = z >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-z[pos]))
    ez = np.exp(z[~pos])
    out[~pos] = ez / (1.0 + ez)
    return out


def forward(x, h0, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev, s_wpos,
            cm_t, gleak, vleak, U, eps):
    """Boundary forward (ltc.py:42-106) in float64.

    Returns (out (B,T,H), h (B,H), tape) where the tape holds the unfold
    pre-states v[t][k] (B,H), the denominators den[t][k] (B,H) and the
    post-states needed by `backward`.
    """
    x = np.asarray(x, np.float64)
    B, T, D = x.shape
    H = h0.shape[1]
    v = np.array(h0, np.float64)
    out = np.zeros((B, T, H))
    tape = {"v": [], "den": []}
    for t in range(T):
        sa = _sig(s_sigma[None] * (x[:, t, :, None] - s_mu[None]))          # (B,D,H)
        num_s = (s_wpos[None] * sa * s_erev[None]).sum(1)
        den_s = (s_wpos[None] * sa).sum(1)
        vs, ds = [], []
        for _ in range(U):
            a = _sig(sigma[None] * (v[:, :, None] - mu[None]))              # (B,H,H)
            num = (a * w_erev[None]).sum(1) + num_s
            den = cm_t + gleak + (a * w_pos[None]).sum(1) + den_s + eps
            vs.append(v)
            ds.append(den)
            v = (cm_t * v + gleak * vleak + num) / den
        tape["v"].append(vs)
        tape["den"].append(ds)
        out[:, t] = v
    return out, v, tape


def backward(x, h0, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev, s_wpos,
             cm_t, gleak, vleak, U, eps, g_out, g_h=None):
    """Closed-form gradients of the boundary, in Function-input order.

    Returns a dict with keys x, state, w_pos, w_erev, mu, sigma, sensory_mu,
    sensory_sigma, sensory_erev, sensory_w_pos, cm_t, gleak_pos, vleak
    (ltc_cuda.py:342-355).

    Per unfold with incoming g = dL/dv^{k+1} (csrc/ltc_kernels.cu:627-667):
      alpha = g/den, beta = -g*v^{k+1}/den
      dC += alpha*(v^k - v^{k+1}), dG += alpha*(L - v^{k+1}), dL += alpha*G,
      dv^k_j += alpha_j*C_j  (direct path)
      delta_ij = (alpha_j*WE_ij + beta_j*WP_ij) * a_ij*(1-a_ij)
      dWE += alpha_j*a, dWP += beta_j*a, dM -= delta*S, dS += delta*(v_i-M),
      dv^k_i += sum_j delta_ij*S_ij
    Sensory, with A = sum_k alpha and Bq = sum_k beta (:323-338):
      gamma = A*Es + Bq, delta = gamma*Ws*a*(1-a)
      dWs += gamma*a, dEs += A*Ws*a, dMs -= delta*Ss, dSs += delta*(x-Ms),
      dx_d += sum_h delta*Ss
    """
    x = np.asarray(x, np.float64)
    B, T, D = x.shape
    H = h0.shape[1]
    out, hT, tape = forward(x, h0, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev,
                            s_wpos, cm_t, gleak, vleak, U, eps)
    g = np.zeros((B, H)) if g_h is None else np.array(g_h, np.float64)
    gr = {k: np.zeros_like(np.asarray(v, np.float64)) for k, v in (
        ("w_pos", w_pos), ("w_erev", w_erev), ("mu", mu), ("sigma", sigma),
        ("sensory_mu", s_mu), ("sensory_sigma", s_sigma), ("sensory_erev", s_erev),
        ("sensory_w_pos", s_wpos), ("cm_t", cm_t), ("gleak_pos", gleak), ("vleak", vleak))}
    gx = np.zeros((B, T, D))
    for t in range(T - 1, -1, -1):
        g = g + g_out[:, t]
        A = np.zeros((B, H))
        Bq = np.zeros((B, H))
        for k in range(U - 1, -1, -1):
            vk = tape["v"][t][k]
            den = tape["den"][t][k]
            vk1 = tape["v"][t][k + 1] if k + 1 < U else out[:, t]
            alpha = g / den
            beta = -g * vk1 / den
            A += alpha
            Bq += beta
            gr["cm_t"] += (alpha * (vk - vk1)).sum(0)
            gr["gleak_pos"] += (alpha * (vleak - vk1)).sum(0)
            gr["vleak"] += (alpha * gleak).sum(0)
            a = _sig(sigma[None] * (vk[:, :, None] - mu[None]))             # (B,i,j)
            delta = (alpha[:, None, :] * w_erev[None] + beta[:, None, :] * w_pos[None]) * a * (1 - a)
            gr["w_erev"] += (alpha[:, None, :] * a).sum(0)
            gr["w_pos"] += (beta[:, None, :] * a).sum(0)
            gr["mu"] += (-delta * sigma[None]).sum(0)
            gr["sigma"] += (delta * (vk[:, :, None] - mu[None])).sum(0)
            g = alpha * cm_t + (delta * sigma[None]).sum(2)
        sa = _sig(s_sigma[None] * (x[:, t, :, None] - s_mu[None]))          # (B,d,h)
        gamma = A[:, None, :] * s_erev[None] + Bq[:, None, :]
        sdelta = gamma * s_wpos[None] * sa * (1 - sa)
        gr["sensory_w_pos"] += (gamma * sa).sum(0)
        gr["sensory_erev"] += (A[:, None, :] * s_wpos[None] * sa).sum(0)
        gr["sensory_mu"] += (-sdelta * s_sigma[None]).sum(0)
        gr["sensory_sigma"] += (sdelta * (x[:, t, :, None] - s_mu[None])).sum(0)
        gx[:, t] = (sdelta * s_sigma[None]).sum(2)
    gr["x"] = gx
    gr["state"] = g
    return gr
