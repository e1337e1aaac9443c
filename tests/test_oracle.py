"""Pins the CPU oracle (oracle/) before anything is compared against it.

Three independent anchors:
  1. golden vectors written by the reference itself (tests/golden/), for the
     init RNG order, forward outputs and all leaf-parameter gradients;
  2. closed forms the mathematics fixes (no synapses, sigma = 0, fixed point,
     scalar brute force, saturation, U sensitivity);
  3. two derivations of the boundary gradients that share no code: autograd
     through `ltc_oracle` and the closed-form `ltc_analytic`, plus gradcheck.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ltc_analytic, ltc_oracle as O


def _module_params(cfg):
    torch.manual_seed(cfg["seed_model"])
    return O.init_params(cfg["D"], cfg["H"], cfg["sparsity"], cfg["sensory_sparsity"],
                         cfg["input_mapping"])


def test_golden_init_matches_reference(golden):
    p = _module_params(golden["cfg"])
    for k, v in p.items():
        ref = golden["state." + k]
        assert np.array_equal(v.numpy(), ref), f"init mismatch in {k}"


def test_golden_forward_matches_reference(golden):
    cfg = golden["cfg"]
    p = _module_params(cfg)
    x = torch.from_numpy(golden["x"])
    h0 = (torch.from_numpy(golden["h0"]),) * 2 if "h0" in golden else None
    with torch.no_grad():
        out, (h, _) = O.module_forward(p, x, h0, dt=cfg["dt"], ode_unfolds=cfg["U"])
    # Same torch ops in the same order as the reference: identical to the bit.
    assert np.array_equal(out.numpy(), golden["out"])
    assert np.array_equal(h.numpy(), golden["h"])
    with torch.no_grad():
        out_s, _ = O.module_forward(p, x, h0, dt=cfg["dt"], ode_unfolds=cfg["U"], scripted=True)
    assert np.abs(out_s.numpy() - golden["out"]).max() < 1e-6


def test_golden_grads_match_reference(golden):
    cfg = golden["cfg"]
    p = _module_params(cfg)
    leaves = {k: v.clone().requires_grad_(("grad." + k) in golden) for k, v in p.items()}
    x = torch.from_numpy(golden["x"])
    h0 = (torch.from_numpy(golden["h0"]),) * 2 if "h0" in golden else None
    out, _ = O.module_forward(leaves, x, h0, dt=cfg["dt"], ode_unfolds=cfg["U"])
    if cfg["loss"] == "mse":
        loss = torch.nn.functional.mse_loss(out, torch.from_numpy(golden["target"]))
    else:
        loss = out.sum()
    loss.backward()
    names = [k[5:] for k in golden if k.startswith("grad.")]
    assert len(names) >= 13
    for k in names:
        ref = golden["grad." + k]
        got = leaves[k].grad.numpy()
        scale = max(1.0, float(np.abs(ref).max()))
        assert np.abs(got - ref).max() <= 1e-5 * scale, f"grad mismatch in {k}"


# --------------------------------------------------------------------------- closed forms

def _boundary(B, T, D, H, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.rand(*s, generator=g, dtype=dtype)
    x = torch.randn(B, T, D, generator=g, dtype=dtype)
    h0 = torch.randn(B, H, generator=g, dtype=dtype) * 0.3
    w_pos = r(H, H) * (r(H, H) < 0.6)
    w_erev = w_pos * torch.where(r(H, H) < 0.8, 1.0, -1.0).to(dtype)
    mu = 0.3 + 0.5 * r(H, H)
    sigma = 3.0 + 5.0 * r(H, H)
    s_mu = 0.3 + 0.5 * r(D, H)
    s_sigma = 3.0 + 5.0 * r(D, H)
    s_erev = torch.where(r(D, H) < 0.8, 1.0, -1.0).to(dtype)
    s_wpos = r(D, H)
    cm = 5.0 + 15.0 * r(H)
    gl = 0.1 + r(H)
    vl = -0.2 + 0.4 * r(H)
    return [x, h0, w_pos, w_erev, mu, sigma, s_mu, s_sigma, s_erev, s_wpos, cm, gl, vl]


def test_no_synapses_geometric_approach_to_vleak():
    B, T, D, H, U, eps = 2, 3, 4, 5, 6, 1e-8
    a = _boundary(B, T, D, H)
    a[2].zero_(); a[3].zero_(); a[9].zero_()      # WP = WE = Ws = 0
    x, h0, *params = a
    out, h = O.forward_loop(x, h0, *params, U, eps)
    cm, gl, vl = params[-3:]
    r = cm / (cm + gl + eps)
    vstar = gl * vl / (gl + eps)
    for t in range(T):
        n = (t + 1) * U
        expect = vstar + (h0 - vstar) * r ** n
        assert torch.allclose(out[:, t], expect, atol=1e-12, rtol=0)


def test_sigma_zero_affine_recurrence():
    B, T, D, H, U, eps = 2, 2, 3, 4, 5, 1e-8
    a = _boundary(B, T, D, H, seed=1)
    a[5].zero_(); a[7].zero_()                      # S = Ss = 0: every gate is 1/2
    x, h0, wp, we, mu, sg, smu, ssg, se, sw, cm, gl, vl = a
    out, _ = O.forward_loop(x, h0, wp, we, mu, sg, smu, ssg, se, sw, cm, gl, vl, U, eps)
    K1 = gl * vl + 0.5 * we.sum(0) + 0.5 * (sw * se).sum(0)
    K2 = cm + gl + 0.5 * wp.sum(0) + 0.5 * sw.sum(0) + eps
    r = cm / K2
    vstar = K1 / (K2 - cm)
    for t in range(T):
        n = (t + 1) * U
        expect = vstar + (h0 - vstar) * r ** n
        assert torch.allclose(out[:, t], expect, atol=1e-12, rtol=0)


def test_fixed_point_at_vleak():
    B, T, D, H, U = 3, 4, 2, 6, 6
    a = _boundary(B, T, D, H, seed=2)
    a[2].zero_(); a[3].zero_(); a[9].zero_()
    x, h0, *params = a
    h0 = params[-1].expand(B, H).clone()            # v0 = vleak, eps = 0
    out, h = O.forward_loop(x, h0, *params, U, 0.0)
    assert torch.allclose(out, params[-1].expand(B, T, H), atol=1e-15, rtol=0)


def test_scalar_brute_force():
    """H = D = 1 evaluated with Python floats and math.exp, line by line."""
    U, eps = 4, 1e-8
    xs = [0.7, -1.3, 0.2]
    v0 = 0.1
    wp, we, mu, sg = 0.6, -0.6, 0.45, 5.0
    smu, ssg, se, sw = 0.5, 4.0, 1.0, 0.8
    cm, gl, vl = 12.0, 0.4, -0.1
    sig = lambda z: 1.0 / (1.0 + math.exp(-z))
    v = v0
    expect = []
    for xv in xs:
        sa = sig(ssg * (xv - smu))
        ns, ds = sw * sa * se, sw * sa
        for _ in range(U):
            a = sig(sg * (v - mu))
            v = (cm * v + gl * vl + a * we + ns) / (cm + gl + a * wp + ds + eps)
        expect.append(v)
    t = lambda val: torch.tensor([[val]], dtype=torch.float64)
    out, _ = O.forward_loop(torch.tensor([[[xv] for xv in xs]], dtype=torch.float64), t(v0),
                            t(wp), t(we), t(mu), t(sg), t(smu), t(ssg), t(se), t(sw),
                            torch.tensor([cm], dtype=torch.float64),
                            torch.tensor([gl], dtype=torch.float64),
                            torch.tensor([vl], dtype=torch.float64), U, eps)
    assert np.allclose(out[0, :, 0].numpy(), expect, rtol=0, atol=1e-15)


def test_unfold_count_matters():
    a = _boundary(1, 3, 4, 5, seed=3, dtype=torch.float32)
    x, h0, *params = a
    o1, _ = O.forward_loop(x, h0, *params, 1, 1e-8)
    o6, _ = O.forward_loop(x, h0, *params, 6, 1e-8)
    assert not torch.allclose(o1, o6, atol=1e-4)


def test_saturation_stays_finite():
    a = _boundary(2, 4, 6, 5, seed=4, dtype=torch.float32)
    a[0] = a[0] * 10.0
    a[5].fill_(100.0)
    a[7].fill_(100.0)
    x, h0, *params = a
    out, h = O.forward_loop(x, h0, *params, 6, 1e-8)
    assert torch.isfinite(out).all() and torch.isfinite(h).all()


# --------------------------------------------------------------------------- gradients

@pytest.mark.parametrize("shape", [(2, 3, 5, 4, 3), (3, 4, 6, 7, 2), (1, 2, 3, 9, 6)])
def test_analytic_backward_matches_autograd(shape):
    B, T, D, H, U = shape
    eps = 1e-8
    a = _boundary(B, T, D, H, seed=sum(shape))
    leaves = [t.clone().requires_grad_(True) for t in a]
    out, h = O.forward_loop(*leaves, U, eps)
    g = torch.Generator().manual_seed(7)
    g_out = torch.randn(B, T, H, generator=g, dtype=torch.float64)
    g_h = torch.randn(B, H, generator=g, dtype=torch.float64)
    torch.autograd.backward([out, h], [g_out, g_h])
    npa = [t.detach().numpy() for t in a]
    R = ltc_analytic.backward(*npa, U, eps, g_out.numpy(), g_h.numpy())
    names = ["x", "state", "w_pos", "w_erev", "mu", "sigma", "sensory_mu", "sensory_sigma",
             "sensory_erev", "sensory_w_pos", "cm_t", "gleak_pos", "vleak"]
    for name, leaf in zip(names, leaves):
        assert np.allclose(R[name], leaf.grad.numpy(), rtol=1e-10, atol=1e-12), name
    out_np, h_np, _ = ltc_analytic.forward(*npa, U, eps)
    assert np.allclose(out_np, out.detach().numpy(), rtol=0, atol=1e-13)


def test_gradcheck_tiny():
    B, T, D, H, U = 2, 2, 3, 3, 2
    a = _boundary(B, T, D, H, seed=11)
    leaves = tuple(t.clone().requires_grad_(True) for t in a)
    fn = lambda *ts: O.forward_loop(*ts, U, 1e-8)
    assert torch.autograd.gradcheck(fn, leaves, eps=1e-6, atol=1e-6, rtol=1e-4)


def test_step_halves_pre_states_and_sensory_sums():
    """`unfolds` returns the pre-state of every unfold: pre[k] is the state after
    k unfolds, so an off-by-one in the saved list fails; `sensory_sums` agrees
    with a scalar loop over (b, d, h) on a tiny case."""
    torch.manual_seed(3)
    B, D, H, U = 2, 3, 4, 6
    p = O.init_params(D, H)
    w_pos, w_erev, cm_t, gleak_pos, s_wpos = O.transforms(p, 1.0 / 30.0, U)
    x = torch.randn(B, D, dtype=torch.float64)
    h0 = torch.randn(B, H, dtype=torch.float64) * 0.2
    d = {k: v.double() for k, v in p.items()}
    sn, sd = O.sensory_sums(x, d["sensory_mu"], d["sensory_sigma"], d["sensory_erev"],
                            s_wpos.double())
    for b in range(B):
        for h in range(H):
            num = den = 0.0
            for i in range(D):
                z = d["sensory_sigma"][i, h].item() * (x[b, i].item() - d["sensory_mu"][i, h].item())
                a = 1.0 / (1.0 + math.exp(-z)) * s_wpos[i, h].item()
                num += a * d["sensory_erev"][i, h].item()
                den += a
            assert abs(sn[b, h].item() - num) < 1e-12 and abs(sd[b, h].item() - den) < 1e-12
    args = (w_pos.double(), w_erev.double(), d["mu"], d["sigma"], sn, sd, cm_t.double(),
            gleak_pos.double(), d["vleak"])
    v6, pre = O.unfolds(h0, *args, U, 1e-8)
    assert len(pre) == U and torch.equal(pre[0], h0)
    for k in range(1, U):
        vk, _ = O.unfolds(h0, *args, k, 1e-8)
        assert torch.equal(pre[k], vk)
    v1, _ = O.unfolds(pre[U - 1], *args, 1, 1e-8)
    assert torch.equal(v1, v6)
