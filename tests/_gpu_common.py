"""Helpers shared by the GPU parity tests: realistic inputs, calls through the
C-ABI, and the float64 oracle with the reference's bars.

The bars are the reference's own (test_ltc_cuda.py, README.md:120-121):
forward max-abs 1e-3, gradients allclose(rtol=5e-2, atol=1e-2). Each gradient
is also held to a tighter bar against the float64 oracle (max error <= 2e-3
of the gradient's largest entry), which catches a dropped term that the loose
bar would let through.
"""

from __future__ import annotations

import os

import pytest
import torch

import ltc
import ltc_cuda
from oracle import ltc_oracle as O

DEV = "cuda:0"
EPS = 1e-8
GRAD_NAMES = ("x", "state", "w_pos", "w_erev", "mu", "sigma", "sensory_mu", "sensory_sigma",
              "sensory_erev", "sensory_w_pos", "cm_t", "gleak_pos", "vleak")


@pytest.fixture(scope="module", autouse=True)
def _native():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    assert ltc_cuda._HAS_CUDA_KERNELS, f"HIP extension not loaded: {ltc_cuda._LOAD_ERROR}"
    assert os.path.realpath(ltc_cuda._cuda_module.capi.path) == os.path.realpath(ltc_cuda.LIB_PATH)


def boundary(B, T, D, H, seed=0, sparsity=0.5, x_scale=1.0, uniform_x=False):
    """Realistic boundary tensors on the CPU: module init + transforms, random x and h0."""
    torch.manual_seed(seed)
    p = O.init_params(D, H, sparsity, sparsity)
    w_pos, w_erev, cm_t, gleak_pos, s_wpos = O.transforms(p, 1.0 / 30.0, 6)
    if uniform_x:
        x = torch.rand(B, T, D) * 6.0 - 3.0
    else:
        x = torch.randn(B, T, D) * x_scale
    h0 = torch.randn(B, H) * 0.2
    return [x, h0, w_pos, w_erev, p["mu"], p["sigma"], p["sensory_mu"], p["sensory_sigma"],
            p["sensory_erev"], s_wpos, cm_t, gleak_pos, p["vleak"]]


def gpu_forward(args, U=6, save=False, x_override=None):
    dev_args = [a.to(DEV) for a in args]
    if x_override is not None:
        dev_args[0] = x_override
    res = ltc_cuda._cuda_module.ltc_full_forward(*dev_args, U, EPS, save)
    torch.cuda.synchronize()
    return dev_args, res


def gpu_backward(dev_args, saved, g_out, g_h, U=6):
    grads = ltc_cuda._cuda_module.ltc_full_backward(
        *dev_args, saved, g_out, g_h, U, EPS, g_h is not None)
    torch.cuda.synchronize()
    return [g.cpu() for g in grads]


def oracle_forward(args, U=6, dtype=torch.float64):
    with torch.no_grad():
        out, h = O.forward_loop(*[a.to(dtype) for a in args], U, EPS)
    return out, h


def oracle_grads(args, g_out, g_h, U=6, dtype=torch.float64):
    leaves = [a.to(dtype).clone().requires_grad_(True) for a in args]
    out, h = O.forward_loop(*leaves, U, EPS)
    outs, gs = [out], [g_out.to(dtype)]
    if g_h is not None:
        outs.append(h)
        gs.append(g_h.to(dtype))
    torch.autograd.backward(outs, gs)
    return [lf.grad for lf in leaves]


def assert_grads_close(got, ref, label):
    for name, g, r in zip(GRAD_NAMES, got, ref):
        g = g.double()
        r = r.double()
        err = (g - r).abs().max().item()
        scale = r.abs().max().item()
        assert torch.isfinite(g).all(), f"{label}: non-finite grad {name}"
        assert torch.allclose(g, r, rtol=5e-2, atol=1e-2), f"{label}: {name} err={err:.3e}"
        assert err <= 2e-3 * scale + 1e-6, f"{label}: {name} err={err:.3e} scale={scale:.3e}"


def _perturbed_module(D, H, seed, mapping="affine", sparsity=0.5):
    """Module with every leaf away from its default, including softplus's x > 20 branch."""
    torch.manual_seed(seed)
    m = ltc.TrueLiquidTimeConstant(D, H, sparsity=sparsity, sensory_sparsity=sparsity,
                                   input_mapping=mapping)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        m.input_norm.weight.add_(0.2 * torch.randn(D, generator=g))
        m.input_norm.bias.add_(0.1 * torch.randn(D, generator=g))
        m.input_w.add_(0.2 * torch.randn(D, generator=g))
        m.input_b.add_(0.1 * torch.randn(D, generator=g))
        m.w.view(-1)[:3] = 25.0
        m.sensory_w.view(-1)[:2] = 22.0
        m.cm.view(-1)[:1] = 21.0
    return m


def _oracle_module_grads(m, x, h0, G, Gh):
    p = {k: v.detach().cpu().double().clone() for k, v in m.state_dict().items()}
    names = dict(m.named_parameters())
    leaves = {k: v.requires_grad_(k in names) for k, v in p.items()}
    xd = x.detach().cpu().double().clone().requires_grad_(True)
    hd = h0.detach().cpu().double().clone().requires_grad_(True)
    out, (h, _) = O.module_forward(leaves, xd, (hd, hd), dt=m.dt, ode_unfolds=m.ode_unfolds,
                                   epsilon=m.epsilon)
    ((out * G.double()).sum() + (h * Gh.double()).sum()).backward()
    return out.detach(), h.detach(), {k: leaves[k].grad for k in names}, xd.grad, hd.grad
