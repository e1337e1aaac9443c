"""The module forward's sensory sums formed inside the prep launch.

With at most 256 blocks of (b,t) row and 64 neurons, D <= 128, H a multiple
of 4 and 16-byte aligned sensory leaves, ltc_module_forward forms each row's
LayerNorm and sensory sums in row blocks of the parameter-image launch (the
plan's module_sens_in_prep field),
reading the sensory leaves directly, instead of launching the sensory kernel
over a prepared image. These tests compare that path with the float64 oracle
at the reference's bars (forward max-abs 1e-3, gradients rtol 5e-2 / atol
1e-2, plus the tighter per-tensor bar), over ragged D (inputs past D in a
64-input chunk), H below Hp (neurons past H in a block) and several 64-neuron
blocks per row, and with the separate sensory launch, which a misaligned
sensory leaf selects, on the same inputs (the two add the sums in different
orders, so they agree to float32 rounding, not bit for bit).
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import DEV, _native, _oracle_module_grads, _perturbed_module  # noqa: F401

pytestmark = pytest.mark.gpu

SHAPES = [(24, 8, 128, 64), (3, 5, 40, 60), (8, 16, 128, 128), (4, 3, 100, 132)]


def _plan(B, T, D, H):
    return ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B%dT%dD%dH%d" % s)
def test_sensory_sums_in_prep_launch_match_oracle(shape):
    B, T, D, H = shape
    assert _plan(B, T, D, H)["module_sens_in_prep"] == 1
    m = _perturbed_module(D, H, seed=B + D + H).to(DEV)
    g = torch.Generator().manual_seed(D * H)
    x = torch.randn(B, T, D, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.2
    G = torch.randn(B, T, H, generator=g)
    Gh = torch.randn(B, H, generator=g)
    xg = x.to(DEV).requires_grad_(True)
    hg = h0.to(DEV).requires_grad_(True)
    out, (h, _) = m(xg, (hg, hg))
    ((out * G.to(DEV)).sum() + (h * Gh.to(DEV)).sum()).backward()
    r_out, r_h, r_g, r_gx, r_gh = _oracle_module_grads(m, x, h0, G, Gh)
    e_out = (out.detach().cpu().double() - r_out).abs().max().item()
    e_h = (h.detach().cpu().double() - r_h).abs().max().item()
    print(f"sensory sums in prep {shape}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
    assert e_out <= 1e-3 and e_h <= 1e-3
    names = ["x", "h0"] + [n for n, _ in m.named_parameters()]
    got = [xg.grad.cpu(), hg.grad.cpu()] + [p.grad.cpu() for _, p in m.named_parameters()]
    ref = [r_gx, r_gh] + [r_g[n] for n, _ in m.named_parameters()]
    for n, a, r in zip(names, got, ref):
        r = r.double()
        err = (a.double() - r).abs().max().item()
        assert torch.isfinite(a).all(), n
        assert torch.allclose(a.double(), r, rtol=5e-2, atol=1e-2), f"{n}: err {err:.2e}"
        assert err <= 2e-3 * r.abs().max().item() + 1e-6, f"{n}: err {err:.2e}"


def _misaligned(t):
    """A contiguous copy of t whose storage starts 4 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 1, device=t.device, dtype=t.dtype)
    v = buf[1:].view_as(t)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


@pytest.mark.parametrize("shape", [(24, 8, 128, 64), (4, 3, 100, 132)],
                         ids=lambda s: "B%dT%dD%dH%d" % s)
def test_sensory_sums_in_prep_launch_match_separate_launch(shape):
    B, T, D, H = shape
    m = _perturbed_module(D, H, seed=7 * D + H).to(DEV)
    sd = dict(m.state_dict())
    g = torch.Generator().manual_seed(B * T)
    x = torch.randn(B, T, D, generator=g).to(DEV)
    h0 = (torch.randn(B, H, generator=g) * 0.2).to(DEV)
    G = torch.randn(B, T, H, generator=g).to(DEV)
    sens = {"sensory_w", "sensory_erev", "sensory_sparsity_mask", "sensory_mu", "sensory_sigma"}
    res = []
    for mis in (False, True):
        leaves = []
        for k in ltc_cuda.MODULE_LEAVES:
            t = sd[k].detach()
            t = _misaligned(t) if (mis and k in sens) else t.clone()
            leaves.append(t.requires_grad_(t.is_floating_point() and "mask" not in k))
        xs = x.clone().requires_grad_(True)
        hs = h0.clone().requires_grad_(True)
        out, h = ltc_cuda.ltc_module_forward(xs, hs, leaves, m.dt, m.ode_unfolds, m.epsilon,
                                             m.input_norm.eps)
        ((out * G).sum() + h.sum()).backward()
        res.append([out.detach(), h.detach(), xs.grad, hs.grad]
                   + [t.grad for t in leaves if t.requires_grad])
    for i, (a, b) in enumerate(zip(*res)):
        assert torch.isfinite(a).all() and torch.isfinite(b).all(), i
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5, msg=f"tensor {i}")
