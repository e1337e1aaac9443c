"""Compacted recurrent images of the register-resident cluster kernels (Hp = 256).

At Hp = 256 the cluster forward evaluates only the synapses whose w_pos or
w_erev is nonzero, and the fused cluster chain on the module path only those
whose mask entry is nonzero; each column's entries are spread over 16 chunks
and a wave runs as many slots as its fullest lane. These tests put columns
with no entry, with every entry and with a single entry next to random ones,
on the boundary and on the module path, and compare with the float64 oracle
at the reference's bars (forward max-abs 1e-3, gradients rtol 5e-2 / atol
1e-2, plus the tighter per-tensor bar of assert_grads_close).
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import (DEV, _native, _oracle_module_grads, _perturbed_module,  # noqa: F401
                         assert_grads_close, boundary, gpu_backward, gpu_forward, oracle_forward,
                         oracle_grads)

pytestmark = pytest.mark.gpu


def _plan(B, T, D, H):
    return ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)


def _extreme_columns(w_pos, w_erev, H, seed):
    """Column 0 without entries, column 1 full, column 2 with only its last row,
    column H-1 with only row 0; the rest keep their Bernoulli(0.5) mask."""
    g = torch.Generator().manual_seed(seed)
    w_pos[:, 0] = 0.0
    w_erev[:, 0] = 0.0
    full = torch.rand(H, generator=g) * 0.8 + 0.1
    w_pos[:, 1] = full
    w_erev[:, 1] = full * torch.where(torch.rand(H, generator=g) < 0.5, -1.0, 1.0)
    for col, row in ((2, H - 1), (H - 1, 0)):
        keep_p, keep_e = w_pos[row, col].item() or 0.7, w_erev[row, col].item() or -0.7
        w_pos[:, col] = 0.0
        w_erev[:, col] = 0.0
        w_pos[row, col] = keep_p
        w_erev[row, col] = keep_e


@pytest.mark.parametrize("shape", [(64, 2, 8, 256), (70, 2, 8, 200), (150, 2, 8, 256)],
                         ids=lambda s: "B%dT%dD%dH%d" % s)
def test_boundary_forward_and_backward_with_extreme_columns(shape):
    B, T, D, H = shape
    plan = _plan(B, T, D, H)
    assert plan["CP"] > 0 and plan["Hp"] == 256 and plan["RC"] == 16 and plan["fuse"] == 1, plan
    args = boundary(B, T, D, H, seed=7 * B + H)
    _extreme_columns(args[2], args[3], H, seed=B)
    dev_args, (out, h, saved) = gpu_forward(args, save=True)
    ref_out, ref_h = oracle_forward(args)
    e_out = (out.cpu().double() - ref_out).abs().max().item()
    e_h = (h.cpu().double() - ref_h).abs().max().item()
    print(f"compacted boundary forward {shape}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
    assert torch.isfinite(out).all() and e_out <= 1e-3 and e_h <= 1e-3
    g = torch.Generator().manual_seed(B + H)
    g_out = torch.randn(B, T, H, generator=g)
    g_h = torch.randn(B, H, generator=g)
    got = gpu_backward(dev_args, saved, g_out.to(DEV), g_h.to(DEV))
    ref = oracle_grads(args, g_out, g_h)
    # the boundary's chain keeps every real synapse: w_pos / w_erev gradients of
    # zero-weight synapses are not zero and must match too
    assert_grads_close(got, ref, f"compacted boundary backward {shape}")


@pytest.mark.parametrize("sparsity", [0.5, 1.0], ids=["sparse", "dense"])
def test_module_path_compacted_chain_with_extreme_masks(sparsity):
    B, T, D, H = 12, 3, 32, 256
    plan = _plan(B, T, D, H)
    assert plan["CP"] > 0 and plan["RC"] == 16 and plan["fuse"] == 1, plan
    m = _perturbed_module(D, H, seed=91, sparsity=sparsity)
    with torch.no_grad():
        mask = m.sparsity_mask
        if sparsity < 1.0:
            mask[:, 3] = 0.0        # a postsynaptic neuron without recurrent inputs
            mask[5, :] = 0.0        # a presynaptic neuron without outputs: no chain entries
            mask[:, 7] = 1.0        # a full forward column
            mask[9, :] = 1.0        # a full chain column
            mask[:, 11] = 0.0
            mask[H - 1, 11] = 1.0   # one entry, in the last row
    m = m.to(DEV)
    g = torch.Generator().manual_seed(5)
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
    print(f"compacted module path ({sparsity}): forward err {e_out:.2e}", flush=True)
    assert e_out <= 1e-3
    assert (h.detach().cpu().double() - r_h).abs().max().item() <= 1e-3
    names = ["x", "h0"] + [n for n, _ in m.named_parameters()]
    got = [xg.grad.cpu(), hg.grad.cpu()] + [p.grad.cpu() for _, p in m.named_parameters()]
    ref = [r_gx, r_gh] + [r_g[n] for n, _ in m.named_parameters()]
    for n, a, r in zip(names, got, ref):
        r = r.double()
        err = (a.double() - r).abs().max().item()
        assert torch.isfinite(a).all(), n
        assert torch.allclose(a.double(), r, rtol=5e-2, atol=1e-2), f"{n}: err {err:.2e}"
        assert err <= 2e-3 * r.abs().max().item() + 1e-6, f"{n}: err {err:.2e}"
    masked = (m.sparsity_mask == 0).cpu()
    for n in ("w", "erev", "mu", "sigma"):
        grad = dict(m.named_parameters())[n].grad.cpu()
        assert (grad[masked] == 0).all(), f"{n}: masked synapses must have zero gradients"
