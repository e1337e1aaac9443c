"""The sensory launches over the unmasked sensory synapses only.

When the sensory sums are not formed in the prep launch, the forward
(ltc_module_forward, and ltc_full_forward behind the eval-mode module) builds,
per 64-input chunk and neuron, the list of inputs whose sensory weight is
nonzero (in the prep launch) and the sensory launch walks only those. The
module backward of these shapes runs the compacted sensory backward
(sens_bwd_cmp_kernel: each lane holds one input's unmasked synapses of an
8-neuron group; the plan asserts that neither fused row backward takes it
over). These tests set the sensory mask so that the lists take every edge
the layout has:
a neuron with no input at all, a neuron with every input, a chunk that is
full for one neuron and empty for the next, a ragged last chunk (D not a
multiple of 64) and a single input, on both thread layouts of the launch (four
row groups per workgroup, and few rows with the inputs split over the waves),
with contiguous and strided x. Forward and gradients are compared with the
float64 oracle at the reference's bars (forward max-abs 1e-3, gradients rtol
5e-2 / atol 1e-2, plus the per-tensor bar of 2e-3 of the largest entry).
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import DEV, O, _native, _oracle_module_grads, _perturbed_module  # noqa: F401

pytestmark = pytest.mark.gpu

# (B, T, D, H, strided x)
CASES = [
    (40, 8, 130, 72, False),  # four row groups per workgroup, ragged third chunk
    (40, 8, 130, 72, True),
    (2, 3, 200, 40, False),   # few rows: the inputs split over the waves
    (300, 2, 1, 8, False),    # one input
    (300, 7, 130, 72, False), # 33 rows per backward block: a full 32-row chunk, then one;
                              # the forward walks one list per neuron over all of D
]


def _edge_mask(D, H, seed):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(D, H, generator=g) < 0.5).float()
    m[:, 0] = 0.0          # a neuron with no input
    if H > 1:
        m[:, 1] = 1.0      # a neuron with every input
    if D > 64 and H > 6:
        m[64:128, 5] = 1.0  # second chunk full for neuron 5 ...
        m[64:128, 6] = 0.0  # ... and empty for neuron 6
    return m


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B%dT%dD%dH%d%s" % (c[:4] + ("s" if c[4] else "",)))
def test_compacted_sensory_forward_matches_oracle(case):
    B, T, D, H, strided = case
    plan = ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)
    assert plan["module_sens_in_prep"] == 0, plan
    assert plan["sens_full_list"] == (1 if (B, T) == (300, 7) else 0), plan
    # the backward's sensory gradients come from sens_bwd_cmp_kernel: no fused
    # row backward, and no Hp = 128 sensory companions (those need Dp <= 128)
    assert plan["module_row_bwd_fused"] == 0, plan
    assert plan["module_row128_rec_fused"] == 0 or plan["Dp"] > 128, plan
    m = _perturbed_module(D, H, seed=5 * D + H).to(DEV)
    with torch.no_grad():
        m.sensory_sparsity_mask.copy_(_edge_mask(D, H, seed=D + H).to(DEV))
    g = torch.Generator().manual_seed(B * T + D)
    x = torch.randn(B, T, D, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.2
    G = torch.randn(B, T, H, generator=g)
    Gh = torch.randn(B, H, generator=g)
    if strided:
        wide = torch.zeros(B, T, 2 * D)
        wide[:, :, 0::2] = x
        xg = wide.to(DEV)[:, :, 0::2].requires_grad_(True)
        assert not xg.is_contiguous()
    else:
        xg = x.to(DEV).requires_grad_(True)
    hg = h0.to(DEV).requires_grad_(True)
    out, (h, _) = m(xg, (hg, hg))
    ((out * G.to(DEV)).sum() + (h * Gh.to(DEV)).sum()).backward()
    r_out, r_h, r_g, r_gx, r_gh = _oracle_module_grads(m, x, h0, G, Gh)
    e_out = (out.detach().cpu().double() - r_out).abs().max().item()
    e_h = (h.detach().cpu().double() - r_h).abs().max().item()
    print(f"compacted sensory {case}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
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


def test_compacted_sensory_forward_no_grad_matches_training_forward():
    """The no-grad forward (its images in the workspace, C5's form) and the
    training forward (images in the saved buffer) read the same compacted
    sensory image and agree bit for bit."""
    B, T, D, H = 128, 4, 96, 64
    assert ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)["module_sens_in_prep"] == 0
    m = _perturbed_module(D, H, seed=11).to(DEV)
    x = torch.randn(B, T, D, generator=torch.Generator().manual_seed(12)).to(DEV)
    with torch.no_grad():
        a, (ha, _) = m(x)
    b, (hb, _) = m(x.clone().requires_grad_(True))
    assert torch.equal(a, b.detach()) and torch.equal(ha, hb.detach())


@pytest.mark.parametrize("shape", [(40, 8, 130, 72), (2, 3, 200, 40)], ids=lambda s: "B%dT%dD%dH%d" % s)
def test_compacted_sensory_forward_boundary_path_matches_oracle(shape):
    """The same edge masks through ltc_full_forward: in eval mode the module
    calls the boundary with its cached transforms, whose prep launch builds
    the compacted lists from the masked sensory weights."""
    B, T, D, H = shape
    m = _perturbed_module(D, H, seed=3 * D + H).to(DEV)
    with torch.no_grad():
        m.sensory_sparsity_mask.copy_(_edge_mask(D, H, seed=2 * D + H).to(DEV))
    m.eval()
    g = torch.Generator().manual_seed(B + T + D)
    x = torch.randn(B, T, D, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.2
    with torch.no_grad():
        out, (h, _) = m(x.to(DEV), (h0.to(DEV), h0.to(DEV)))
    r_out, r_h, _, _, _ = _oracle_module_grads(m, x, h0, torch.zeros(B, T, H), torch.zeros(B, H))
    e_out = (out.cpu().double() - r_out).abs().max().item()
    e_h = (h.cpu().double() - r_h).abs().max().item()
    print(f"compacted sensory, boundary {shape}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
    assert e_out <= 1e-3 and e_h <= 1e-3


def _sens_rows_per_wave(B, T, Hp):
    """Rows per wave of the sensory forward with four row groups per
    workgroup: halved from 8 until the grid has at least 1024 workgroups."""
    BT, hb, rpw = B * T, Hp // 64, 8
    while rpw > 1 and hb * ((BT + 4 * rpw - 1) // (4 * rpw)) < 1024:
        rpw //= 2
    return rpw


@pytest.mark.parametrize("shape,rpw", [((512, 8, 130, 72), 2), ((1024, 8, 130, 72), 4)],
                         ids=lambda v: "B%dT%dD%dH%d" % v if isinstance(v, tuple) else "rpw%d" % v)
def test_full_list_sensory_forward_rows_per_wave(shape, rpw):
    """The per-neuron sensory forward (one list over all of D, the block's rows
    of x staged whole in LDS) at 2 and 4 rows per wave; C3 runs 8 and the
    (300, 7) case above 1. The no-grad forward and the training forward agree
    bit for bit, and both match the float64 oracle (max-abs 1e-3)."""
    B, T, D, H = shape
    plan = ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)
    assert plan["sens_full_list"] == 1 and plan["module_sens_in_prep"] == 0, plan
    assert _sens_rows_per_wave(B, T, plan["Hp"]) == rpw
    m = _perturbed_module(D, H, seed=7 * D + B).to(DEV)
    with torch.no_grad():
        m.sensory_sparsity_mask.copy_(_edge_mask(D, H, seed=D + B).to(DEV))
    g = torch.Generator().manual_seed(B + D)
    x = torch.randn(B, T, D, generator=g)
    h0 = torch.randn(B, H, generator=g) * 0.2
    xd, hd = x.to(DEV), h0.to(DEV)
    with torch.no_grad():
        a, (ha, _) = m(xd, (hd, hd))
    b, (hb, _) = m(xd.clone().requires_grad_(True), (hd, hd))
    assert torch.equal(a, b.detach()) and torch.equal(ha, hb.detach())
    p = {k: v.detach().cpu().double() for k, v in m.state_dict().items()}
    with torch.no_grad():
        r_out, (r_h, _) = O.module_forward(p, x.double(), (h0.double(), h0.double()), dt=m.dt,
                                           ode_unfolds=m.ode_unfolds, epsilon=m.epsilon)
    e_out = (a.cpu().double() - r_out).abs().max().item()
    e_h = (ha.cpu().double() - r_h).abs().max().item()
    print(f"full-list sensory forward {shape} rpw {rpw}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
    assert e_out <= 1e-3 and e_h <= 1e-3


@pytest.mark.parametrize("shape", [(512, 4, 40, 64), (1024, 4, 64, 64)], ids=lambda s: "B%dT%dD%dH%d" % s)
def test_no_grad_forward_normalises_rows_in_the_sensory_launch(shape):
    """A no-grad forward with D <= 64 and many rows (C5's form) normalises the
    input rows inside the sensory launch instead of the prep launch. With
    ln_row's arithmetic the outputs equal the training forward's (which keeps
    the prep launch's rows for the backward) bit for bit, also for a strided
    x, and match the float64 oracle."""
    B, T, D, H = shape
    m = _perturbed_module(D, H, seed=B + D).to(DEV)
    g = torch.Generator().manual_seed(D + H)
    wide = torch.randn(B, T, 2 * D, generator=g)
    x = wide[:, :, 0::2]
    xd = wide.to(DEV)[:, :, 0::2]
    assert not xd.is_contiguous()
    with torch.no_grad():
        a, (ha, _) = m(xd)
    b, (hb, _) = m(xd.clone().requires_grad_(True))
    assert torch.equal(a, b.detach()) and torch.equal(ha, hb.detach())
    h0 = torch.zeros(B, H)
    r_out, r_h, _, _, _ = _oracle_module_grads(m, x.contiguous(), h0, torch.zeros(B, T, H), torch.zeros(B, H))
    e_out = (a.cpu().double() - r_out).abs().max().item()
    print(f"no-grad rows normalised in the sensory launch {shape}: out err {e_out:.2e}", flush=True)
    assert e_out <= 1e-3
