"""Hidden sizes above 1024 (the reference's kernels have no H limit:
csrc/ltc_kernels.cu:1223-1225 sizes the forward's shared memory by H).

Above H = 1024 no single workgroup holds a batch row's neurons, so the ODE
kernels run as clusters of Hp/64 workgroups, streamed operands, and when the
batch has more rows than one launch of at most one workgroup per CU holds,
the call makes one launch per NCL * NB rows (plan field launches_fwd /
launches_bwd). Forward and every gradient are compared with the float64
oracle at the reference's bars (forward max-abs 1e-3; gradients allclose
rtol 5e-2 / atol 1e-2, plus max error <= 2e-3 of each gradient's largest
entry), through ltc_full_forward / ltc_full_backward and through the module.
The oracle runs over groups of batch rows (rows are independent; parameter
gradients are summed over the groups) to bound its memory at H = 2048.
"""

from __future__ import annotations

import pytest
import torch

import ltc
import ltc_cuda
from _gpu_common import (DEV, EPS, _native, _oracle_module_grads, assert_grads_close,  # noqa: F401
                         boundary, gpu_backward, gpu_forward)
from oracle import ltc_oracle as O

pytestmark = pytest.mark.gpu

# (B, T, D, H, U, launches)
CASES = [
    (3, 2, 40, 1100, 6, 1),
    (2, 2, 64, 2048, 2, 1),
    (60, 1, 40, 1100, 2, 2),   # 56 rows per launch
    (40, 1, 24, 2048, 1, 2),   # 32 rows per launch
    (2, 1, 16, 4096, 1, 1),    # LTC_MAX_HIDDEN: 64 members per cluster
]


def _oracle_by_rows(args, g_out, g_h, U, rows=4):
    """Outputs and the 13 boundary gradients of the float64 oracle, taken over
    groups of `rows` batch rows."""
    B = args[0].shape[0]
    outs, hs, gx, gs = [], [], [], []
    gp = None
    for r0 in range(0, B, rows):
        sl = slice(r0, min(B, r0 + rows))
        leaves = [a[sl] if i < 2 else a for i, a in enumerate(args)]
        leaves = [a.double().clone().requires_grad_(True) for a in leaves]
        out, h = O.forward_loop(*leaves, U, EPS)
        torch.autograd.backward([out, h], [g_out[sl].double(), g_h[sl].double()])
        outs.append(out.detach())
        hs.append(h.detach())
        gx.append(leaves[0].grad)
        gs.append(leaves[1].grad)
        g = [lf.grad for lf in leaves[2:]]
        gp = g if gp is None else [a + b for a, b in zip(gp, g)]
    return torch.cat(outs), torch.cat(hs), [torch.cat(gx), torch.cat(gs)] + gp


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B%dT%dD%dH%dU%d" % c[:5])
def test_wide_hidden_boundary_matches_oracle(case):
    B, T, D, H, U, launches = case
    plan = ltc_cuda._cuda_module.capi.plan(B, T, D, H, U)
    print(f"{case}: plan CP={plan['CP']} NCL={plan['NCL']} NB={plan['NB']} KS={plan['KS']} "
          f"launches={plan['launches_fwd']}/{plan['launches_bwd']}", flush=True)
    assert plan["CP"] == plan["Hp"] // 64
    assert plan["launches_fwd"] == plan["launches_bwd"] == launches
    assert plan["ode_workgroups"] <= 256
    args = boundary(B, T, D, H, seed=H + B)
    g = torch.Generator().manual_seed(7)
    g_out = torch.randn(B, T, H, generator=g)
    g_h = torch.randn(B, H, generator=g)
    dev_args, (out, h, saved) = gpu_forward(args, U=U, save=True)
    grads = gpu_backward(dev_args, saved, g_out.to(DEV), g_h.to(DEV), U=U)
    r_out, r_h, r_grads = _oracle_by_rows(args, g_out, g_h, U)
    e_out = (out.cpu().double() - r_out).abs().max().item()
    e_h = (h.cpu().double() - r_h).abs().max().item()
    print(f"{case}: out err {e_out:.2e} h err {e_h:.2e}", flush=True)
    assert e_out <= 1e-3 and e_h <= 1e-3
    assert_grads_close(grads, r_grads, f"H={H} B={B}")


@pytest.mark.parametrize("shape", [(3, 2, 40, 1100, 6), (2, 2, 32, 2048, 2)],
                         ids=lambda s: "B%dT%dD%dH%dU%d" % s)
def test_wide_hidden_module_matches_oracle(shape):
    B, T, D, H, U = shape
    torch.manual_seed(B + H)
    m = ltc.TrueLiquidTimeConstant(D, H, ode_unfolds=U).to(DEV)
    g = torch.Generator().manual_seed(3)
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
    print(f"module {shape}: out err {e_out:.2e}", flush=True)
    assert e_out <= 1e-3
    assert (h.detach().cpu().double() - r_h).abs().max().item() <= 1e-3
    names = ["x", "h0"] + [n for n, _ in m.named_parameters()]
    got = [xg.grad.cpu(), hg.grad.cpu()] + [p.grad.cpu() for _, p in m.named_parameters()]
    ref = [r_gx, r_gh] + [r_g[n] for n, _ in m.named_parameters()]
    for n, a, r in zip(names, got, ref):
        r = r.double()
        err = (a.double() - r).abs().max().item()
        assert torch.isfinite(a).all(), n
        assert torch.allclose(a.double(), r, rtol=5e-2, atol=1e-2), f"{n}: {err:.2e}"
        assert err <= 2e-3 * r.abs().max().item() + 1e-6, f"{n}: {err:.2e}"


def test_wide_hidden_give_up_over_several_launches():
    """With a wait budget of 0 every member of both launches leaves at its first
    wait; the second launch's clear keeps the first launch's status word, so
    every output of the call is NaN and the fault is reported once."""
    capi = ltc_cuda._cuda_module.capi
    B, T, D, H, U = 60, 1, 40, 1100, 2
    assert capi.plan(B, T, D, H, U)["launches_fwd"] == 2
    capi.device_status(clear=True)
    args = boundary(B, T, D, H, seed=5)
    prev = capi.lib.ltc_set_cluster_spin_ticks(0)
    try:
        dev_args, (out, h, saved) = gpu_forward(args, U=U, save=True)
    finally:
        capi.lib.ltc_set_cluster_spin_ticks(prev)
    assert torch.isnan(out).all() and torch.isnan(h).all() and torch.isnan(saved).all()
    assert capi.lib.ltc_device_status(1) == 3
    assert capi.lib.ltc_device_status(0) == 0
    dev_args, (out, h, saved) = gpu_forward(args, U=U, save=True)
    assert torch.isfinite(out).all()
    g_out = torch.randn(B, T, H, device=DEV)
    prev = capi.lib.ltc_set_cluster_spin_ticks(0)
    try:
        grads = gpu_backward(dev_args, saved, g_out, None, U=U)
    finally:
        capi.lib.ltc_set_cluster_spin_ticks(prev)
    for gr in grads:
        assert torch.isnan(gr).all()
    assert capi.lib.ltc_device_status(1) == 3
    grads = gpu_backward(dev_args, saved, g_out, None, U=U)
    for gr in grads:
        assert torch.isfinite(gr).all()
    capi.device_status()
