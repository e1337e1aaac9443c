"""BASELINE configurations, and the code paths they run, against the float64 oracle.

* The training-mode module path (what bench.py times) at the settings C3 and
  C4 use: D = 256 and 512 LayerNorm rows, the fused cluster chains at
  Hp = 256 and 512 with their parameter-gradient partials, more than 4096
  (b, t) rows, and the full C3/C4 workloads themselves.
* C2 forward and backward at its full shape.
* C5, the streaming-inference workload: x[:, :, 0::2] of a (4096, 4, 128)
  tensor, no grad, in training and eval mode, and the state carried across
  calls (reference ltc.py:270-288, test_ltc_verification.py:126-140).
* The function-level entry point ltc_cuda_forward with autograd
  (reference ltc_cuda.py:241-388, test_ltc_cuda.py:140-163).
* The reference's remaining GPU cases: the D = 224 production shape
  (test_ltc_cuda.py:101-120), backward stability over 3 input scales x 3
  seeds with an MSE loss (:165-207) and odd hidden sizes in the backward
  (:262-287).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import ltc
import ltc_cuda
from _gpu_common import (  # noqa: F401  (_native: the module's autouse fixture)
    DEV, EPS, _native, _oracle_module_grads, _perturbed_module, assert_grads_close, boundary,
    oracle_forward, oracle_grads)
from oracle import ltc_oracle as O

pytestmark = pytest.mark.gpu


def _plan(B, T, D, H):
    return ltc_cuda._cuda_module.capi.plan(B, T, D, H, 6)


def _close(name, got, ref, rtol=5e-2, atol=1e-2, tight=2e-3):
    """The reference's bar and the tighter float64 bar on one tensor."""
    g = got.detach().cpu().double()
    r = ref.detach().double()
    err = (g - r).abs().max().item()
    scale = r.abs().max().item()
    assert torch.isfinite(g).all(), f"{name}: non-finite"
    assert torch.allclose(g, r, rtol=rtol, atol=atol), f"{name}: err {err:.2e}"
    assert err <= tight * scale + 1e-6, f"{name}: err {err:.2e} scale {scale:.2e}"
    return err


def _state_leaves(m):
    return {k: v.detach().cpu().double().clone() for k, v in m.state_dict().items()}


def _module(D, H, sparsity=0.5, seed=42):
    torch.manual_seed(seed)
    return ltc.TrueLiquidTimeConstant(D, H, dt=1.0 / 30.0, ode_unfolds=6, sparsity=sparsity,
                                      sensory_sparsity=sparsity)


# --------------------------------------------------------------------------- module path

MODULE_PATH_CASES = [
    # (B, T, D, H): what the plan runs
    (300, 20, 256, 16),  # 4 columns per lane in the LayerNorm kernels; B*T = 6000 > 4096
                         # (16 rows per LayerNorm-backward block) and a LayerNorm pre-sum
    (520, 8, 256, 8),    # B*T = 4160: just past the 16-rows-per-block switch
    (8, 4, 512, 256),    # 8 columns per lane; fused cluster chain at Hp = 256 with
                         # register-resident operands; finalize over cluster partials
    (2, 3, 200, 500),    # fused cluster chain at Hp = 512 with streamed operands
    (24, 8, 224, 64),    # the reference's production shape (D = 224)
]


@pytest.mark.parametrize("shape", MODULE_PATH_CASES, ids=lambda s: "B%dT%dD%dH%d" % s)
def test_module_path_at_large_config_settings(shape):
    B, T, D, H = shape
    plan = _plan(B, T, D, H)
    if H >= 256:
        assert plan["CP"] > 0 and plan["fuse"] == 1, plan
    m = _perturbed_module(D, H, seed=B + T + D + H).to(DEV)
    assert m.training
    g = torch.Generator().manual_seed(17)
    x = torch.randn(B, T, D, generator=g) * 2.0
    h0 = torch.randn(B, H, generator=g) * 0.2
    G = torch.randn(B, T, H, generator=g)
    Gh = torch.randn(B, H, generator=g)
    xg = x.to(DEV).requires_grad_(True)
    hg = h0.to(DEV).requires_grad_(True)
    out, (h, _) = m(xg, (hg, hg))
    ((out * G.to(DEV)).sum() + (h * Gh.to(DEV)).sum()).backward()
    r_out, r_h, r_g, r_gx, r_gh = _oracle_module_grads(m, x, h0, G, Gh)
    e_out = (out.detach().cpu().double() - r_out).abs().max().item()
    print(f"module path {shape}: forward err {e_out:.2e}", flush=True)
    assert e_out <= 1e-3
    assert (h.detach().cpu().double() - r_h).abs().max().item() <= 1e-3
    _close("x", xg.grad, r_gx)
    _close("h0", hg.grad, r_gh)
    for n, p in m.named_parameters():
        _close(n, p.grad, r_g[n])


def _full_config(cfg):
    if cfg == "C3":
        B, T, D, H, sp = 256, 64, 256, 256, 0.5
    else:
        B, T, D, H, sp = 128, 32, 512, 512, 1.0
    m = _module(D, H, sp)
    if cfg == "C3":
        x = torch.randn(B, T, D)
        target = torch.randn(B, T, H)
    else:
        x = torch.rand(B, T, D) * 6.0 - 3.0
        target = None
    return m.to(DEV), x, target


@pytest.mark.parametrize("cfg", ["C3", "C4"])
def test_full_size_module_path(cfg):
    """The training step bench.py times at C3 (MSE loss) and C4 (dense masks,
    U(-3, 3) input, sum loss), at full size.

    Rows are independent (LayerNorm included), so sampled rows of the output,
    and the input gradient of two rows, are checked against the float64
    oracle directly. Parameter gradients sum over rows: the full batch's must
    equal the sum of its two halves' under the same upstream gradient, and a
    two-row batch's are checked against the oracle.
    """
    m, x, target = _full_config(cfg)
    B, T, D = x.shape
    H = m.hidden_dim
    plan = _plan(B, T, D, H)
    assert plan["CP"] > 0 and plan["fuse"] == 1, plan
    xg = x.to(DEV).requires_grad_(True)
    out, (h, _) = m(xg)
    if target is not None:
        loss = F.mse_loss(out, target.to(DEV))
        G = (2.0 / out.numel()) * (out.detach() - target.to(DEV))
    else:
        loss = out.sum()
        G = torch.ones_like(out)
    loss.backward()
    full = {n: p.grad.detach().clone() for n, p in m.named_parameters()}
    gx = xg.grad.detach().clone()

    p = _state_leaves(m)
    rows = torch.tensor([0, 1, B // 2, B - 1])
    with torch.no_grad():
        r_out, (r_h, _) = O.module_forward(p, x[rows].double())
    e = (out.detach()[rows].cpu().double() - r_out).abs().max().item()
    eh = (h.detach()[rows].cpu().double() - r_h).abs().max().item()
    print(f"{cfg} module forward rows: err {e:.2e} / h {eh:.2e}", flush=True)
    assert e <= 1e-3 and eh <= 1e-3

    # input gradient of rows 0 and 1 under the full batch's upstream gradient
    leaves = {k: v.clone().requires_grad_(k in full) for k, v in p.items()}
    x2 = x[:2].double().clone().requires_grad_(True)
    o2, _ = O.module_forward(leaves, x2)
    (o2 * G[:2].cpu().double()).sum().backward()
    _close(f"{cfg} dx rows 0-1", gx[:2], x2.grad)

    # linearity over the batch
    sums = {n: torch.zeros_like(v) for n, v in full.items()}
    for sl in (slice(0, B // 2), slice(B // 2, B)):
        m.zero_grad(set_to_none=True)
        oh, _ = m(x[sl].to(DEV))
        (oh * G[sl]).sum().backward()
        for n, prm in m.named_parameters():
            sums[n] += prm.grad
    for n, v in full.items():
        err = (sums[n] - v).abs().max().item()
        assert err <= 1e-4 * v.abs().max().item() + 1e-7, f"{cfg} {n}: halves {err:.2e}"

    # parameter gradients of a two-row batch against the oracle
    m.zero_grad(set_to_none=True)
    o2g, _ = m(x[:2].to(DEV))
    (o2g * G[:2]).sum().backward()
    for n, prm in m.named_parameters():
        _close(f"{cfg} two-row {n}", prm.grad, leaves[n].grad)


def test_c2_full_shape_fwd_bwd_matches_oracle():
    """BASELINE config 2 at full size: B=32 T=16 D=128 H=128, loss = sum(out)."""
    m = _module(128, 128).to(DEV)
    x = torch.randn(32, 16, 128)
    xg = x.to(DEV).requires_grad_(True)
    out, (h, _) = m(xg)
    out.sum().backward()
    p = _state_leaves(m)
    names = dict(m.named_parameters())
    leaves = {k: v.clone().requires_grad_(k in names) for k, v in p.items()}
    xd = x.double().clone().requires_grad_(True)
    r_out, (r_h, _) = O.module_forward(leaves, xd)
    r_out.sum().backward()
    e = (out.detach().cpu().double() - r_out.detach()).abs().max().item()
    print(f"C2 forward err {e:.2e}", flush=True)
    assert e <= 1e-3
    assert (h.detach().cpu().double() - r_h.detach()).abs().max().item() <= 1e-3
    _close("x", xg.grad, xd.grad)
    for n, prm in names.items():
        _close(n, prm.grad, leaves[n].grad)


# --------------------------------------------------------------------------- C5 streaming

@pytest.mark.parametrize("mode", ["train", "eval"])
def test_c5_streaming_inference_matches_oracle(mode):
    """BASELINE config 5 exactly: seeded module, x = randn(4096, 4, 128)[:, :, 0::2]
    on the GPU, no grad. Training mode reads the strided view in place (module
    path); eval mode runs the cached transforms and the boundary path."""
    m = _module(64, 64)
    wide = torch.randn(4096, 4, 128)
    m = m.to(DEV)
    m.train(mode == "train")
    xv = wide.to(DEV)[:, :, 0::2]
    assert xv.stride() == (512, 128, 2)
    with torch.no_grad():
        out, (h, c) = m(xv)
    assert torch.equal(h, c) and out.shape == (4096, 4, 64)
    gen = torch.Generator().manual_seed(5)
    rows = torch.cat([torch.tensor([0, 1, 2047, 4095]), torch.randint(0, 4096, (4,), generator=gen)])
    p = _state_leaves(m)
    with torch.no_grad():
        r_out, (r_h, _) = O.module_forward(p, wide[rows][:, :, 0::2].double())
    e = (out[rows].cpu().double() - r_out).abs().max().item()
    eh = (h[rows].cpu().double() - r_h).abs().max().item()
    print(f"C5 {mode}: rows err {e:.2e} / h {eh:.2e}", flush=True)
    assert e <= 1e-3 and eh <= 1e-3
    # streaming: the state carried over two T=2 calls equals one T=4 call
    with torch.no_grad():
        o1, (h1, _) = m(xv[:, :2])
        o2, (h2, _) = m(xv[:, 2:], (h1, h1))
    d_out = (torch.cat([o1, o2], 1) - out).abs().max().item()
    d_h = (h2 - h).abs().max().item()
    print(f"C5 {mode}: carried state vs one call: out {d_out:.2e} h {d_h:.2e}", flush=True)
    assert d_out <= 1e-5 and d_h <= 1e-5
    # and the state matters (reference test_ltc_verification.py:126-140)
    with torch.no_grad():
        o2_fresh, _ = m(xv[:, 2:])
    assert not torch.allclose(o2_fresh, o2, atol=1e-6)


# --------------------------------------------------------------------------- function level

@pytest.mark.parametrize("shape", [(24, 8, 128, 64), (6, 3, 40, 256)],
                         ids=["C1", "B6T3D40H256-cluster"])
def test_ltc_cuda_forward_autograd_matches_oracle(shape):
    """ltc_cuda.ltc_cuda_forward on the 13 boundary tensors as autograd leaves:
    outputs and all 13 gradients against the float64 oracle."""
    B, T, D, H = shape
    args = boundary(B, T, D, H, seed=B * T + H)
    leaves = [a.to(DEV).clone().requires_grad_(True) for a in args]
    out, h = ltc_cuda.ltc_cuda_forward(*leaves, 6, EPS)
    g = torch.Generator().manual_seed(H)
    G = torch.randn(B, T, H, generator=g)
    Gh = torch.randn(B, H, generator=g)
    ((out * G.to(DEV)).sum() + (h * Gh.to(DEV)).sum()).backward()
    r_out, r_h = oracle_forward(args)
    assert (out.detach().cpu().double() - r_out).abs().max().item() <= 1e-3
    assert (h.detach().cpu().double() - r_h).abs().max().item() <= 1e-3
    ref = oracle_grads(args, G, Gh)
    assert_grads_close([lf.grad.cpu() for lf in leaves], ref, f"ltc_cuda_forward {shape}")
    # without grad mode nothing is saved, and the outputs are the same
    with torch.no_grad():
        out_ng, h_ng = ltc_cuda.ltc_cuda_forward(*leaves, 6, EPS)
    assert torch.equal(out_ng, out.detach()) and torch.equal(h_ng, h.detach())


# --------------------------------------------------------------------------- reference edge cases

def test_production_shape_d224_matches_torchscript_and_oracle():
    """test_ltc_cuda.py:101-120: B=24 T=8 D=224 H=64 with a zero state; the
    module's own TorchScript loop on the GPU (the reference's comparison) and
    the float64 oracle."""
    m = _module(224, 64).to(DEV)
    torch.manual_seed(101)
    x = torch.randn(24, 8, 224, device=DEV)
    z = torch.zeros(24, 64, device=DEV)
    m._force_torchscript = True
    with torch.no_grad():
        ts_out, _ = m(x, (z, z))
    m._force_torchscript = False
    with torch.no_grad():
        out, _ = m(x, (z, z))
    assert (ts_out - out).abs().max().item() < 1e-3
    with torch.no_grad():
        r_out, _ = O.module_forward(_state_leaves(m), x.cpu().double())
    assert (out.cpu().double() - r_out).abs().max().item() <= 1e-3


@pytest.mark.parametrize("input_scale", [0.1, 1.0, 5.0])
@pytest.mark.parametrize("seed", [11, 23, 47])
def test_backward_stability_mse(input_scale, seed):
    """test_ltc_cuda.py:165-207: D=48 H=24, B=3 T=6, MSE loss against a target of
    the same scale; the reference's bar (rtol 6e-2, atol 2e-2) and the tighter
    float64 bar on every parameter gradient."""
    m = _module(48, 24, seed=seed).to(DEV)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(3, 6, 48, generator=g) * input_scale
    target = torch.randn(3, 6, 24, generator=g) * input_scale
    out, _ = m(x.to(DEV))
    F.mse_loss(out, target.to(DEV)).backward()
    names = dict(m.named_parameters())
    leaves = {k: v.clone().requires_grad_(k in names) for k, v in _state_leaves(m).items()}
    r_out, _ = O.module_forward(leaves, x.double())
    F.mse_loss(r_out, target.double()).backward()
    for n, prm in names.items():
        _close(f"scale {input_scale} seed {seed} {n}", prm.grad, leaves[n].grad,
               rtol=6e-2, atol=2e-2)


@pytest.mark.parametrize("H", [17, 33, 63, 65])
def test_module_backward_odd_hidden(H):
    """test_ltc_cuda.py:262-287 (H = 33, 63) and the forward's odd sizes (17, 65):
    module fwd+bwd at D=32, B=2 T=4, loss = sum(out)."""
    m = _module(32, H).to(DEV)
    torch.manual_seed(909)
    x = torch.randn(2, 4, 32)
    out, _ = m(x.to(DEV))
    out.sum().backward()
    names = dict(m.named_parameters())
    leaves = {k: v.clone().requires_grad_(k in names) for k, v in _state_leaves(m).items()}
    r_out, _ = O.module_forward(leaves, x.double())
    r_out.sum().backward()
    assert (out.detach().cpu().double() - r_out.detach()).abs().max().item() <= 1e-3
    for n, prm in names.items():
        err = _close(f"H={H} {n}", prm.grad, leaves[n].grad)
        assert err < 0.05  # the reference's own bar
