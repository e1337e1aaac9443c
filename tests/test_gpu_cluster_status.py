"""A cluster member that gives up waiting is reported, and its call's outputs are NaN.

The failure is forced from the host: a wait budget of 0 ticks makes every
member leave at its first exchange (ltc_set_cluster_spin_ticks), so every
kernel still exits normally. The call then overwrites every output it writes
with NaN and raises the device's fault flag, which ltc_device_status()
reports and clears.
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import DEV, _native, _perturbed_module, boundary, gpu_backward, gpu_forward  # noqa: F401

pytestmark = pytest.mark.gpu

T, D, H = 2, 8, 256
DEFAULT_TICKS = 20000000
# Batch sizes at H = 256: one row per cluster in the forward and the chain
# (the one-group kernels), one-row forward and two-row chain clusters, and
# four-row forward and eight-row chain clusters (the two-group kernels).
BATCHES = [16, 48, 200]


@pytest.fixture(params=BATCHES, ids=lambda b: f"B{b}")
def B(request):
    return request.param


@pytest.fixture()
def capi(B):
    c = ltc_cuda._cuda_module.capi
    plan = c.plan(B, T, D, H, 6)
    assert plan["CP"] > 0
    print(f"B={B}: forward rows per cluster {plan['NB']}, chain {plan['NBB']}", flush=True)
    c.device_status(clear=True)  # start clean
    yield c
    assert c.lib.ltc_set_cluster_spin_ticks(DEFAULT_TICKS) >= 0
    c.lib.ltc_device_status(1)


@pytest.fixture()
def capi_row():
    """The library, for the single-workgroup give-up tests (no cluster plan)."""
    c = ltc_cuda._cuda_module.capi
    c.device_status(clear=True)
    yield c
    assert c.lib.ltc_set_cluster_spin_ticks(DEFAULT_TICKS) >= 0
    c.lib.ltc_device_status(1)


class _NoWait:
    """Wait budget of 0 ticks inside the block, the default after it."""

    def __init__(self, capi):
        self.capi = capi

    def __enter__(self):
        assert self.capi.lib.ltc_set_cluster_spin_ticks(0) == DEFAULT_TICKS

    def __exit__(self, *exc):
        assert self.capi.lib.ltc_set_cluster_spin_ticks(DEFAULT_TICKS) == 0


def _expect_fault(capi):
    rc = capi.lib.ltc_device_status(1)
    assert rc == 3 and "gave up" in capi.last_error(), (rc, capi.last_error())
    assert capi.lib.ltc_device_status(0) == 0  # the first read cleared it


def test_forward_give_up_sets_every_output_to_nan(capi, B):
    args = boundary(B, T, D, H, seed=31)
    with _NoWait(capi):
        _, (out, h, saved) = gpu_forward(args, save=True)
    assert torch.isnan(out).all() and torch.isnan(h).all() and torch.isnan(saved).all()
    _expect_fault(capi)
    # the default budget again: finite results and a clean status
    _, (out, h, saved) = gpu_forward(args, save=True)
    assert torch.isfinite(out).all() and torch.isfinite(h).all()
    capi.device_status()


def test_backward_give_up_sets_every_gradient_to_nan(capi, B):
    args = boundary(B, T, D, H, seed=32)
    dev_args, (out, h, saved) = gpu_forward(args, save=True)
    assert torch.isfinite(out).all()
    g_out = torch.randn(B, T, H, device=DEV)
    g_h = torch.randn(B, H, device=DEV)
    with _NoWait(capi):
        grads = gpu_backward(dev_args, saved, g_out, g_h)
    for g in grads:
        assert torch.isnan(g).all()
    _expect_fault(capi)
    grads = gpu_backward(dev_args, saved, g_out, g_h)
    for g in grads:
        assert torch.isfinite(g).all()
    capi.device_status()


def test_module_path_give_up_is_reported_through_python(capi, B):
    m = _perturbed_module(D, H, seed=33).to(DEV)
    x = torch.randn(B, T, D, device=DEV)
    with _NoWait(capi):
        out, (h, _) = m(x)
        out.sum().backward()
    assert torch.isnan(out).all() and torch.isnan(h).all()
    for n, p in m.named_parameters():
        assert torch.isnan(p.grad).all(), n
    with pytest.raises(RuntimeError, match="gave up"):
        ltc_cuda.device_status()
    ltc_cuda.device_status()  # cleared by the call that raised


@pytest.mark.parametrize("D1", [128, 48])
def test_fused_row_backward_give_up_sets_every_gradient_to_nan(capi_row, D1):
    capi = capi_row
    """At H = 64 the module backward's sensory and LayerNorm part runs in
    companion workgroups that wait for the chain's words: with a budget of 0
    they leave at once, and the finalize writes NaN into every gradient."""
    B1, T1, H1 = 24, 8, 64
    plan = capi.plan(B1, T1, D1, H1, 6)
    assert plan["CP"] == 0 and plan["Hp"] == 64 and plan["NB"] == 1 and plan["fuse"] == 1, plan
    m = _perturbed_module(D1, H1, seed=34).to(DEV)
    x = torch.randn(B1, T1, D1, device=DEV, requires_grad=True)
    h0 = (torch.randn(B1, H1, device=DEV) * 0.2).requires_grad_(True)
    out, (h, _) = m(x, (h0, h0))
    assert torch.isfinite(out).all()
    with _NoWait(capi):
        (out.sum() + h.sum()).backward()
    assert torch.isnan(x.grad).all() and torch.isnan(h0.grad).all()
    for n, p in m.named_parameters():
        assert torch.isnan(p.grad).all(), n
    _expect_fault(capi)
    m.zero_grad(set_to_none=True)
    x.grad = h0.grad = None
    out, (h, _) = m(x, (h0, h0))
    (out.sum() + h.sum()).backward()
    assert torch.isfinite(x.grad).all() and torch.isfinite(h0.grad).all()
    for n, p in m.named_parameters():
        assert torch.isfinite(p.grad).all(), n
    capi.device_status()



@pytest.mark.parametrize("shape", [(32, 4, 128, 128), (5, 3, 40, 100), (4, 3, 200, 100)],
                         ids=lambda s: "B%dT%dD%dH%d" % s)
def test_recurrent_gradient_companions_give_up_sets_every_gradient_to_nan(capi_row, shape):
    capi = capi_row
    """At Hp = 128 the module backward forms the recurrent parameter-gradient
    sums in companion workgroups that wait for the chain's alpha/beta words:
    with a budget of 0 they leave at once, and the finalize writes NaN into
    every gradient, dL/dx and dL/dh0; with the default budget again the
    results are finite and the status clean."""
    B1, T1, D1, H1 = shape
    plan = capi.plan(B1, T1, D1, H1, 6)
    assert plan["module_row128_rec_fused"] == 1, plan
    m = _perturbed_module(D1, H1, seed=35).to(DEV)
    x = torch.randn(B1, T1, D1, device=DEV, requires_grad=True)
    h0 = (torch.randn(B1, H1, device=DEV) * 0.2).requires_grad_(True)
    out, (h, _) = m(x, (h0, h0))
    assert torch.isfinite(out).all()
    with _NoWait(capi):
        (out.sum() + h.sum()).backward()
    assert torch.isnan(x.grad).all() and torch.isnan(h0.grad).all()
    for n, p in m.named_parameters():
        assert torch.isnan(p.grad).all(), n
    _expect_fault(capi)
    m.zero_grad(set_to_none=True)
    x.grad = h0.grad = None
    out, (h, _) = m(x, (h0, h0))
    (out.sum() + h.sum()).backward()
    assert torch.isfinite(x.grad).all() and torch.isfinite(h0.grad).all()
    for n, p in m.named_parameters():
        assert torch.isfinite(p.grad).all(), n
    capi.device_status()
