"""Autograd semantics of the fused module path's backward node.

The C++ glue (`_ltc_torch`) records a plain autograd Node per layer call; the
Python fallback records an autograd Function with save_for_backward, as the
reference's LTCCudaFunction does (ltc_cuda.py:241-388). Both must behave the
same way towards autograd: one node for both outputs, an error on a second
backward through a freed graph and on a leaf edited in place after the
forward, gradients only where they are asked for, and no node at all when
nothing requires a gradient.
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import DEV, _native, _perturbed_module  # noqa: F401

pytestmark = pytest.mark.gpu

B, T, D, H = 6, 4, 40, 24


def _module(seed=21):
    return _perturbed_module(D, H, seed=seed).to(DEV)


@pytest.fixture(params=[True, False], ids=["cpp", "python"])
def use_ext(request):
    saved = ltc_cuda._torch_ext
    if request.param:
        assert saved is not None, "torch extension (_ltc_torch) not loaded"
    else:
        ltc_cuda._torch_ext = None
    yield request.param
    ltc_cuda._torch_ext = saved


def test_one_node_for_both_outputs(use_ext):
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    out, (h, _) = m(x)
    assert out.grad_fn is not None and out.grad_fn is h.grad_fn
    if use_ext:
        assert out.grad_fn.name() == "LTCModuleBackward"


def test_second_backward_through_a_freed_graph_raises(use_ext):
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    out, _ = m(x)
    loss = out.sum()
    loss.backward()
    with pytest.raises(RuntimeError, match="second time"):
        loss.backward()


def test_leaf_edited_in_place_after_forward_raises(use_ext):
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    out, _ = m(x)
    with torch.no_grad():
        m.w.add_(1.0)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        out.sum().backward()


def test_gradients_only_where_asked(use_ext):
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    G = torch.randn(B, T, H, device=DEV)
    xa = x.clone().requires_grad_(True)
    out, _ = m(xa)
    (out * G).sum().backward()
    full_gx = xa.grad.clone()
    full_gw = m.w.grad.clone()
    # frozen parameters: only x gets a gradient, the same one
    m.zero_grad(set_to_none=True)
    for p in m.parameters():
        p.requires_grad_(False)
    xb = x.clone().requires_grad_(True)
    out_b, _ = m(xb)
    assert out_b.requires_grad
    (out_b * G).sum().backward()
    assert torch.equal(xb.grad, full_gx)
    assert all(p.grad is None for p in m.parameters())
    # nothing requires a gradient: no node, same outputs
    out_c, (h_c, _) = m(x)
    assert not out_c.requires_grad and out_c.grad_fn is None and h_c.grad_fn is None
    assert torch.equal(out_c, out_b.detach())
    # torch.autograd.grad over a subset
    for p in m.parameters():
        p.requires_grad_(True)
    xd = x.clone().requires_grad_(True)
    out_d, _ = m(xd)
    gx, gw = torch.autograd.grad((out_d * G).sum(), [xd, m.w])
    assert torch.equal(gx, full_gx) and torch.equal(gw, full_gw)
    assert m.w.grad is None


def test_output_gradient_of_another_dtype(use_ext):
    """A double-precision loss sends a float64 output gradient back through
    the cast; the node receives it as float32 and gives the float32 result."""
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    G = torch.randn(B, T, H, device=DEV)
    out, _ = m(x)
    (out * G).sum().backward()
    ref = [p.grad.clone() for p in m.parameters()]
    m.zero_grad(set_to_none=True)
    out2, _ = m(x)
    (out2.double() * G.double()).sum().backward()
    for a, b in zip(ref, [p.grad for p in m.parameters()]):
        assert a.dtype == b.dtype == torch.float32
        assert torch.allclose(a, b, rtol=1e-6, atol=1e-7)


def test_inference_mode_matches_no_grad(use_ext):
    """Under torch.inference_mode the layer records nothing and returns the
    no-grad forward's outputs bitwise (inference tensors)."""
    m = _module()
    x = torch.randn(B, T, D, device=DEV)
    with torch.no_grad():
        ref, (rh, _) = m(x)
    with torch.inference_mode():
        out, (h, _) = m(x)
    assert out.is_inference() and h.is_inference()
    assert out.grad_fn is None
    assert torch.equal(out, ref) and torch.equal(h, rh)
