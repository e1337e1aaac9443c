"""Drop-in API contract of the product module on the CPU.

Ports the property checks of the reference's test_ltc_verification.py
(:24-202) to this build's `ltc.TrueLiquidTimeConstant`, and checks that a
seed builds bit-identical parameters to the reference (golden state dicts)
and that the module's own CPU path reproduces the reference outputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ltc
import ltc_cuda
from ltc import TemporalLTC, TrueLiquidTimeConstant


def _build(cfg):
    torch.manual_seed(cfg["seed_model"])
    return TrueLiquidTimeConstant(cfg["D"], cfg["H"], dt=cfg["dt"], ode_unfolds=cfg["U"],
                                  sparsity=cfg["sparsity"],
                                  sensory_sparsity=cfg["sensory_sparsity"],
                                  input_mapping=cfg["input_mapping"])


def test_seed_builds_reference_state_dict(golden):
    m = _build(golden["cfg"])
    sd = m.state_dict()
    ref_keys = sorted(k[6:] for k in golden if k.startswith("state."))
    assert sorted(sd.keys()) == ref_keys
    for k in ref_keys:
        assert np.array_equal(sd[k].numpy(), golden["state." + k]), k
    params = sorted(n for n, _ in m.named_parameters())
    assert params == sorted(k[5:] for k in golden if k.startswith("grad."))


def test_cpu_forward_and_grads_match_reference(golden):
    cfg = golden["cfg"]
    m = _build(cfg)
    x = torch.from_numpy(golden["x"])
    h0 = (torch.from_numpy(golden["h0"]),) * 2 if "h0" in golden else None
    with torch.no_grad():
        out, (h, c) = m(x, h0)
    assert np.abs(out.numpy() - golden["out"]).max() < 1e-6
    assert torch.equal(h, c)
    m.zero_grad(set_to_none=True)
    out2, _ = m(x, h0)
    if cfg["loss"] == "mse":
        loss = F.mse_loss(out2, torch.from_numpy(golden["target"]))
    else:
        loss = out2.sum()
    loss.backward()
    for n, p in m.named_parameters():
        ref = golden["grad." + n]
        scale = max(1.0, float(np.abs(ref).max()))
        assert np.abs(p.grad.numpy() - ref).max() <= 1e-5 * scale, n


@pytest.fixture
def ltc_model():
    return TrueLiquidTimeConstant(input_dim=10, hidden_dim=8, dt=0.1, ode_unfolds=6,
                                  sparsity=0.5, sensory_sparsity=0.5)


def test_constructor_params(ltc_model):
    H, D = ltc_model.hidden_dim, ltc_model.input_dim
    for name in ("gleak", "vleak", "cm"):
        assert getattr(ltc_model, name).shape == (H,)
    for name in ("w", "mu", "sigma", "erev", "sparsity_mask"):
        assert getattr(ltc_model, name).shape == (H, H)
    for name in ("sensory_w", "sensory_mu", "sensory_sigma", "sensory_erev",
                 "sensory_sparsity_mask"):
        assert getattr(ltc_model, name).shape == (D, H)


def test_forward_shapes_and_lstm_api(ltc_model):
    x = torch.randn(2, 5, ltc_model.input_dim)
    out, (h, c) = ltc_model(x)
    assert out.shape == (2, 5, ltc_model.hidden_dim)
    assert h.shape == (2, ltc_model.hidden_dim)
    assert torch.equal(c, h)
    out1, (h1, _) = ltc_model(torch.randn(3, 1, ltc_model.input_dim))
    assert out1.shape == (3, 1, ltc_model.hidden_dim) and h1.shape == (3, ltc_model.hidden_dim)


def test_state_not_clamped(ltc_model):
    ltc_model.vleak.data.fill_(5.0)
    ltc_model.gleak.data.fill_(10.0)
    _, (h, _) = ltc_model(torch.ones(2, 8, ltc_model.input_dim) * 5.0)
    assert torch.isfinite(h).all()
    assert h.abs().max().item() > 1.0


def test_gates_and_positivity(ltc_model):
    v = torch.randn(3, ltc_model.hidden_dim)
    g = torch.sigmoid(ltc_model.sigma * (v.unsqueeze(-1) - ltc_model.mu))
    assert g.shape == (3, 8, 8) and (g >= 0).all() and (g <= 1).all()
    xi = torch.randn(3, ltc_model.input_dim)
    gs = torch.sigmoid(ltc_model.sensory_sigma * (xi.unsqueeze(-1) - ltc_model.sensory_mu))
    assert gs.shape == (3, 10, 8)
    for name in ("w", "cm", "gleak", "sensory_w"):
        assert (F.softplus(getattr(ltc_model, name)) > 0).all()


def test_masks(ltc_model):
    for mask in (ltc_model.sparsity_mask, ltc_model.sensory_sparsity_mask):
        assert ((mask == 0) | (mask == 1)).all()
        assert mask.any(dim=0).all()
    assert abs(ltc_model.sparsity_mask.mean().item() - ltc_model.sparsity) < 0.2
    erev = ltc_model.erev.detach()
    assert (erev > 0).any() and (erev < 0).any()


def test_state_persistence(ltc_model):
    x1 = torch.randn(1, 3, ltc_model.input_dim)
    x2 = torch.randn(1, 3, ltc_model.input_dim)
    _, s1 = ltc_model(x1)
    a, _ = ltc_model(x2, h0=s1)
    b, _ = ltc_model(x2)
    assert not torch.allclose(a, b, atol=1e-6)


def test_gradient_flow(ltc_model):
    out, _ = ltc_model(torch.randn(2, 4, ltc_model.input_dim))
    out.sum().backward()
    for name in ("w", "mu", "sigma", "erev", "sensory_w", "sensory_mu", "sensory_sigma",
                 "sensory_erev", "gleak", "vleak", "cm"):
        g = getattr(ltc_model, name).grad
        assert g is not None and (g != 0).any(), name


def test_compat_shims(ltc_model):
    assert ltc_model.W_rec is ltc_model.w
    with pytest.raises(NotImplementedError):
        ltc_model.fused_euler_step()
    assert TemporalLTC is TrueLiquidTimeConstant


def test_bounded_dynamics_and_unfolds():
    torch.manual_seed(42)
    m1 = TrueLiquidTimeConstant(10, 8, ode_unfolds=1)
    torch.manual_seed(42)
    m6 = TrueLiquidTimeConstant(10, 8, ode_unfolds=6)
    x = torch.randn(1, 3, 10)
    assert not torch.allclose(m1(x)[0], m6(x)[0], atol=1e-4)
    out, _ = m6(torch.ones(1, 20, 10) * 100.0)
    assert torch.isfinite(out).all()


def test_eval_cache_and_train_reset(ltc_model):
    ltc_model.eval()
    x = torch.randn(2, 3, ltc_model.input_dim)
    with torch.no_grad():
        a, _ = ltc_model(x)
    assert ltc_model._cached_transforms is not None
    with torch.no_grad():
        b, _ = ltc_model(x)
    assert torch.equal(a, b)
    ltc_model.train()
    assert ltc_model._cached_transforms is None


def test_input_mapping_buffers():
    m = TrueLiquidTimeConstant(6, 4, input_mapping="linear")
    names = dict(m.named_parameters())
    assert "input_w" in names and "input_b" not in names
    m = TrueLiquidTimeConstant(6, 4, input_mapping="none")
    names = dict(m.named_parameters())
    assert "input_w" not in names and "input_b" not in names


def test_reference_import_surface():
    assert hasattr(ltc, "_HAS_CUDA_KERNELS")
    assert callable(ltc.ltc_cuda_forward)
    for name in ("_HAS_CUDA_KERNELS", "_cuda_module", "LTCCudaForward", "ltc_cuda_forward",
                 "_try_load_cuda_kernels"):
        assert hasattr(ltc_cuda, name)


def test_fused_path_fails_loudly_without_kernels(monkeypatch):
    """With no loaded extension the fused entry raises instead of switching paths."""
    monkeypatch.setattr(ltc_cuda, "_HAS_CUDA_KERNELS", False)
    monkeypatch.setattr(ltc_cuda, "_cuda_module", None)
    monkeypatch.setattr(ltc_cuda, "_LOAD_ERROR", "simulated: library missing")
    with pytest.raises(RuntimeError, match="simulated: library missing"):
        ltc_cuda.require_kernels()
    z = torch.zeros(1)
    with pytest.raises(RuntimeError, match="not loaded"):
        ltc_cuda.LTCCudaForward.apply(*([z] * 13), 6, 1e-8, False)


def test_module_apply_takes_absent_state_to_its_own_checks():
    """The C++ Function receives no initial state as None (a zero state in the library):
    autograd must accept it and the call must reach the extension's own input checks."""
    ext = pytest.importorskip("_ltc_torch")
    x = torch.randn(2, 3, 4)
    lv = ([torch.randn(5, 5)] * 5 + [torch.randn(4, 5)] * 5 + [torch.randn(5)] * 3
          + [torch.randn(4)] * 4)
    for grad in (False, True):
        with torch.set_grad_enabled(grad), pytest.raises(RuntimeError, match="fp32-only"):
            ext.module_apply(x, None, lv, 0.1, 6, 1e-8, 1e-5)


@pytest.mark.parametrize("set_to_none", [True, False])
def test_zero_grad_matches_nn_module(set_to_none):
    """The layer's own zero_grad walks its registries directly; it must leave every
    gradient as nn.Module.zero_grad does, and defer to it for other structures."""
    torch.manual_seed(0)
    a = ltc.TrueLiquidTimeConstant(6, 5)
    b = ltc.TrueLiquidTimeConstant(6, 5)
    b.load_state_dict(a.state_dict())
    x = torch.randn(2, 3, 6)
    for m in (a, b):
        out, _ = m(x)
        out.sum().backward()
    a.zero_grad(set_to_none=set_to_none)
    torch.nn.Module.zero_grad(b, set_to_none=set_to_none)
    for (n, pa), (_, pb) in zip(a.named_parameters(), b.named_parameters()):
        if set_to_none:
            assert pa.grad is None and pb.grad is None, n
        else:
            assert torch.equal(pa.grad, pb.grad) and not pa.grad.any(), n
    # an extra submodule: nn.Module's own walk reaches its parameters too
    a.extra = torch.nn.Linear(2, 2)
    a.extra.weight.grad = torch.ones(2, 2)
    a.zero_grad()
    assert a.extra.weight.grad is None
