"""GPU parity of the per-step entry points (ltc_sensory_fwd/bwd, ltc_ode_unfold_fwd/bwd).

The reference exports these beside its T-loop drivers (csrc/ltc_kernels.cu:675-950,
1308-1311). Each is checked against the float64 oracle halves `sensory_sums` and
`unfolds` (oracle/ltc_oracle.py) on the same seeded inputs, through the C-ABI,
with the reference's bars: forward max-abs 1e-3, gradients allclose(rtol=5e-2,
atol=1e-2), and each gradient's max error <= 2e-3 of its largest entry.
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from oracle import ltc_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-8
U = 6


@pytest.fixture(scope="module", autouse=True)
def _native():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    assert ltc_cuda._HAS_CUDA_KERNELS, f"HIP extension not loaded: {ltc_cuda._LOAD_ERROR}"


def _mod():
    return ltc_cuda._cuda_module


def _params(D, H, seed):
    torch.manual_seed(seed)
    p = O.init_params(D, H, 0.5, 0.5)
    w_pos, w_erev, cm_t, gleak_pos, s_wpos = O.transforms(p, 1.0 / 30.0, U)
    rec = [w_pos, w_erev, p["mu"], p["sigma"]]
    sens = {"mu": p["sensory_mu"], "sigma": p["sensory_sigma"], "erev": p["sensory_erev"],
            "w_pos": s_wpos}
    neuron = [cm_t, gleak_pos, p["vleak"]]
    return rec, sens, neuron


def _close_fwd(got, ref, label):
    err = (got.cpu().double() - ref).abs().max().item()
    assert torch.isfinite(got).all(), label
    assert err <= 1e-3, f"{label}: max-abs {err:.3e}"


def _close_grad(got, ref, label):
    g, r = got.cpu().double(), ref.double()
    err = (g - r).abs().max().item()
    scale = r.abs().max().item()
    assert torch.isfinite(g).all(), f"{label}: non-finite"
    assert torch.allclose(g, r, rtol=5e-2, atol=1e-2), f"{label}: err={err:.3e}"
    assert err <= 2e-3 * scale + 1e-6, f"{label}: err={err:.3e} scale={scale:.3e}"


SENS_SHAPES = [(3, 5, 4), (24, 128, 64), (7, 33, 65), (4, 16, 256), (2, 8, 512), (1, 1, 1),
               (300, 64, 64)]


@pytest.mark.parametrize("shape", SENS_SHAPES, ids=lambda s: "B%dD%dH%d" % s)
@pytest.mark.parametrize("strided", [False, True])
def test_sensory_fwd_and_bwd_match_oracle(shape, strided):
    B, D, H = shape
    _, sens, _ = _params(D, H, seed=B + D + H)
    torch.manual_seed(7)
    xw = torch.randn(B, 2 * D)
    x = xw[:, 0::2] if strided else xw[:, :D].contiguous()
    gn, gd = torch.randn(B, H), torch.randn(B, H)
    xd = xw.to(DEV)[:, 0::2] if strided else x.to(DEV)
    if strided:
        assert xd.stride() == (2 * D, 2)
    order = ("sigma", "mu", "w_pos", "erev")  # reference argument order
    dev_p = [sens[k].to(DEV) for k in order]
    wn, wd = _mod().ltc_sensory_fwd(xd, *dev_p)
    grads = _mod().ltc_sensory_bwd(gn.to(DEV), gd.to(DEV), xd, *dev_p)
    torch.cuda.synchronize()

    leaves = {k: v.double().requires_grad_(True) for k, v in sens.items()}
    xl = x.double().requires_grad_(True)
    rn, rd = O.sensory_sums(xl, leaves["mu"], leaves["sigma"], leaves["erev"], leaves["w_pos"])
    _close_fwd(wn, rn.detach(), "w_num_sensory")
    _close_fwd(wd, rd.detach(), "w_den_sensory")
    torch.autograd.backward([rn, rd], [gn.double(), gd.double()])
    refs = [xl.grad] + [leaves[k].grad for k in order]
    for name, g, r in zip(("inputs",) + order, grads, refs):
        _close_grad(g, r, f"grad {name}")


UNFOLD_SHAPES = [(2, 4), (24, 64), (5, 65), (3, 192), (4, 256), (9, 320), (2, 512), (1, 1),
                 (600, 16), (1100, 24)]


@pytest.mark.parametrize("shape", UNFOLD_SHAPES, ids=lambda s: "B%dH%d" % s)
def test_ode_unfold_fwd_and_bwd_match_oracle(shape):
    B, H = shape
    rec, _, neuron = _params(8, H, seed=B * 3 + H)
    torch.manual_seed(11)
    h0 = torch.randn(B, H) * 0.2
    sn, sd = torch.rand(B, H) * 2.0 - 1.0, torch.rand(B, H) * 2.0
    g_out = torch.randn(B, H)
    dev = [t.to(DEV) for t in [h0] + rec + [sn, sd] + neuron]
    state_new, vbuf = _mod().ltc_ode_unfold_fwd(*dev, U, EPS, True)
    grads = _mod().ltc_ode_unfold_bwd(vbuf, *dev[1:], g_out.to(DEV), U, EPS)
    torch.cuda.synchronize()
    assert vbuf.shape == (U, B, H)

    lv = [t.double().requires_grad_(True) for t in [h0] + rec + [sn, sd] + neuron]
    v, pre = O.unfolds(*lv, U, EPS)
    _close_fwd(state_new, v.detach(), "state_out")
    for k in range(U):
        _close_fwd(vbuf[k], pre[k].detach(), f"v_buffer[{k}]")
    v.backward(g_out.double())
    # reference output order: grad_v, grad_w_num, grad_w_den, 4 recurrent, 3 neuron
    refs = [lv[0].grad, lv[5].grad, lv[6].grad] + [t.grad for t in lv[1:5]] + \
        [t.grad for t in lv[7:]]
    names = ("v", "w_num_sensory", "w_den_sensory", "w_pos", "w_erev", "mu", "sigma", "cm_t",
             "gleak_pos", "vleak")
    for name, g, r in zip(names, grads, refs):
        _close_grad(g, r, f"grad {name}")


def test_ode_unfold_fwd_without_saving_and_empty_batch():
    rec, _, neuron = _params(8, 33, seed=1)
    h0 = torch.randn(4, 33) * 0.2
    sn, sd = torch.rand(4, 33), torch.rand(4, 33)
    dev = [t.to(DEV) for t in [h0] + rec + [sn, sd] + neuron]
    a, vb = _mod().ltc_ode_unfold_fwd(*dev, U, EPS, False)
    b, _ = _mod().ltc_ode_unfold_fwd(*dev, U, EPS, True)
    torch.cuda.synchronize()
    assert vb is None and torch.equal(a, b)
    z = [t[:0] if t.dim() == 2 and t.shape[0] == 4 else t for t in dev]
    e, ve = _mod().ltc_ode_unfold_fwd(*z, U, EPS, True)
    assert e.shape == (0, 33) and ve.shape == (U, 0, 33)
    x0 = torch.zeros(0, 8, device=DEV)
    _, sens, _ = _params(8, 33, seed=1)
    wn, wd = _mod().ltc_sensory_fwd(x0, *[sens[k].to(DEV) for k in ("sigma", "mu", "w_pos",
                                                                   "erev")])
    assert wn.shape == (0, 33) and wd.shape == (0, 33)


def test_step_entry_points_compose_to_the_full_forward():
    """A Python T loop over ltc_sensory_fwd + ltc_ode_unfold_fwd (the loop the
    reference's per-step exports served) reproduces ltc_full_forward."""
    B, T, D, H = 6, 5, 32, 48
    rec, sens, neuron = _params(D, H, seed=5)
    torch.manual_seed(2)
    x = torch.randn(B, T, D, device=DEV)
    h = (torch.randn(B, H) * 0.2).to(DEV)
    rec_d, neuron_d = [t.to(DEV) for t in rec], [t.to(DEV) for t in neuron]
    sens_d = {k: v.to(DEV) for k, v in sens.items()}
    full_out, full_h = _mod().ltc_full_forward(
        x, h, *rec_d, sens_d["mu"], sens_d["sigma"], sens_d["erev"], sens_d["w_pos"],
        *neuron_d, U, EPS, False)
    outs = []
    for t in range(T):
        wn, wd = _mod().ltc_sensory_fwd(x[:, t, :], sens_d["sigma"], sens_d["mu"],
                                        sens_d["w_pos"], sens_d["erev"])
        h, _ = _mod().ltc_ode_unfold_fwd(h, *rec_d, wn, wd, *neuron_d, U, EPS, False)
        outs.append(h)
    torch.cuda.synchronize()
    step_out = torch.stack(outs, dim=1)
    assert (step_out - full_out).abs().max().item() <= 1e-5
    assert (h - full_h).abs().max().item() <= 1e-5
