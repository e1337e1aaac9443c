"""Where a non-finite input goes, on ltc_full_forward.

The reference multiplies every synapse's gate by its weight, masked or not
(ltc.py:44-47, 53-58), so a NaN at one input reaches every neuron through
0 * NaN = NaN. This library's compacted kernels skip the synapses whose
weights are zero, on purpose:

- the sensory launch of every ltc_full_forward walks only the inputs with a
  nonzero sensory weight, so a NaN input reaches exactly the neurons that
  input is connected to;
- plans that read a compacted recurrent image (plan field cmp_fwd) skip the
  recurrent synapses with w_pos = w_erev = 0, so a NaN state reaches exactly
  the neurons it has a nonzero recurrent weight to, per unfold;
- plans with dense recurrent images (cmp_fwd = 0) evaluate every recurrent
  synapse, as the reference does, and a NaN state reaches every neuron.

These tests pin that behaviour exactly, and check that every finite entry
equals the float64 oracle run with the offending value replaced by zero (which
the skipped synapses multiply by an exact zero weight), within the forward
bar of 1e-3.
"""

from __future__ import annotations

import pytest
import torch

import ltc_cuda
from _gpu_common import DEV, _native, boundary, gpu_forward, oracle_forward  # noqa: F401

pytestmark = pytest.mark.gpu


def _finite_match(got, ref, label):
    fin = torch.isfinite(got)
    err = (got[fin].double() - ref[fin]).abs().max().item()
    print(f"{label}: finite-entry err {err:.2e}", flush=True)
    assert err <= 1e-3, (label, err)


@pytest.mark.parametrize("shape", [(3, 1, 70, 40), (3, 1, 130, 300)],
                         ids=["H40", "H300"])
def test_nan_input_reaches_only_neurons_it_is_connected_to(shape):
    B, T, D, H = shape
    args = boundary(B, T, D, H, seed=11)
    s_wpos = args[9]
    d0 = 5
    connected = s_wpos[d0] != 0
    assert bool(connected.any()) and bool((~connected).any())
    x = args[0].clone()
    x[1, 0, d0] = float("nan")
    _, res = gpu_forward([x] + args[1:], U=1)
    out = res[0].cpu()
    nan = torch.isnan(out[1, 0])
    print(f"{shape}: {int(nan.sum())} of {H} neurons NaN, "
          f"{int(connected.sum())} connected", flush=True)
    assert torch.equal(nan, connected)
    assert torch.isfinite(out[0]).all() and torch.isfinite(out[2]).all()
    x0 = args[0].clone()
    x0[1, 0, d0] = 0.0
    r_out, _ = oracle_forward([x0] + args[1:], U=1)
    _finite_match(out, r_out, f"nan input {shape}")


def test_nan_state_follows_nonzero_recurrent_weights_in_compacted_plans():
    B, T, D, H = 2, 1, 40, 64
    plan = ltc_cuda._cuda_module.capi.plan(B, T, D, H, 1)
    assert plan["cmp_fwd"] == 1, plan
    args = boundary(B, T, D, H, seed=12)
    w_pos, w_erev = args[2], args[3]
    i0 = 3
    reach = (w_pos[i0] != 0) | (w_erev[i0] != 0)
    reach[i0] = True  # the neuron's own leak term C * v
    assert bool((~reach).any())
    h0 = args[1].clone()
    h0[0, i0] = float("nan")
    _, res = gpu_forward([args[0], h0] + args[2:], U=1)
    out = res[0].cpu()
    assert torch.equal(torch.isnan(out[0, 0]), reach)
    assert torch.isfinite(out[1]).all()
    h00 = args[1].clone()
    h00[0, i0] = 0.0
    r_out, _ = oracle_forward([args[0], h00] + args[2:], U=1)
    # the unreached neurons do not depend on v_i0 at all
    got = out[0, 0][~reach].double()
    ref = r_out[0, 0][~reach]
    assert (got - ref).abs().max().item() <= 1e-3


def test_nan_state_reaches_every_neuron_in_dense_plans():
    B, T, D, H = 2, 1, 40, 320
    plan = ltc_cuda._cuda_module.capi.plan(B, T, D, H, 1)
    assert plan["cmp_fwd"] == 0, plan
    args = boundary(B, T, D, H, seed=13)
    h0 = args[1].clone()
    h0[0, 7] = float("nan")
    _, res = gpu_forward([args[0], h0] + args[2:], U=1)
    out = res[0].cpu()
    assert torch.isnan(out[0]).all()
    assert torch.isfinite(out[1]).all()
