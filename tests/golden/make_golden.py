"""Write golden vectors from the reference implementation (run in the build container only).

The reference's own tests hold no fixtures: every parity check there compares
two live paths (test_ltc_cuda.py:46-287). Two things cannot be pinned by
mathematics alone:
  * the module init, i.e. which tensors a seed produces (RNG consumption order,
    ltc.py:149-231), and
  * the end-to-end composition LayerNorm -> affine -> softplus/mask -> T loop
    under the TorchScript executor (ltc.py:19-106, 249-326), including every
    leaf-parameter gradient autograd produces through it.
So this script imports the reference module on the CPU, from its read-only
tree, and records inputs and outputs as small float32/float64 .npz fixtures.
The reference never travels to the GPU box; only these arrays do.

Usage (build container):  python tests/golden/make_golden.py [REFERENCE_DIR]
"""

from __future__ import annotations

import os
import sys

import numpy as np

sys.dont_write_bytecode = True  # the reference tree is read-only

HERE = os.path.dirname(os.path.abspath(__file__))


def _load_reference(ref_dir):
    sys.path.insert(0, ref_dir)
    import torch  # noqa: F401  (imported before the reference, as it does)
    import ltc as ref_ltc
    return ref_ltc


def _state(m):
    return {k: v.detach().cpu().numpy().copy() for k, v in m.state_dict().items()}


def _grads(m):
    return {n: p.grad.detach().cpu().numpy().copy()
            for n, p in m.named_parameters() if p.grad is not None}


def _case(ref_ltc, torch, name, D, H, seed_model, seed_x, B, T, *, dt=1.0 / 30.0, U=6,
          sparsity=0.5, sensory_sparsity=0.5, input_mapping="affine", h0=False,
          loss="sum", x_scale=1.0):
    """Build a reference module, run forward (no_grad) and forward+backward."""
    torch.manual_seed(seed_model)
    m = ref_ltc.TrueLiquidTimeConstant(D, H, dt=dt, ode_unfolds=U, sparsity=sparsity,
                                       sensory_sparsity=sensory_sparsity,
                                       input_mapping=input_mapping)
    m._force_torchscript = True
    m.train()
    rec = {"state." + k: v for k, v in _state(m).items()}
    torch.manual_seed(seed_x)
    x = torch.randn(B, T, D) * x_scale
    hstate = None
    if h0:
        hstate = (torch.randn(B, H), torch.randn(B, H))
        rec["h0"] = hstate[0].numpy().copy()
    target = torch.randn(B, T, H) if loss == "mse" else None
    rec["x"] = x.numpy().copy()
    with torch.no_grad():
        out, (h, c) = m(x, hstate)
    rec["out"] = out.numpy().copy()
    rec["h"] = h.numpy().copy()
    m.zero_grad(set_to_none=True)
    out2, _ = m(x, hstate)
    if loss == "mse":
        rec["target"] = target.numpy().copy()
        lval = torch.nn.functional.mse_loss(out2, target)
    else:
        lval = out2.sum()
    lval.backward()
    rec.update({"grad." + k: v for k, v in _grads(m).items()})
    rec["meta"] = np.array([D, H, B, T, U, seed_model, seed_x], np.int64)
    rec["meta_f"] = np.array([dt, sparsity, sensory_sparsity, x_scale], np.float64)
    rec["meta_s"] = np.array([input_mapping, loss])
    np.savez_compressed(os.path.join(HERE, f"ref_{name}.npz"), **rec)
    print(f"wrote ref_{name}.npz", {k: v.shape for k, v in rec.items() if k.startswith(('out', 'x'))})


def main():
    ref_dir = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref_ltc = _load_reference(ref_dir)
    import torch
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    # Shapes of the reference's own CUDA-vs-TorchScript tests (test_ltc_cuda.py:27-39, 46-287).
    _case(ref_ltc, torch, "d32h16", 32, 16, 42, 123, 4, 8, h0=True)
    _case(ref_ltc, torch, "d32h16_grad", 32, 16, 42, 202, 2, 4)
    _case(ref_ltc, torch, "d32h17", 32, 17, 42, 808, 4, 4)
    _case(ref_ltc, torch, "d32h33", 32, 33, 42, 909, 2, 4)
    _case(ref_ltc, torch, "d48h24_mse", 48, 24, 47, 11, 3, 6, loss="mse", x_scale=5.0)
    # Spec-test fixture shape (test_ltc_verification.py:12-22), other mappings, dense wiring.
    _case(ref_ltc, torch, "d10h8_dt01", 10, 8, 7, 8, 2, 5, dt=0.1)
    _case(ref_ltc, torch, "d10h8_linear", 10, 8, 9, 10, 2, 3, input_mapping="linear")
    _case(ref_ltc, torch, "d10h8_none_u1", 10, 8, 11, 12, 2, 3, input_mapping="none", U=1)
    _case(ref_ltc, torch, "d16h12_dense", 16, 12, 13, 14, 3, 4, sparsity=1.0,
          sensory_sparsity=1.0)
    # The headline bench shape: B=24 T=8 D=128 H=64, seed 42.
    _case(ref_ltc, torch, "c1", 128, 64, 42, 43, 24, 8)


if __name__ == "__main__":
    main()
