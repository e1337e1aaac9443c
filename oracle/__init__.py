"""CPU oracle for the LTC fused ODE-solver path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`ltc-cuda_amd/`)
imports this package. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker or
the timed CPU baseline, never as the thing measured on the GPU.

Modules:
  ltc_oracle   - torch restatement of the reference TorchScript path,
                 the module init (RNG order) and the pre-transforms.
  ltc_analytic - float64 numpy restatement of the closed-form backward,
                 independent of autograd, used to pin the autograd gradients.
"""
