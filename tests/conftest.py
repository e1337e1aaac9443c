"""Shared test setup: import paths, the `gpu` marker and golden-vector loading."""

from __future__ import annotations

import glob
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ltc-cuda_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device and the built libltc_hip.so")


def golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "ref_*.npz")))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    rec = {k: z[k] for k in z.files}
    D, H, B, T, U, seed_model, seed_x = (int(v) for v in rec["meta"])
    dt, sp, ssp, xs = (float(v) for v in rec["meta_f"])
    mapping, loss = (str(v) for v in rec["meta_s"])
    rec["cfg"] = dict(D=D, H=H, B=B, T=T, U=U, seed_model=seed_model, seed_x=seed_x, dt=dt,
                      sparsity=sp, sensory_sparsity=ssp, x_scale=xs, input_mapping=mapping,
                      loss=loss)
    return rec


@pytest.fixture(params=golden_files(), ids=lambda p: os.path.basename(p)[4:-4])
def golden(request):
    return load_golden(request.param)
