"""The no-allocation forward (ltc_full_forward_noalloc) against ltc_full_forward.

Both run the same kernels; the no-allocation entry point takes its scratch
from a static per-device array instead of the caller's workspace. Its outputs
must equal the workspace entry point's bit for bit, call after call, whatever
an earlier call left in the shared array.
"""

from __future__ import annotations

import ctypes
import os

import pytest
import torch

import ltc_cuda
from oracle import ltc_oracle as O

DEV = "cuda:0"
EPS = 1e-8
U = 6
SCRATCH_BYTES = 64 * 1024 * 1024  # LTC_NOALLOC_SCRATCH_BYTES in include/ltc_capi.h


def _capi():
    if not os.path.isfile(ltc_cuda.LIB_PATH):
        pytest.skip("libltc_hip.so not built")
    return ltc_cuda.load_capi(ltc_cuda.LIB_PATH)


def _boundary(B, T, D, H, seed):
    torch.manual_seed(seed)
    p = O.init_params(D, H, 0.5, 0.5)
    w_pos, w_erev, cm_t, gleak_pos, s_wpos = O.transforms(p, 1.0 / 30.0, U)
    x = torch.randn(B, T, D)
    h0 = 0.2 * torch.randn(B, H)
    return [x, h0, w_pos, w_erev, p["mu"], p["sigma"], p["sensory_mu"], p["sensory_sigma"],
            p["sensory_erev"], s_wpos, cm_t, gleak_pos, p["vleak"]]


def _run(capi, args, save, noalloc):
    """One forward through the C-ABI; returns (out, h, saved or None)."""
    B, T, D = args[0].shape
    H = args[1].shape[1]
    dev = [a.to(DEV).contiguous() for a in args]
    f32 = dict(device=DEV, dtype=torch.float32)
    out = torch.full((B, T, H), float("nan"), **f32)
    h = torch.full((B, H), float("nan"), **f32)
    saved = torch.full((capi.lib.ltc_saved_floats(B, T, H, U),), float("nan"), **f32) if save else None
    x = dev[0]
    sx = x.stride()
    stream = torch.cuda.current_stream().cuda_stream
    common = [x.data_ptr(), sx[0], sx[1], sx[2], dev[1].data_ptr()] + [t.data_ptr() for t in dev[2:]]
    common += [B, T, D, H, U, EPS, 1 if save else 0, out.data_ptr(), h.data_ptr(),
               None if saved is None else saved.data_ptr()]
    if noalloc:
        rc = capi.lib.ltc_full_forward_noalloc(*common, stream)
        what = "ltc_full_forward_noalloc"
    else:
        need = capi.lib.ltc_fwd_workspace_bytes(B, T, D, H, U)
        ws = torch.empty(need + 256, dtype=torch.uint8, device=DEV)
        rc = capi.lib.ltc_full_forward(*common, (ws.data_ptr() + 255) & ~255, need, stream)
        what = "ltc_full_forward"
    capi.check(rc, what)
    torch.cuda.synchronize()
    return out, h, saved


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """Validation happens before any device call, so this runs without a GPU."""
    capi = _capi()
    B, T, D, H = 1024, 64, 64, 256
    assert capi.lib.ltc_fwd_workspace_bytes(B, T, D, H, U) > SCRATCH_BYTES
    rc = capi.lib.ltc_full_forward_noalloc(1, 0, 0, 0, 1, *([1] * 11), B, T, D, H, U, EPS, 0,
                                           1, 1, None, None)
    assert rc == 2 and "scratch" in capi.last_error()
    rc = capi.lib.ltc_full_forward_noalloc(1, 0, 0, 0, 1, *([1] * 11), 2, 3, 4, 0, U, EPS, 0,
                                           1, 1, None, None)
    assert rc == 1 and "H >= 1" in capi.last_error()


# C1 first, then a smaller input, then the cluster path (exchange words in the
# scratch array), then the C1 shape again over what the others left behind.
SEQUENCE = [((24, 8, 128, 64), True), ((5, 3, 32, 17), False), ((8, 2, 16, 256), True),
            ((24, 8, 128, 64), False)]


@pytest.mark.gpu
def test_noalloc_forward_equals_workspace_forward():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    capi = _capi()
    assert capi.lib.ltc_device_count() >= 1
    for i, (shape, save) in enumerate(SEQUENCE):
        B, T, D, H = shape
        print(f"no-alloc call {i}: B={B} T={T} D={D} H={H} save={save}", flush=True)
        assert capi.lib.ltc_fwd_workspace_bytes(B, T, D, H, U) <= SCRATCH_BYTES
        args = _boundary(B, T, D, H, seed=100 + i)
        ref = _run(capi, args, save, noalloc=False)
        got = _run(capi, args, save, noalloc=True)
        for a, b in zip(got, ref):
            if b is None:
                assert a is None
                continue
            assert torch.isfinite(a).all()
            assert torch.equal(a, b)
        # and the oracle, at the forward's bar (max-abs 1e-3)
        with torch.no_grad():
            r_out, r_h = O.forward_loop(*[a.double() for a in args], U, EPS)
        assert (got[0].cpu().double() - r_out).abs().max().item() <= 1e-3
        assert (got[1].cpu().double() - r_h).abs().max().item() <= 1e-3
