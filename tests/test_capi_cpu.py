"""C-ABI library checks that need no GPU: it loads, exports what the header
declares, reports sizes, and rejects bad arguments before touching a device."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (loads torch's HIP runtime first, as in production)

import ltc_cuda

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ltc_capi.h")

pytestmark = pytest.mark.skipif(not os.path.isfile(ltc_cuda.LIB_PATH),
                                reason="libltc_hip.so not built (python ltc-cuda_amd/build.py)")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_ ]+\**\s*\**(ltc_\w+)\s*\(", text,
                                 flags=re.M)))


@pytest.fixture(scope="module")
def capi():
    return ltc_cuda.load_capi(ltc_cuda.LIB_PATH)


def test_header_declares_the_boundary():
    names = _declared_functions()
    for must in ("ltc_full_forward", "ltc_full_backward", "ltc_fwd_workspace_bytes",
                 "ltc_bwd_workspace_bytes", "ltc_saved_floats", "ltc_last_error",
                 "ltc_abi_version", "ltc_device_count"):
        assert must in names
    assert set(names) == set(ltc_cuda.CApi.SYMBOLS)


def test_library_exports_every_declared_symbol(capi):
    for name in _declared_functions():
        assert hasattr(capi.lib, name), name
        assert ctypes.cast(getattr(capi.lib, name), ctypes.c_void_p).value


def test_abi_version(capi):
    assert capi.lib.ltc_abi_version() == ltc_cuda.ABI_VERSION


def test_sizes(capi):
    lib = capi.lib
    # saved = (T*U + 1) * B * Hp + T*U*B*Hp floats, Hp = H rounded up to 64
    assert lib.ltc_saved_floats(24, 8, 64, 6) == (8 * 6 + 1) * 24 * 64 + 8 * 6 * 24 * 64
    assert lib.ltc_saved_floats(2, 3, 65, 1) == (3 + 1) * 2 * 128 + 3 * 2 * 128
    a = lib.ltc_fwd_workspace_bytes(24, 8, 128, 64, 6)
    b = lib.ltc_fwd_workspace_bytes(48, 8, 128, 64, 6)
    assert 0 < a < b and a % 256 == 0
    assert lib.ltc_bwd_workspace_bytes(24, 8, 128, 64, 6) > 0
    assert lib.ltc_fwd_workspace_bytes(1, 1, 1, 0, 6) == -1
    assert lib.ltc_fwd_workspace_bytes(1, 1, 1, 5000, 6) == -1
    assert lib.ltc_fwd_workspace_bytes(1, 1, 1, 2000, 6) > 0  # clusters above H = 1024
    assert lib.ltc_bwd_workspace_bytes(1, 1, 1, 8, 0) == -1


def _fwd_call(capi, **over):
    args = dict(x=1, s=(0, 0, 0), state=1, params=[1] * 11, B=2, T=3, D=4, H=5, U=6,
                eps=1e-8, save=0, out=1, h=1, saved=None, ws=256, wsb=1 << 30, stream=None)
    args.update(over)
    return capi.lib.ltc_full_forward(
        args["x"], *args["s"], args["state"], *args["params"], args["B"], args["T"],
        args["D"], args["H"], args["U"], args["eps"], args["save"], args["out"], args["h"],
        args["saved"], args["ws"], args["wsb"], args["stream"])


def test_forward_rejects_bad_arguments_before_launch(capi):
    # Fake non-NULL addresses: every case must fail validation, so nothing runs.
    assert _fwd_call(capi, H=0) == 1 and "H >= 1" in capi.last_error()
    assert _fwd_call(capi, U=0) == 1 and "ode_unfolds" in capi.last_error()
    assert _fwd_call(capi, H=4097) == 2 and "exceeds" in capi.last_error()
    assert _fwd_call(capi, params=[1] * 10 + [None]) == 1
    assert _fwd_call(capi, save=1, saved=None) == 1 and "saved" in capi.last_error()
    assert _fwd_call(capi, wsb=16) == 1 and "workspace too small" in capi.last_error()
    assert _fwd_call(capi, ws=256 + 8) == 1 and "aligned" in capi.last_error()
    assert _fwd_call(capi, x=None) == 1


def test_backward_rejects_bad_arguments_before_launch(capi):
    lib = capi.lib
    p = [1] * 11
    g = [1] * 13
    rc = lib.ltc_full_backward(1, 0, 0, 0, *p, 1, 1, 0, 0, 0, None, 2, 3, 4, 5, 0, 1e-8,
                               *g, 256, 1 << 30, None)
    assert rc == 1 and "ode_unfolds" in capi.last_error()
    rc = lib.ltc_full_backward(1, 0, 0, 0, *p, None, 1, 0, 0, 0, None, 2, 3, 4, 5, 6, 1e-8,
                               *g, 256, 1 << 30, None)
    assert rc == 1 and "NULL" in capi.last_error()
    rc = lib.ltc_full_backward(1, 0, 0, 0, *p, 1, 1, 0, 0, 0, None, 2, 3, 4, 5, 6, 1e-8,
                               *g, 256, 100, None)
    assert rc == 1 and "workspace" in capi.last_error()


def test_step_entry_point_sizes(capi):
    lib = capi.lib
    for fn in (lib.ltc_sensory_fwd_workspace_bytes, lib.ltc_sensory_bwd_workspace_bytes):
        a, b = fn(24, 128, 64), fn(48, 128, 64)
        assert 0 < a < b and a % 256 == 0
        assert fn(1, 0, 8) == -1 and fn(1, 8, 0) == -1 and fn(-1, 8, 8) == -1
        assert fn(1, 8, 5000) == -1 and fn(1, 8, 2000) > 0
    for fn in (lib.ltc_ode_unfold_fwd_workspace_bytes, lib.ltc_ode_unfold_bwd_workspace_bytes):
        a, b = fn(24, 64, 6), fn(48, 64, 6)
        assert 0 < a < b and a % 256 == 0
        assert fn(1, 8, 0) == -1 and fn(1, 0, 6) == -1 and fn(1, 5000, 6) == -1
    # the backward also recomputes the forward, so it needs more
    assert lib.ltc_ode_unfold_bwd_workspace_bytes(24, 64, 6) > \
        lib.ltc_ode_unfold_fwd_workspace_bytes(24, 64, 6)


def test_step_entry_points_reject_bad_arguments_before_launch(capi):
    """Fake non-NULL addresses: every case fails validation, so nothing runs."""
    lib = capi.lib
    big = 1 << 30
    # ltc_sensory_fwd(inputs, sib, sid, sigma, mu, w_pos, erev, B, D, H, wn, wd, ws, wsb, s)
    assert lib.ltc_sensory_fwd(1, 4, 1, 1, 1, 1, 1, 2, 0, 5, 1, 1, 256, big, None) == 1
    assert lib.ltc_sensory_fwd(1, 4, 1, 1, None, 1, 1, 2, 4, 5, 1, 1, 256, big, None) == 1
    assert "NULL" in capi.last_error()
    assert lib.ltc_sensory_fwd(1, 4, 1, 1, 1, 1, 1, 2, 4, 5, None, 1, 256, big, None) == 1
    assert lib.ltc_sensory_fwd(1, 4, 1, 1, 1, 1, 1, 2, 4, 5, 1, 1, 256, 64, None) == 1
    assert "workspace too small" in capi.last_error()
    assert lib.ltc_sensory_fwd(1, 4, 1, 1, 1, 1, 1, 2, 4, 5, 1, 1, 264, big, None) == 1
    assert "aligned" in capi.last_error()
    # ltc_sensory_bwd(gn, gd, inputs, sib, sid, sigma, mu, w_pos, erev, B, D, H, 5 grads, ...)
    assert lib.ltc_sensory_bwd(1, 1, 1, 4, 1, 1, 1, 1, 1, 2, 4, 5, 1, 1, 1, None, 1,
                               256, big, None) == 1
    assert "gradient output" in capi.last_error()
    assert lib.ltc_sensory_bwd(1, 1, 1, 4, 1, 1, 1, 1, 1, 2, 4, 5, 1, 1, 1, 1, 1,
                               256, 16, None) == 1
    # ltc_ode_unfold_fwd(state, 9 tensors, B, H, U, eps, save, out, vbuf, ws, wsb, s)
    t9 = [1] * 9
    assert lib.ltc_ode_unfold_fwd(1, *t9, 2, 5, 0, 1e-8, 0, 1, None, 256, big, None) == 1
    assert "ode_unfolds" in capi.last_error()
    assert lib.ltc_ode_unfold_fwd(1, *t9, 2, 5, 6, 1e-8, 1, 1, None, 256, big, None) == 1
    assert "v_buffer" in capi.last_error()
    assert lib.ltc_ode_unfold_fwd(1, *t9, 2, 4097, 6, 1e-8, 0, 1, None, 256, big, None) == 2
    assert lib.ltc_ode_unfold_fwd(1, *t9, 2, 5, 6, 1e-8, 0, 1, None, 256, 16, None) == 1
    # ltc_ode_unfold_bwd(vbuf, 9 tensors, grad_out, B, H, U, eps, 10 grads, ws, wsb, s)
    g10 = [1] * 10
    assert lib.ltc_ode_unfold_bwd(1, *t9, None, 2, 5, 6, 1e-8, *g10, 256, big, None) == 1
    assert "NULL" in capi.last_error()
    assert lib.ltc_ode_unfold_bwd(1, *t9, 1, 2, 5, 6, 1e-8, *g10[:9], None, 256, big,
                                  None) == 1
    assert lib.ltc_ode_unfold_bwd(1, *t9, 1, 2, 5, 6, 1e-8, *g10, 256, 16, None) == 1
    assert "workspace too small" in capi.last_error()


def test_timing_surface(capi):
    n = capi.lib.ltc_kernel_count()
    names = [capi.lib.ltc_kernel_name(k).decode() for k in range(n)]
    assert "ltc_ode_fwd" in names and "ltc_ode_bwd" in names
    assert capi.lib.ltc_kernel_name(n) == b""


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the GPU-less host")
def test_no_device_reported_without_gpu(capi):
    assert capi.lib.ltc_device_count() == 0
    assert not ltc_cuda._HAS_CUDA_KERNELS
    assert ltc_cuda._LOAD_ERROR


def _max_threads(nb):
    # Mirror of ode_max_threads() in ltc-cuda_amd/csrc/ltc_internal.h.
    return 1024 if nb <= 1 else (512 if nb <= 4 else 256)


SHAPES = [(B, T, D, H, U) for B in (1, 2, 24, 255, 256, 257, 511, 1024, 4096, 5000)
          for (D, H) in ((1, 1), (5, 4), (128, 64), (32, 65), (128, 128), (7, 192), (256, 256),
                         (512, 512), (64, 1000), (3, 1024), (16, 320), (16, 200), (40, 1100),
                         (24, 2048), (16, 4096))
          for (T, U) in ((8, 6), (1, 1))]


@pytest.mark.parametrize("shape", SHAPES + [(24, 8, 128, 64, 6), (4096, 4, 64, 64, 6),
                                                  (256, 64, 256, 256, 6), (128, 32, 512, 512, 6),
                                                  (32, 16, 128, 128, 6)])
def test_launch_plan_fits_the_hardware_limits(capi, shape):
    """Every launch the plan makes fits the kernels' compiled assumptions."""
    B, T, D, H, U = shape
    p = capi.plan(B, T, D, H, U)
    assert p["Hp"] % 64 == 0 and p["Hp"] >= H and p["Hp"] - H < 64
    assert p["Dp"] % 64 == 0 and p["Dp"] >= D and p["Dp"] - D < 64
    if p["CP"] > 0:
        # cluster forward: state rows and partials (at most 60 KiB), plus the
        # compacted form's slot table (Hp = 256, 16 rows per thread)
        Hp, NB, KS = p["Hp"], p["NB"], p["KS"]
        base = NB * Hp * 4 + KS * NB * 64 * 8
        assert base <= 60 * 1024
        # plus the balanced lane order's scratch (an int per thread, 17 per wave)
        table = (64 * KS * 16 * 4 + 64 * KS * 4 + KS * 17 * 4
                 if (Hp == 256 and KS == 16 and p["RC"] == 16) else 0)
        assert p["lds_fwd"] == base + table <= 159 * 1024
    else:
        # state rows and partials under 64 KiB; with register-resident operands
        # (RC of 4, 8 or 16, not the single-row kernel) plus the compacted
        # image's slot table, one int per slot per thread
        Hp, NB, KS, RC = p["Hp"], p["NB"], p["KS"], p["RC"]
        base = NB * Hp * 4 + KS * NB * Hp * 8
        assert base <= 65536
        if NB == 1 and Hp == 128 and KS == 8 and RC == 16:
            # the wave-owned single-row forward: the state by unfold parity and
            # 32 staged steps of sensory sums
            assert p["lds_fwd"] == 2 * Hp * 4 + 2 * 32 * Hp * 4
        elif not (NB == 1 and Hp == 64):
            # the slot table, and the balanced lane order's scratch (an int per
            # thread and 17 per wave)
            thr = Hp * KS
            table = thr * RC * 4 + thr * 4 + thr // 64 * 17 * 4 if RC in (4, 8, 16) else 0
            assert p["lds_fwd"] == base + table <= 159 * 1024
    # the cluster chain may use up to one CU's LDS (160 KiB on MI355X, less 1 KiB);
    # the single-workgroup chain its partials under 64 KiB, or with FUSE one padded
    # [Hp][Hp+1] plane for the transposed gradient stores (four in the single-row
    # chain)
    if p["CP"] > 0:
        assert p["lds_bwd"] <= 159 * 1024
    else:
        Hp, NB, KSB = p["Hp"], p["NB"], p["KSB"]
        base = NB * Hp * 8 + KSB * NB * Hp * 4
        assert base <= 65536
        if not p["fuse"] and p["RCB"] in (4, 8, 16) and not (NB == 1 and Hp == 64):
            # the unfused chain's compacted image: its slot table
            base += Hp * KSB * p["RCB"] * 4
        if NB == 1 and Hp == 64:
            # single-row kernels: two partial buffers and every wave's own copy
            # of the row state (forward) or of alpha/beta (chain); the
            # wave-owned forms (forward RC = 16, fused chain RCB = 8) also
            # stage 32 steps of sensory sums (forward) or 48 unfolds of saved
            # v, 1/den and dL/dout rows (chain) in LDS
            row_b = 2 * KSB * Hp * 4 + KSB * Hp * 8
            if p["fuse"] and p["RCB"] == 8:
                row_b = max(row_b, 2 * Hp * 8 + (3 * 48 + 1) * Hp * 4)
            base = max(base, row_b)
            row_f = 2 * p["KS"] * Hp * 8 + p["KS"] * Hp * 4
            if p["RC"] == 16:
                row_f = max(row_f, 2 * Hp * 4 + 2 * 32 * Hp * 4)
            assert p["lds_fwd"] == max(Hp * 4 + p["KS"] * Hp * 8, row_f)
        planes = 4 if (NB == 1 and Hp == 64) else 1
        plane = planes * Hp * (Hp + 1) * 4 if p["fuse"] else 0
        # the module backward's sensory companions in the chain launch (Hp = 64
        # or 128, one row per workgroup, Dp <= 128, B <= 64): operands of the
        # second 64-input block in LDS, the step's row, per-wave sums, a flag
        comp = 0
        if p["module_row_bwd_fused"] or (p["module_row128_rec_fused"] and p["Dp"] <= 128):
            DC = p["Dp"] // 64
            comp = (DC - 1) * 8 * 8 * 64 * 16 + 64 * 8 + 9 * 64 * DC * 4 + 16
        if NB == 1 and Hp == 128 and not p["fuse"] and KSB == 8 and p["RCB"] == 16:
            # the unfused wave-owned single-row chain: alpha/beta by parity and
            # 48 unfolds of staged v, 1/den and dL/dout rows
            chain = 2 * Hp * 8 + (3 * 48 + 1) * Hp * 4
        else:
            chain = max(base, plane)
        assert p["lds_bwd"] == max(chain, comp) <= 159 * 1024
    assert 1 <= p["NRC"] <= 64
    if p["CP"] > 0:
        # Cluster path: CP members of 64 columns each, the whole grid resident
        # at once (one 1024-thread workgroup per CU at most; 256 CUs without a
        # device), and every member finishes at most one row per thread.
        assert p["Hp"] >= 256 and p["CP"] == p["Hp"] // 64
        assert p["NB"] in (1, 2, 4, 8)
        assert p["ode_workgroups"] == p["NCL"] * p["CP"] <= 256
        # one launch covers the batch, or (Hp > 1024 only) each launch takes the
        # next NCL * NB rows
        L = p["launches_fwd"]
        assert L == p["launches_bwd"] and L == -(-B // (p["NCL"] * p["NB"]))
        if p["Hp"] <= 1024:
            assert L == 1 and p["NCL"] == -(-B // p["NB"])
        else:
            assert p["NCL"] == min(-(-B // p["NB"]), 256 // p["CP"]) and not p["fuse"]
        assert p["KS"] in (8, 16) and p["KS"] >= p["NB"]
        assert p["KS"] * p["RC"] == p["Hp"] and p["RC"] % 8 == 0
        assert p["threads"] == 64 * p["KS"] <= 1024
        assert p["ode_workgroups_bwd"] <= 256 and p["NBB"] in (1, 2, 4, 8)
        assert p["ode_workgroups_bwd"] == p["CPB"] * min(-(-B // p["NBB"]), 256 // p["CPB"])
        assert p["KSB"] >= p["NBB"]
        if p["fuse"]:
            # Hp = 256 / 512 chain: Hp/32 members of 32 columns, 512 threads,
            # Hp/16 synapses per thread, one partial per cluster.
            assert p["Hp"] in (256, 512) and p["CPB"] == p["Hp"] // 32
            assert p["KSB"] == 16 and p["RCB"] == p["Hp"] // 16
            assert p["threads_bwd"] == 512
            assert p["NCH"] == p["ode_workgroups_bwd"] // p["CPB"]
        else:
            assert (p["CPB"], p["NBB"], p["KSB"], p["RCB"]) == (p["CP"], p["NB"], p["KS"], p["RC"])
            assert p["threads_bwd"] == 64 * p["KSB"] and 1 <= p["NCH"] <= 64
        return
    assert p["NB"] in (1, 2, 4, 8, 16)
    assert p["KS"] >= 1 and p["KS"] * p["RC"] == p["Hp"] and p["RC"] % 4 == 0
    assert p["threads"] == p["Hp"] * p["KS"] <= _max_threads(p["NB"])
    assert p["KSB"] >= 1 and p["KSB"] * p["RCB"] == p["Hp"] and p["RCB"] % 4 == 0
    assert p["threads_bwd"] == p["Hp"] * p["KSB"] <= _max_threads(p["NB"])
    # rows finished per thread fit the kernel's compile-time per-row registers
    owned = p["NB"] if p["NB"] <= 2 else p["NB"] // 4
    assert -(-p["NB"] // p["KS"]) <= owned and -(-p["NB"] // p["KSB"]) <= owned
    if p["fuse"]:
        # one partial per chain workgroup; operands and accumulators in registers
        assert p["RCB"] in (4, 8, 16) and p["NCH"] == p["ode_workgroups"]
        if p["NB"] == 1 and p["Hp"] == 64:  # the single-row chain: 8 waves of 8 synapses
            assert (p["KSB"], p["RCB"]) == (8, 8)
        else:
            assert (p["NB"], p["RCB"]) in ((4, 4), (4, 8), (8, 4), (8, 8), (16, 4))
    else:
        assert 1 <= p["NCH"] <= 64
    assert p["ode_workgroups"] * p["NB"] >= B > (p["ode_workgroups"] - 1) * p["NB"] or B == 0


def test_cluster_path_is_planned_for_the_large_configurations(capi):
    """C3 and C4 run as clusters that fill the 256 CUs with 4 rows per member."""
    c3 = capi.plan(256, 64, 256, 256, 6)
    assert (c3["CP"], c3["NB"], c3["NCL"], c3["RC"]) == (4, 4, 64, 16)
    assert (c3["fuse"], c3["CPB"], c3["NBB"], c3["NCH"]) == (1, 8, 8, 32)
    c4 = capi.plan(128, 32, 512, 512, 6)
    assert (c4["CP"], c4["NB"], c4["NCL"], c4["RC"]) == (8, 4, 32, 32)
    assert (c4["fuse"], c4["CPB"], c4["NBB"], c4["NCH"], c4["RCB"]) == (1, 16, 8, 16, 32)
    assert capi.plan(24, 8, 128, 64, 6)["CP"] == 0      # C1: one workgroup per row
    assert capi.plan(4096, 4, 64, 64, 6)["CP"] == 0     # C5


@pytest.mark.parametrize("shape,lds", [
    # D = 100, H = 120: the Hp = 128 chain's staging (76288 B) beats the
    # sensory companion's (DC = 2: 70672 B)
    ((6, 3, 100, 120, 6), 2 * 128 * 8 + (3 * 48 + 1) * 128 * 4),
    ((32, 16, 128, 128, 6), 2 * 128 * 8 + (3 * 48 + 1) * 128 * 4),  # C2
    # C1: the companion's (70672 B) beats the chain's four gradient planes (66560 B)
    ((24, 8, 128, 64, 6), 8 * 8 * 64 * 16 + 64 * 8 + 9 * 128 * 4 + 16),
])
def test_chain_launch_lds_covers_the_companions(capi, shape, lds):
    assert capi.plan(*shape)["lds_bwd"] == lds


@pytest.mark.parametrize("shape,sens_in_prep,row_bwd,rec128", [
    ((24, 8, 128, 64, 6), 1, 1, 0),     # C1: 192 row blocks, companions in the chain launch
    ((3, 5, 40, 60, 6), 1, 1, 0),
    ((8, 16, 128, 128, 6), 1, 0, 1),    # 2 blocks per row: 256 of them
    ((32, 16, 128, 128, 6), 0, 0, 1),   # C2: 1024 row blocks would not fit the chip at once
    ((24, 8, 129, 64, 6), 0, 0, 0),     # D > 128
    ((24, 8, 128, 62, 6), 0, 1, 0),     # H not a multiple of 4
    ((5, 3, 40, 100, 6), 1, 0, 1),      # H below Hp = 128
    ((6, 3, 100, 120, 6), 1, 0, 1),     # two ragged 64-input blocks at Hp = 128
    ((65, 2, 40, 128, 6), 0, 0, 0),     # B > 64
    ((100, 2, 40, 100, 6), 0, 0, 0),    # B > 64 below Hp = 128: rec_grad after the chain
    ((4, 3, 200, 100, 6), 0, 0, 1),     # D > 128: recurrent-gradient companions only
    ((64, 85, 40, 100, 6), 0, 0, 1),    # B*T*U = 32640: the words fit their 64 MiB budget
    ((64, 86, 40, 100, 6), 0, 0, 0),    # B*T*U = 33024: alpha/beta saved for rec_grad
    ((4096, 4, 64, 64, 6), 0, 0, 0),    # C5
    ((256, 64, 256, 256, 6), 0, 0, 0),  # C3
])
def test_module_path_fusion_fields(capi, shape, sens_in_prep, row_bwd, rec128):
    """The plan reports when the module forward forms the sensory sums in its
    parameter-image launch (at most 256 (row, 64-neuron) blocks, D <= 128,
    H % 4 == 0), when the module backward runs the sensory and LayerNorm
    backward inside the chain launch (Hp = 64, one row per workgroup, D <= 128,
    B <= 64), and when it forms the recurrent parameter-gradient sums inside
    the chain launch (Hp = 128, one row per workgroup, B <= 64)."""
    p = capi.plan(*shape)
    got = (p["module_sens_in_prep"], p["module_row_bwd_fused"], p["module_row128_rec_fused"])
    assert got == (sens_in_prep, row_bwd, rec128)


def _ext_path():
    import sysconfig
    return os.path.join(os.path.dirname(ltc_cuda.LIB_PATH),
                        "_ltc_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


@pytest.mark.skipif(not os.path.isfile(_ext_path()), reason="torch extension not built")
def test_torch_extension_shares_the_library_and_validates_on_cpu():
    """The C++ autograd glue links libltc_hip.so by SONAME (one library instance per
    process) and rejects host tensors before it reaches the library."""
    import importlib.machinery
    import importlib.util
    loader = importlib.machinery.ExtensionFileLoader("_ltc_torch", _ext_path())
    spec = importlib.util.spec_from_file_location("_ltc_torch", _ext_path(), loader=loader)
    ext = importlib.util.module_from_spec(spec)
    loader.exec_module(ext)
    assert ext.abi_version() == ltc_cuda.ABI_VERSION
    B, T, D, H = 2, 3, 4, 5
    leaves = [torch.zeros(H, H)] * 5 + [torch.zeros(D, H)] * 5 + [torch.zeros(H)] * 3 \
        + [torch.zeros(D)] * 4
    with pytest.raises(RuntimeError, match="fp32-only"):
        ext.module_apply(torch.zeros(B, T, D), torch.zeros(B, H), leaves, 0.1, 6, 1e-8, 1e-5)
    with pytest.raises(RuntimeError, match="17 LTC leaves"):
        ext.module_apply(torch.zeros(B, T, D), torch.zeros(B, H), leaves[:3], 0.1, 6, 1e-8,
                         1e-5)


def test_cluster_wait_budget_and_status_without_gpu(capi):
    """The budget setter needs no device; the status query reports the missing one."""
    lib = capi.lib
    prev = lib.ltc_set_cluster_spin_ticks(123)
    try:
        assert prev == 20000000
        assert lib.ltc_set_cluster_spin_ticks(-1) == -1  # rejected, budget unchanged
        assert lib.ltc_set_cluster_spin_ticks(0) == 123
    finally:
        lib.ltc_set_cluster_spin_ticks(prev)
    if lib.ltc_device_count() == 0:
        assert lib.ltc_device_status(0) == 3 and capi.last_error()


@pytest.mark.parametrize("shape,nrc", [((256, 64, 256, 256, 6), 48), ((128, 32, 512, 512, 6), 12),
                                       ((4, 3, 40, 100, 6), 2), ((600, 2, 8, 16, 6), 64)],
                         ids=["C3", "C4", "few-rows", "cap"])
def test_sensory_backward_row_chunks(capi, shape, nrc):
    """Row chunks of the sensory backward: two rounds of three resident blocks
    per CU (256 CUs without a device), at most 64 chunks and at least 8 rows
    each."""
    B, T, D, H, U = shape
    p = capi.plan(B, T, D, H, U)
    assert p["NRC"] == nrc
    bpc = (p["Dp"] // 64) * (p["Hp"] // 32)
    assert p["NRC"] * bpc >= min(6 * 256, bpc * min(64, (B * T + 7) // 8))


@pytest.mark.parametrize("shape,full", [
    ((256, 64, 256, 256, 6), 1),  # C3: four 64-input chunks, many rows
    ((300, 7, 130, 72, 6), 1),    # three chunks, ragged
    ((40, 8, 130, 72, 6), 0),     # few rows: the waves split D instead
    ((4096, 4, 64, 64, 6), 0),    # C5: one chunk is already one list per neuron
    ((128, 32, 512, 512, 6), 0),  # C4: D past the staged rows' LDS
])
def test_sensory_forward_full_lists(capi, shape, full):
    """The module forward's sensory launch walks one list per neuron over all
    of D (the block's rows of x staged whole) when 64 < Dp <= 256 and the
    plan has four row groups per workgroup; otherwise the per-chunk lists."""
    B, T, D, H, U = shape
    p = capi.plan(B, T, D, H, U)
    assert p["sens_full_list"] == full
    if full:
        assert 64 < p["Dp"] <= 256


@pytest.mark.parametrize("B,nb,nbb", [(16, 1, 1), (48, 1, 2), (100, 2, 4), (200, 4, 8)])
def test_two_group_cluster_plans(capi, B, nb, nbb):
    """Rows per cluster at H = 256 (forward NB, chain NBB; the two-group kernels
    run from two rows on), and the chain's LDS: alpha/beta rows padded to NBB + 2
    pairs, the KS partials, the prefetched saved values (1/den and v: 12 bytes per
    row and column, 20 in the two-group form, which keeps 1/den of two unfolds and
    v of three slots), the slot table and the balanced-order scratch."""
    p = capi.plan(B, 2, 8, 256, 6)
    assert (p["CP"], p["NB"], p["NBB"]) == (4, nb, nbb)
    Hp, ks, jw, thr = 256, 16, 32, 512
    pf = 20 if nbb >= 2 else 12
    lds = ((nbb + 2) * Hp * 8 + ks * nbb * jw * 4 + pf * nbb * Hp + thr * 16 * 4
           + thr * 4 + (thr // 64) * 17 * 4)
    assert p["lds_bwd"] == lds <= 159 * 1024
