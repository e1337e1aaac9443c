"""MI355X HIP backend for the LTC fused ODE solver (drop-in for the reference ltc_cuda.py).

The reference builds a pybind11 CUDA extension at import time and exposes
`_HAS_CUDA_KERNELS`, `_cuda_module`, `LTCCudaForward` and `ltc_cuda_forward`
(ltc_cuda.py:23-24, 241-388). This module keeps those names and signatures.
Behind them sits `libltc_hip.so`, a C-ABI library of hand-written gfx950
kernels (include/ltc_capi.h), bound here with ctypes. ctypes releases the
GIL during each call, and every call only enqueues work on the current torch
stream.

Differences from the reference, all deliberate:
  * `_cuda_module.ltc_full_forward/backward` keep the reference's argument
    lists and return lists of tensors, but the saved-for-backward set is one
    opaque `saved` tensor (unfold states and reciprocal denominators) instead of the
    transposed parameter copies and sensory stacks (ltc_cuda.py:281-299).
  * Inputs are validated (device, dtype, shape) and a failing launch raises
    RuntimeError with the library's message; the reference checks nothing.
  * The library is built in-tree (`python ltc-cuda_amd/build.py`). Like the
    reference, which JIT-compiles with an mtime-checked cache
    (ltc_cuda.py:138-234), a missing library is built on first use for the
    visible device (gfx950 only), and a library older than its sources is
    reported, and rebuilt when LTC_JIT=1 (LTC_JIT=0 never builds). A library
    that cannot be built or loaded leaves `_HAS_CUDA_KERNELS = False` with
    the reason in `_LOAD_ERROR`, and `ltc.py` then raises for CUDA inputs
    instead of silently switching paths.
"""

from __future__ import annotations

import ctypes
import importlib.util
import logging
import os

import torch

logger = logging.getLogger(__name__)

_HAS_CUDA_KERNELS = False
_cuda_module = None
_LOAD_ERROR: str | None = None
# C++ autograd node of the fused module path (csrc/ltc_torch_ext.cpp), over
# the same library; None when that extension is not built.
_torch_ext = None

LIB_NAME = "libltc_hip.so"
PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ABI_VERSION = 1
# The one GPU target the kernels are written for.
TARGET_ARCH = "gfx950"

_f32p = ctypes.c_void_p
_i64 = ctypes.c_longlong
_int = ctypes.c_int
_flt = ctypes.c_float


class CApi:
    """ctypes view of include/ltc_capi.h."""

    SYMBOLS = (
        "ltc_abi_version", "ltc_last_error", "ltc_device_count", "ltc_saved_floats",
        "ltc_fwd_workspace_bytes", "ltc_bwd_workspace_bytes", "ltc_full_forward",
        "ltc_full_backward", "ltc_module_saved_floats", "ltc_module_fwd_workspace_bytes",
        "ltc_module_bwd_workspace_bytes", "ltc_module_forward", "ltc_module_backward",
        "ltc_launch_plan", "ltc_timing_enable", "ltc_timing_read", "ltc_kernel_count",
        "ltc_kernel_name", "ltc_sensory_fwd_workspace_bytes", "ltc_sensory_fwd",
        "ltc_ode_unfold_fwd_workspace_bytes", "ltc_ode_unfold_fwd",
        "ltc_sensory_bwd_workspace_bytes", "ltc_sensory_bwd",
        "ltc_ode_unfold_bwd_workspace_bytes", "ltc_ode_unfold_bwd",
        "ltc_full_forward_noalloc", "ltc_device_status", "ltc_set_cluster_spin_ticks",
    )
    PLAN_FIELDS = ("Hp", "Dp", "NB", "KS", "RC", "threads", "lds_fwd", "lds_bwd", "NCH",
                   "NRC", "ode_workgroups", "fuse", "KSB", "RCB",
                   "threads_bwd", "CP", "NCL", "CPB", "NBB", "ode_workgroups_bwd",
                   "cmp_fwd", "cmp_bwd", "module_sens_in_prep", "module_row_bwd_fused",
                   "module_row128_rec_fused", "launches_fwd", "launches_bwd", "sens_full_list")

    def __init__(self, path: str = LIB_PATH):
        self.path = path
        self._sizes = {}
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.ltc_abi_version.restype = _int
        lib.ltc_abi_version.argtypes = []
        lib.ltc_last_error.restype = ctypes.c_char_p
        lib.ltc_last_error.argtypes = []
        lib.ltc_device_count.restype = _int
        lib.ltc_device_count.argtypes = []
        lib.ltc_saved_floats.restype = _i64
        lib.ltc_saved_floats.argtypes = [_int, _int, _int, _int]
        for name in ("ltc_fwd_workspace_bytes", "ltc_bwd_workspace_bytes"):
            fn = getattr(lib, name)
            fn.restype = _i64
            fn.argtypes = [_int, _int, _int, _int, _int]
        lib.ltc_full_forward.restype = _int
        lib.ltc_full_forward.argtypes = (
            [_f32p, _i64, _i64, _i64, _f32p] + [_f32p] * 11
            + [_int, _int, _int, _int, _int, _flt, _int]
            + [_f32p, _f32p, _f32p, _f32p, _i64, ctypes.c_void_p])
        lib.ltc_full_forward_noalloc.restype = _int
        lib.ltc_full_forward_noalloc.argtypes = (
            [_f32p, _i64, _i64, _i64, _f32p] + [_f32p] * 11
            + [_int, _int, _int, _int, _int, _flt, _int]
            + [_f32p, _f32p, _f32p, ctypes.c_void_p])
        lib.ltc_full_backward.restype = _int
        lib.ltc_full_backward.argtypes = (
            [_f32p, _i64, _i64, _i64] + [_f32p] * 11 + [_f32p]
            + [_f32p, _i64, _i64, _i64, _f32p]
            + [_int, _int, _int, _int, _int, _flt]
            + [_f32p] * 13 + [_f32p, _i64, ctypes.c_void_p])
        for name in ("ltc_module_saved_floats", "ltc_module_fwd_workspace_bytes",
                     "ltc_module_bwd_workspace_bytes"):
            fn = getattr(lib, name)
            fn.restype = _i64
            fn.argtypes = [_int, _int, _int, _int, _int]
        lib.ltc_module_forward.restype = _int
        lib.ltc_module_forward.argtypes = (
            [_f32p, _i64, _i64, _i64, _f32p] + [_f32p] * 17
            + [_int, _int, _int, _int, _int, _flt, _flt, _flt, _int]
            + [_f32p, _f32p, _f32p, _f32p, _i64, ctypes.c_void_p])
        lib.ltc_module_backward.restype = _int
        lib.ltc_module_backward.argtypes = (
            [_f32p, _i64, _i64, _i64] + [_f32p] * 17 + [_f32p]
            + [_f32p, _i64, _i64, _i64, _f32p]
            + [_int, _int, _int, _int, _int, _flt, _flt, _flt]
            + [_f32p] * 17 + [_f32p, _i64, ctypes.c_void_p])
        for name in ("ltc_sensory_fwd_workspace_bytes", "ltc_sensory_bwd_workspace_bytes",
                     "ltc_ode_unfold_fwd_workspace_bytes", "ltc_ode_unfold_bwd_workspace_bytes"):
            fn = getattr(lib, name)
            fn.restype = _i64
            fn.argtypes = [_int, _int, _int]
        lib.ltc_sensory_fwd.restype = _int
        lib.ltc_sensory_fwd.argtypes = (
            [_f32p, _i64, _i64] + [_f32p] * 4 + [_int, _int, _int] + [_f32p, _f32p]
            + [_f32p, _i64, ctypes.c_void_p])
        lib.ltc_ode_unfold_fwd.restype = _int
        lib.ltc_ode_unfold_fwd.argtypes = (
            [_f32p] * 10 + [_int, _int, _int, _flt, _int] + [_f32p, _f32p]
            + [_f32p, _i64, ctypes.c_void_p])
        lib.ltc_sensory_bwd.restype = _int
        lib.ltc_sensory_bwd.argtypes = (
            [_f32p, _f32p, _f32p, _i64, _i64] + [_f32p] * 4 + [_int, _int, _int]
            + [_f32p] * 5 + [_f32p, _i64, ctypes.c_void_p])
        lib.ltc_ode_unfold_bwd.restype = _int
        lib.ltc_ode_unfold_bwd.argtypes = (
            [_f32p] * 11 + [_int, _int, _int, _flt] + [_f32p] * 10
            + [_f32p, _i64, ctypes.c_void_p])
        lib.ltc_device_status.restype = _int
        lib.ltc_device_status.argtypes = [_int]
        lib.ltc_set_cluster_spin_ticks.restype = _i64
        lib.ltc_set_cluster_spin_ticks.argtypes = [_i64]
        lib.ltc_launch_plan.restype = _int
        lib.ltc_launch_plan.argtypes = [_int, _int, _int, _int, _int,
                                        ctypes.POINTER(ctypes.c_longlong), _int]
        lib.ltc_timing_enable.restype = _int
        lib.ltc_timing_enable.argtypes = [_int]
        lib.ltc_timing_read.restype = _int
        lib.ltc_timing_read.argtypes = [_int, ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_longlong)]
        lib.ltc_kernel_count.restype = _int
        lib.ltc_kernel_count.argtypes = []
        lib.ltc_kernel_name.restype = ctypes.c_char_p
        lib.ltc_kernel_name.argtypes = [_int]

    def sizes(self, kind: str, B: int, T: int, D: int, H: int, U: int) -> int:
        """Cached size query (saved floats / workspace bytes) for one shape."""
        key = (kind, B, T, D, H, U)
        v = self._sizes.get(key)
        if v is None:
            fn = {"saved": lambda: self.lib.ltc_saved_floats(B, T, H, U),
                  "fwd_ws": lambda: self.lib.ltc_fwd_workspace_bytes(B, T, D, H, U),
                  "bwd_ws": lambda: self.lib.ltc_bwd_workspace_bytes(B, T, D, H, U),
                  "msaved": lambda: self.lib.ltc_module_saved_floats(B, T, D, H, U),
                  "mfwd_ws": lambda: self.lib.ltc_module_fwd_workspace_bytes(B, T, D, H, U),
                  "mbwd_ws": lambda: self.lib.ltc_module_bwd_workspace_bytes(B, T, D, H, U),
                  "sfwd_ws": lambda: self.lib.ltc_sensory_fwd_workspace_bytes(B, D, H),
                  "sbwd_ws": lambda: self.lib.ltc_sensory_bwd_workspace_bytes(B, D, H),
                  "ufwd_ws": lambda: self.lib.ltc_ode_unfold_fwd_workspace_bytes(B, H, U),
                  "ubwd_ws": lambda: self.lib.ltc_ode_unfold_bwd_workspace_bytes(B, H, U)}[kind]
            v = int(fn())
            if v < 0:
                raise ValueError(f"unsupported LTC sizes B={B} T={T} D={D} H={H} U={U}")
            self._sizes[key] = v
        return v

    def device_status(self, clear: bool = True) -> None:
        """Raise RuntimeError if a cluster launch on the current device gave up
        (its outputs were set to NaN); waits for the device. Clears the flag
        unless clear is False."""
        self.check(self.lib.ltc_device_status(1 if clear else 0), "ltc_device_status")

    def last_error(self) -> str:
        return self.lib.ltc_last_error().decode(errors="replace")

    def check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed (code {rc}): {self.last_error()}")

    def plan(self, B: int, T: int, D: int, H: int, U: int) -> dict:
        """Launch plan the library would use for these sizes."""
        n = len(self.PLAN_FIELDS)
        buf = (ctypes.c_longlong * n)()
        got = self.lib.ltc_launch_plan(B, T, D, H, U, buf, n)
        if got < 0:
            raise ValueError(f"invalid LTC sizes B={B} T={T} D={D} H={H} U={U}")
        return dict(zip(self.PLAN_FIELDS, list(buf)[:got]))

    # -- per-kernel event timing -------------------------------------------------
    def timing_enable(self, on: bool) -> None:
        self.check(self.lib.ltc_timing_enable(1 if on else 0), "ltc_timing_enable")

    def timing_read(self) -> dict:
        out = {}
        for k in range(self.lib.ltc_kernel_count()):
            ms = ctypes.c_double(0.0)
            n = ctypes.c_longlong(0)
            self.check(self.lib.ltc_timing_read(k, ctypes.byref(ms), ctypes.byref(n)),
                       "ltc_timing_read")
            out[self.lib.ltc_kernel_name(k).decode()] = (ms.value, n.value)
        return out


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _workspace(nbytes: int, device) -> torch.Tensor:
    ws = torch.empty(max(int(nbytes), 256) + 256, dtype=torch.uint8, device=device)
    return ws


def _aligned(ws: torch.Tensor) -> int:
    p = ws.data_ptr()
    return (p + 255) & ~255


class _HipModule:
    """Stands in for the reference's pybind module (`_cuda_module`).

    Same entry-point names and argument lists as csrc/ltc_kernels.cu:1165-1182
    and :962-984, minus the transposed copies, plus one `saved` tensor.
    """

    def __init__(self, capi: CApi):
        self.capi = capi

    @staticmethod
    def _check_inputs(x_seq, state, params, H, D):
        dev = x_seq.device
        if x_seq.dim() != 3:
            raise ValueError(f"x_seq must be (B, T, D), got {tuple(x_seq.shape)}")
        if state.dim() != 2 or state.shape[0] != x_seq.shape[0]:
            raise ValueError(f"state must be (B, H), got {tuple(state.shape)}")
        shapes = [(H, H)] * 4 + [(D, H)] * 4 + [(H,)] * 3
        for t, shp in zip(params, shapes):
            if tuple(t.shape) != shp:
                raise ValueError(f"parameter shape {tuple(t.shape)} != expected {shp}")
        for t in (x_seq, state, *params):
            if t.device != dev or not t.is_cuda:
                raise ValueError("all LTC tensors must be on the same CUDA (HIP) device")
            if t.dtype != torch.float32:
                raise TypeError(f"LTC HIP kernels are fp32-only, got {t.dtype}")

    def ltc_full_forward(self, x_seq, state, w_pos, w_erev, mu, sigma,
                         sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                         cm_t, gleak_pos, vleak, ode_unfolds, epsilon, save_intermediates):
        B, T, D = x_seq.shape
        H = state.shape[1]
        params = (w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma, sensory_erev,
                  sensory_w_pos, cm_t, gleak_pos, vleak)
        self._check_inputs(x_seq, state, params, H, D)
        dev = x_seq.device
        params = [p.contiguous() for p in params]
        state_c = state.contiguous()
        lib = self.capi.lib
        U = int(ode_unfolds)
        out = torch.empty(B, T, H, device=dev, dtype=torch.float32)
        h = torch.empty(B, H, device=dev, dtype=torch.float32)
        saved = None
        if save_intermediates:
            n = self.capi.sizes("saved", B, T, D, H, U)
            saved = torch.empty(max(n, 1), device=dev, dtype=torch.float32)
        need = self.capi.sizes("fwd_ws", B, T, D, H, U)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            sx = x_seq.stride()
            rc = lib.ltc_full_forward(
                _ptr(x_seq), sx[0], sx[1], sx[2], _ptr(state_c),
                *[_ptr(p) for p in params],
                B, T, D, H, U, float(epsilon), 1 if save_intermediates else 0,
                _ptr(out), _ptr(h), _ptr(saved), _aligned(ws), int(need),
                _stream_handle(dev))
        self.capi.check(rc, "ltc_full_forward")
        return [out, h] if saved is None else [out, h, saved]

    def ltc_full_backward(self, x_seq, state, w_pos, w_erev, mu, sigma,
                          sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                          cm_t, gleak_pos, vleak, saved, grad_outputs, grad_final_state,
                          ode_unfolds, epsilon, has_grad_state):
        B, T, D = x_seq.shape
        H = state.shape[1]
        params = (w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma, sensory_erev,
                  sensory_w_pos, cm_t, gleak_pos, vleak)
        self._check_inputs(x_seq, state, params, H, D)
        dev = x_seq.device
        params = [p.contiguous() for p in params]
        lib = self.capi.lib
        U = int(ode_unfolds)
        if tuple(grad_outputs.shape) != (B, T, H):
            raise ValueError(f"grad_outputs must be (B, T, H), got {tuple(grad_outputs.shape)}")
        go = grad_outputs
        if go.dtype != torch.float32 or go.device != dev:
            go = go.to(device=dev, dtype=torch.float32)
        ghf = None
        if has_grad_state and grad_final_state is not None:
            ghf = grad_final_state.to(device=dev, dtype=torch.float32).contiguous()
        f32 = dict(device=dev, dtype=torch.float32)
        grads = [torch.empty(B, T, D, **f32), torch.empty(B, H, **f32)]
        grads += [torch.empty(H, H, **f32) for _ in range(4)]
        grads += [torch.empty(D, H, **f32) for _ in range(4)]
        grads += [torch.empty(H, **f32) for _ in range(3)]
        need = self.capi.sizes("bwd_ws", B, T, D, H, U)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            sx = x_seq.stride()
            sg = go.stride()
            rc = lib.ltc_full_backward(
                _ptr(x_seq), sx[0], sx[1], sx[2],
                *[_ptr(p) for p in params], _ptr(saved),
                _ptr(go), sg[0], sg[1], sg[2], _ptr(ghf),
                B, T, D, H, U, float(epsilon),
                *[_ptr(g) for g in grads], _aligned(ws), int(need), _stream_handle(dev))
        self.capi.check(rc, "ltc_full_backward")
        return grads


    # -- per-step entry points (csrc/ltc_kernels.cu:675-950, bound at :1308-1311) --------

    @staticmethod
    def _check_f32(dev, *tensors):
        for t in tensors:
            if t.device != dev or not t.is_cuda:
                raise ValueError("all LTC tensors must be on the same CUDA (HIP) device")
            if t.dtype != torch.float32:
                raise TypeError(f"LTC HIP kernels are fp32-only, got {t.dtype}")

    @staticmethod
    def _check_shapes(pairs):
        for t, shp in pairs:
            if tuple(t.shape) != tuple(shp):
                raise ValueError(f"tensor shape {tuple(t.shape)} != expected {tuple(shp)}")

    def ltc_sensory_fwd(self, inputs, sensory_sigma, sensory_mu, sensory_w_pos, sensory_erev):
        """One step's sensory sums -> [w_num_sensory (B,H), w_den_sensory (B,H)]."""
        if inputs.dim() != 2:
            raise ValueError(f"inputs must be (B, D), got {tuple(inputs.shape)}")
        B, D = inputs.shape
        H = sensory_sigma.shape[-1]
        params = [sensory_sigma, sensory_mu, sensory_w_pos, sensory_erev]
        self._check_shapes([(p, (D, H)) for p in params])
        dev = inputs.device
        self._check_f32(dev, inputs, *params)
        params = [p.contiguous() for p in params]
        f32 = dict(device=dev, dtype=torch.float32)
        wn, wd = torch.empty(B, H, **f32), torch.empty(B, H, **f32)
        need = self.capi.sizes("sfwd_ws", B, 1, D, H, 1)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            si = inputs.stride()
            rc = self.capi.lib.ltc_sensory_fwd(
                _ptr(inputs), si[0], si[1], *[_ptr(p) for p in params], B, D, H,
                _ptr(wn), _ptr(wd), _aligned(ws), int(need), _stream_handle(dev))
        self.capi.check(rc, "ltc_sensory_fwd")
        return [wn, wd]

    def ltc_ode_unfold_fwd(self, state, w_pos, w_erev, mu, sigma, w_num_sensory,
                           w_den_sensory, cm_t, gleak_pos, vleak, ode_unfolds, epsilon,
                           save_intermediates):
        """One step's unfolds -> [state_new (B,H), v_buffer (U,B,H) or None]."""
        if state.dim() != 2:
            raise ValueError(f"state must be (B, H), got {tuple(state.shape)}")
        B, H = state.shape
        U = int(ode_unfolds)
        ins = [w_pos, w_erev, mu, sigma, w_num_sensory, w_den_sensory, cm_t, gleak_pos, vleak]
        self._check_shapes(list(zip(ins, [(H, H)] * 4 + [(B, H)] * 2 + [(H,)] * 3)))
        dev = state.device
        self._check_f32(dev, state, *ins)
        state_c = state.contiguous()
        ins = [t.contiguous() for t in ins]
        f32 = dict(device=dev, dtype=torch.float32)
        out = torch.empty(B, H, **f32)
        vbuf = torch.empty(U, B, H, **f32) if save_intermediates else None
        need = self.capi.sizes("ufwd_ws", B, 1, 1, H, U)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            rc = self.capi.lib.ltc_ode_unfold_fwd(
                _ptr(state_c), *[_ptr(t) for t in ins], B, H, U, float(epsilon),
                1 if save_intermediates else 0, _ptr(out), _ptr(vbuf), _aligned(ws), int(need),
                _stream_handle(dev))
        self.capi.check(rc, "ltc_ode_unfold_fwd")
        return [out, vbuf]

    def ltc_sensory_bwd(self, grad_w_num, grad_w_den, inputs, sensory_sigma, sensory_mu,
                        sensory_w_pos, sensory_erev):
        """-> [grad_inputs (B,D), grad_sigma, grad_mu, grad_w_pos, grad_erev (D,H)]."""
        if inputs.dim() != 2:
            raise ValueError(f"inputs must be (B, D), got {tuple(inputs.shape)}")
        B, D = inputs.shape
        H = sensory_sigma.shape[-1]
        params = [sensory_sigma, sensory_mu, sensory_w_pos, sensory_erev]
        self._check_shapes([(p, (D, H)) for p in params]
                           + [(grad_w_num, (B, H)), (grad_w_den, (B, H))])
        dev = inputs.device
        self._check_f32(dev, inputs, grad_w_num, grad_w_den, *params)
        params = [p.contiguous() for p in params]
        gn, gd = grad_w_num.contiguous(), grad_w_den.contiguous()
        f32 = dict(device=dev, dtype=torch.float32)
        grads = [torch.empty(B, D, **f32)] + [torch.empty(D, H, **f32) for _ in range(4)]
        need = self.capi.sizes("sbwd_ws", B, 1, D, H, 1)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            si = inputs.stride()
            rc = self.capi.lib.ltc_sensory_bwd(
                _ptr(gn), _ptr(gd), _ptr(inputs), si[0], si[1], *[_ptr(p) for p in params],
                B, D, H, *[_ptr(g) for g in grads], _aligned(ws), int(need),
                _stream_handle(dev))
        self.capi.check(rc, "ltc_sensory_bwd")
        return grads

    def ltc_ode_unfold_bwd(self, v_buffer, w_pos, w_erev, mu, sigma, w_num_sensory,
                           w_den_sensory, cm_t, gleak_pos, vleak, grad_output, ode_unfolds,
                           epsilon):
        """-> [grad_v, grad_w_num_sensory, grad_w_den_sensory (B,H), grad_w_pos,
        grad_w_erev, grad_mu, grad_sigma (H,H), grad_cm, grad_gleak, grad_vleak (H)]."""
        if v_buffer.dim() != 3:
            raise ValueError(f"v_buffer must be (U, B, H), got {tuple(v_buffer.shape)}")
        U = int(ode_unfolds)
        _, B, H = v_buffer.shape
        if v_buffer.shape[0] < 1:
            raise ValueError("v_buffer holds no unfold")
        ins = [w_pos, w_erev, mu, sigma, w_num_sensory, w_den_sensory, cm_t, gleak_pos, vleak,
               grad_output]
        self._check_shapes(list(zip(ins, [(H, H)] * 4 + [(B, H)] * 2 + [(H,)] * 3
                                    + [(B, H)])))
        dev = v_buffer.device
        self._check_f32(dev, v_buffer, *ins)
        v0 = v_buffer[0].contiguous()
        ins = [t.contiguous() for t in ins]
        f32 = dict(device=dev, dtype=torch.float32)
        grads = [torch.empty(B, H, **f32) for _ in range(3)]
        grads += [torch.empty(H, H, **f32) for _ in range(4)]
        grads += [torch.empty(H, **f32) for _ in range(3)]
        need = self.capi.sizes("ubwd_ws", B, 1, 1, H, U)
        with torch.cuda.device(dev):
            ws = _workspace(need, dev)
            rc = self.capi.lib.ltc_ode_unfold_bwd(
                _ptr(v0), *[_ptr(t) for t in ins], B, H, U, float(epsilon),
                *[_ptr(g) for g in grads], _aligned(ws), int(need), _stream_handle(dev))
        self.capi.check(rc, "ltc_ode_unfold_bwd")
        return grads


MODULE_MAX_D = 1024  # kModuleMaxD in csrc/ltc_internal.h

# Leaf order of the module path (ltc_module_forward argument order).
MODULE_LEAVES = ("w", "erev", "sparsity_mask", "mu", "sigma", "sensory_w", "sensory_erev",
                 "sensory_sparsity_mask", "sensory_mu", "sensory_sigma", "gleak", "vleak", "cm",
                 "input_w", "input_b", "input_norm.weight", "input_norm.bias")
# Leaves that get a gradient, in ltc_module_backward output order (after x, state).
MODULE_GRADS = ("w", "erev", "mu", "sigma", "sensory_w", "sensory_erev", "sensory_mu",
                "sensory_sigma", "gleak", "vleak", "cm", "input_w", "input_b",
                "input_norm.weight", "input_norm.bias")


def _module_forward(capi, x, state, leaves, dt, U, eps, ln_eps, save):
    B, T, D = x.shape
    H = state.shape[1]
    dev = x.device
    lib = capi.lib
    leaves = [t if t.is_contiguous() else t.contiguous() for t in leaves]
    state_c = state if state.is_contiguous() else state.contiguous()
    out = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    h = torch.empty(B, H, device=dev, dtype=torch.float32)
    saved = None
    if save:
        n = capi.sizes("msaved", B, T, D, H, U)
        saved = torch.empty(max(n, 1), device=dev, dtype=torch.float32)
    need = capi.sizes("mfwd_ws", B, T, D, H, U)
    with torch.cuda.device(dev):
        ws = _workspace(need, dev)
        sx = x.stride()
        rc = lib.ltc_module_forward(
            _ptr(x), sx[0], sx[1], sx[2], _ptr(state_c), *[_ptr(t) for t in leaves],
            B, T, D, H, U, float(dt), float(eps), float(ln_eps), 1 if save else 0,
            _ptr(out), _ptr(h), _ptr(saved), _aligned(ws), int(need), _stream_handle(dev))
    capi.check(rc, "ltc_module_forward")
    return out, h, saved


def _module_backward(capi, x, state, leaves, saved, grad_out, grad_h, dt, U, eps, ln_eps):
    B, T, D = x.shape
    H = state.shape[1]
    dev = x.device
    lib = capi.lib
    leaves = [t if t.is_contiguous() else t.contiguous() for t in leaves]
    go = grad_out
    if go.dtype != torch.float32 or go.device != dev:
        go = go.to(device=dev, dtype=torch.float32)
    ghf = None if grad_h is None else grad_h.to(device=dev, dtype=torch.float32).contiguous()
    f32 = dict(device=dev, dtype=torch.float32)
    grads = [torch.empty(B, T, D, **f32), torch.empty(B, H, **f32)]
    grads += [torch.empty(H, H, **f32) for _ in range(4)]
    grads += [torch.empty(D, H, **f32) for _ in range(4)]
    grads += [torch.empty(H, **f32) for _ in range(3)]
    grads += [torch.empty(D, **f32) for _ in range(4)]
    need = capi.sizes("mbwd_ws", B, T, D, H, U)
    with torch.cuda.device(dev):
        ws = _workspace(need, dev)
        sx = x.stride()
        sg = go.stride()
        rc = lib.ltc_module_backward(
            _ptr(x), sx[0], sx[1], sx[2], *[_ptr(t) for t in leaves], _ptr(saved),
            _ptr(go), sg[0], sg[1], sg[2], _ptr(ghf), B, T, D, H, U, float(dt), float(eps),
            float(ln_eps), *[_ptr(g) for g in grads], _aligned(ws), int(need),
            _stream_handle(dev))
    capi.check(rc, "ltc_module_backward")
    return grads


class LTCModuleFunction(torch.autograd.Function):
    """The whole layer forward/backward in two library calls.

    Inputs: x (B,T,D) raw (before LayerNorm), state (B,H), then the module's
    leaves in MODULE_LEAVES order (masks are buffers and get no gradient),
    then dt, ode_unfolds, epsilon, ln_eps, needs_grad. The pre-transforms of
    the reference module (ltc.py:259-283) run inside the library, so their
    ~25 PyTorch launches and autograd nodes are gone.
    """

    @staticmethod
    def forward(ctx, x, state, *rest):
        leaves = rest[:17]
        dt, U, eps, ln_eps, needs_grad = rest[17:]
        capi = require_kernels().capi
        out, h, saved = _module_forward(capi, x, state, leaves, dt, U, eps, ln_eps, needs_grad)
        if needs_grad:
            ctx.save_for_backward(x, state, *leaves, saved)
        ctx.cfg = (dt, U, eps, ln_eps)
        return out, h

    @staticmethod
    def backward(ctx, grad_out, grad_h):
        saved_t = ctx.saved_tensors
        if not saved_t:
            raise RuntimeError("LTCModuleFunction.backward called on a forward run without grad")
        x, state = saved_t[0], saved_t[1]
        leaves, buf = saved_t[2:19], saved_t[19]
        dt, U, eps, ln_eps = ctx.cfg
        if grad_out is None:
            grad_out = torch.zeros(x.shape[0], x.shape[1], state.shape[1], device=x.device)
        g = _module_backward(require_kernels().capi, x, state, leaves, buf, grad_out, grad_h,
                             dt, U, eps, ln_eps)
        gx, gstate = g[0], g[1]
        (gw, gerev, gmu, gsig, gsw, gserev, gsmu, gssig, ggl, gvl, gcm, giw, gib, glw,
         glb) = g[2:]
        leaf_grads = (gw, gerev, None, gmu, gsig, gsw, gserev, None, gsmu, gssig, ggl, gvl,
                      gcm, giw, gib, glw, glb)
        return (gx, gstate, *leaf_grads, None, None, None, None, None)


def ltc_module_forward(x_seq, state, leaves, dt, ode_unfolds, epsilon, ln_eps):
    """Whole-layer fused call; `leaves` in MODULE_LEAVES order, `state` None
    for a zero initial state.

    Runs through the C++ autograd node when the torch extension is built
    (no Python in the per-step forward or backward), else through
    LTCModuleFunction; both call the same two library entry points.
    """
    ext = _torch_ext
    if ext is not None:
        return tuple(ext.module_apply(x_seq, state, leaves, float(dt), int(ode_unfolds),
                                      float(epsilon), float(ln_eps)))
    require_kernels()
    if state is None:
        state = torch.zeros(x_seq.shape[0], leaves[0].shape[0], device=x_seq.device,
                            dtype=torch.float32)
    needs_grad = torch.is_grad_enabled()
    return LTCModuleFunction.apply(x_seq, state, *leaves, float(dt), int(ode_unfolds),
                                   float(epsilon), float(ln_eps), needs_grad)


def load_capi(path: str = LIB_PATH) -> CApi:
    """Load the C-ABI library and check its ABI version (no device needed)."""
    capi = CApi(path)
    ver = capi.lib.ltc_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {ver}, expected {ABI_VERSION}")
    return capi


def device_arch(props) -> str:
    """gfx target of a device from torch's device properties: the part of
    `gcnArchName` before its feature flags ('gfx950:sramecc+:xnack-' -> 'gfx950')."""
    return (getattr(props, "gcnArchName", "") or "").split(":")[0]


def _build_script():
    spec = importlib.util.spec_from_file_location("ltc_build", os.path.join(PKG_DIR, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def stale_sources(lib_path: str, sources) -> list:
    """Sources modified after the library was built (the reference's cache
    check compares the same mtimes, ltc_cuda.py:150-160)."""
    lib_t = os.path.getmtime(lib_path)
    return [s for s in sources if os.path.isfile(s) and os.path.getmtime(s) > lib_t]


def load_action(lib_exists: bool, stale: bool, jit: str) -> str:
    """What the loader does: 'load', 'build' (none built yet), 'rebuild'
    (stale and LTC_JIT=1), 'warn' (stale, load it anyway) or 'missing'
    (none built and LTC_JIT=0)."""
    if not lib_exists:
        return "missing" if jit == "0" else "build"
    if stale:
        return "rebuild" if jit == "1" else "warn"
    return "load"


def _try_load_hip_kernels() -> bool:
    """Load libltc_hip.so when a HIP device is present (ltc_cuda.py:138-234).

    A missing library is compiled here (hipcc for the device's gfx target,
    about a minute) unless LTC_JIT=0; a library older than its sources is
    rebuilt only when LTC_JIT=1, else loaded with a warning.
    """
    global _HAS_CUDA_KERNELS, _cuda_module, _LOAD_ERROR
    _HAS_CUDA_KERNELS = False
    _cuda_module = None
    if not torch.cuda.is_available():
        _LOAD_ERROR = "no HIP device visible to torch"
        return False
    arch = device_arch(torch.cuda.get_device_properties(torch.cuda.current_device()))
    if arch and arch != TARGET_ARCH:
        _LOAD_ERROR = f"device is {arch}; libltc_hip.so is written for {TARGET_ARCH} only"
        logger.warning("LTC HIP kernels unavailable: %s", _LOAD_ERROR)
        return False
    jit = os.environ.get("LTC_JIT", "")
    exists = os.path.isfile(LIB_PATH)
    stale = []
    if exists:
        try:
            stale = stale_sources(LIB_PATH, _build_script().source_files())
        except (OSError, ImportError) as exc:
            logger.info("LTC source freshness check skipped: %s", exc)
    action = load_action(exists, bool(stale), jit)
    if action == "missing":
        _LOAD_ERROR = (f"{LIB_PATH} not found (LTC_JIT=0); build it with "
                       f"`python {os.path.join(PKG_DIR, 'build.py')}`")
        logger.warning("LTC HIP kernels unavailable: %s", _LOAD_ERROR)
        return False
    if action == "warn":
        logger.warning("LTC: %s is older than %s; rebuild with build.py or set LTC_JIT=1",
                       LIB_PATH, ", ".join(os.path.basename(p) for p in stale))
    if action in ("build", "rebuild"):
        logger.warning("LTC: building %s for %s (first use)", LIB_PATH, arch or TARGET_ARCH)
        try:
            _build_script().build(arch=arch or TARGET_ARCH)
        except (OSError, RuntimeError) as exc:
            _LOAD_ERROR = f"building {LIB_PATH} failed: {exc}"
            logger.warning("LTC HIP kernels unavailable: %s", _LOAD_ERROR)
            return False
    try:
        capi = load_capi(LIB_PATH)
        if capi.lib.ltc_device_count() < 1:
            raise RuntimeError("libltc_hip.so sees no HIP device")
    except (OSError, RuntimeError) as exc:
        _LOAD_ERROR = f"failed to load {LIB_PATH}: {exc}"
        logger.warning("LTC HIP kernels unavailable: %s", _LOAD_ERROR)
        return False
    _cuda_module = _HipModule(capi)
    _HAS_CUDA_KERNELS = True
    _LOAD_ERROR = None
    _load_torch_ext()
    logger.info("Loaded LTC HIP kernels from %s", LIB_PATH)
    return True


def _load_torch_ext() -> None:
    """Import the C++ autograd glue built beside the library, if present."""
    global _torch_ext
    import importlib.machinery
    import importlib.util
    import sysconfig
    _torch_ext = None
    path = os.path.join(os.path.dirname(LIB_PATH),
                        "_ltc_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.isfile(path):
        logger.info("LTC torch extension not built; module path uses the Python Function")
        return
    try:
        loader = importlib.machinery.ExtensionFileLoader("_ltc_torch", path)
        spec = importlib.util.spec_from_file_location("_ltc_torch", path, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
    except ImportError as exc:
        logger.warning("LTC torch extension failed to load (%s); using the Python Function",
                       exc)
        return
    if mod.abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: linked against ABI {mod.abi_version()}, "
                           f"expected {ABI_VERSION}")
    _torch_ext = mod


# Name kept for callers of the reference loader.
_try_load_cuda_kernels = _try_load_hip_kernels

_try_load_hip_kernels()


def require_kernels():
    """Return the loaded backend or raise with the reason it is missing."""
    if not _HAS_CUDA_KERNELS or _cuda_module is None:
        raise RuntimeError(f"LTC HIP extension is not loaded: {_LOAD_ERROR}")
    return _cuda_module


def device_status(clear: bool = True) -> None:
    """Raise RuntimeError if a launch on the current device gave up waiting
    for its partner workgroups since the last check: a cluster launch
    (H > 192), or the companion workgroups of a module backward with one batch
    row per workgroup (the sensory and LayerNorm companions at H <= 64, the
    recurrent-gradient and sensory companions at 64 < H <= 128). The outputs
    of that call were set to NaN. Synchronises the device."""
    require_kernels().capi.device_status(clear)


class LTCCudaForward(torch.autograd.Function):
    """Autograd Function over the fused HIP forward/backward (ltc_cuda.py:241-359).

    forward inputs and backward gradients keep the reference order:
    x_seq, state, w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma,
    sensory_erev, sensory_w_pos, cm_t, gleak_pos, vleak, then None for
    ode_unfolds, epsilon and needs_grad.
    """

    @staticmethod
    def forward(ctx, x_seq, state, w_pos, w_erev, mu, sigma,
                sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                cm_t, gleak_pos, vleak, ode_unfolds, epsilon, needs_grad):
        mod = require_kernels()
        result = mod.ltc_full_forward(
            x_seq, state, w_pos, w_erev, mu, sigma,
            sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
            cm_t, gleak_pos, vleak, ode_unfolds, epsilon, needs_grad)
        outputs, current_state = result[0], result[1]
        if needs_grad:
            ctx.save_for_backward(x_seq, state, w_pos, w_erev, mu, sigma,
                                  sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                                  cm_t, gleak_pos, vleak, result[2])
        ctx.ode_unfolds = ode_unfolds
        ctx.epsilon = epsilon
        return outputs, current_state

    @staticmethod
    def backward(ctx, grad_outputs, grad_state):
        saved = ctx.saved_tensors
        if not saved:
            raise RuntimeError("LTCCudaForward.backward called on a forward run without grad")
        (x_seq, state, w_pos, w_erev, mu, sigma, sensory_mu, sensory_sigma, sensory_erev,
         sensory_w_pos, cm_t, gleak_pos, vleak, buf) = saved
        B, T, _ = x_seq.shape
        H = state.shape[1]
        if grad_outputs is None:
            grad_outputs = torch.zeros(B, T, H, device=x_seq.device, dtype=x_seq.dtype)
        has_grad_state = grad_state is not None
        grads = require_kernels().ltc_full_backward(
            x_seq, state, w_pos, w_erev, mu, sigma,
            sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
            cm_t, gleak_pos, vleak, buf, grad_outputs, grad_state,
            ctx.ode_unfolds, ctx.epsilon, has_grad_state)
        return (*grads, None, None, None)


def ltc_cuda_forward(x_seq, state, w_pos, w_erev, mu, sigma,
                     sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
                     cm_t, gleak_pos, vleak, ode_unfolds, epsilon):
    """Entry point of the fused path (ltc_cuda.py:362-388).

    Grad mode is read here, outside Function.forward where it is always off.
    """
    needs_grad = torch.is_grad_enabled()
    return LTCCudaForward.apply(
        x_seq, state, w_pos, w_erev, mu, sigma,
        sensory_mu, sensory_sigma, sensory_erev, sensory_w_pos,
        cm_t, gleak_pos, vleak, ode_unfolds, epsilon, needs_grad)


def _detach_tree(obj):
    if isinstance(obj, torch.Tensor):
        return obj.detach()
    if isinstance(obj, (tuple, list)):
        return type(obj)(_detach_tree(o) for o in obj)
    return obj


class CapturedStep:
    """One training step of a module (forward, loss, backward) as one HIP graph.

    At small sizes a step is bound by the host: at B=24 T=8 D=128 H=64 the
    GPU work is about 0.08 ms (four library kernels plus the loss and its
    gradient), while issuing it eagerly through autograd costs more host time
    than that. Replaying the captured step issues it with one graph launch.

    How the step is captured:

    * a few warm-up steps run first on a side stream (torch's recipe for
      whole-network capture), so that lazily built state such as allocator
      blocks exists before capture;
    * the backward is `torch.autograd.grad` over the module's parameters, not
      `loss.backward()`: it runs no AccumulateGrad node, so an autograd graph
      kept alive from an earlier eager step (whose AccumulateGrad nodes belong
      to the default stream, which capture forbids touching) cannot reach
      into the capture;
    * the captured gradients are then installed as the parameters' `.grad`,
      and every replay rewrites them in place. Zeroing or replacing `.grad`
      between replays detaches them from the graph; `install_grads()` puts
      them back;
    * a scalar loss's seed gradient (the 1 that `loss.backward()` starts
      from) is a tensor made once before capture, so the graph holds no fill
      kernel for it; a non-scalar loss is seeded with ones of its shape, as
      `loss.backward(torch.ones_like(loss))` would be.

    `inputs` are static: copy new data into them (`step.inputs[0].copy_(x)`)
    before `replay()`. `outputs` and `loss` are detached views of the graph's
    output memory, rewritten by every replay.
    """

    def __init__(self, module, inputs, loss_fn, warmup: int = 3):
        self.module = module
        self.inputs = tuple(inputs)
        self.params = [p for p in module.parameters() if p.requires_grad]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        seed = None
        with torch.cuda.stream(side):
            for _ in range(max(1, int(warmup))):
                loss = loss_fn(module(*self.inputs))
                if seed is None:
                    seed = torch.ones_like(loss)
                torch.autograd.grad(loss, self.params, grad_outputs=seed, allow_unused=True)
                del loss
        torch.cuda.current_stream().wait_stream(side)
        self._seed = seed
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            out = module(*self.inputs)
            loss = loss_fn(out)
            grads = torch.autograd.grad(loss, self.params, grad_outputs=self._seed,
                                        allow_unused=True)
            # a parameter the loss does not reach gets zeros, as backward() leaves none
            grads = [torch.zeros_like(p) if g is None else g for p, g in zip(self.params, grads)]
        self.outputs = _detach_tree(out)
        self.loss = loss.detach()
        self.grads = [g.detach() for g in grads]
        self.install_grads()

    def install_grads(self) -> None:
        """Point every parameter's .grad at the graph's gradient tensor."""
        for p, g in zip(self.params, self.grads):
            p.grad = g

    def replay(self):
        """Run the captured step once on the current stream; returns the loss tensor."""
        self.graph.replay()
        return self.loss
