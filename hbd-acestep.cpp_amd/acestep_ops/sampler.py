"""The DiT flow-matching loop with the latents resident on the device
(reference: dit_ggml_generate, dit-sampler.h:408-640). Per step: the model's
conditional and unconditional velocities (a callable returning device
tensors), APG when guidance_scale > 1 (dit-sampler.h:172, 536-590), then the
solver step (solvers/) or, at the last step, the x0 prediction
(dit-sampler.h:601-605) -- no host round trip between steps. Latents and
velocities are F32 DTensors of shape (N, T, Oc) (ggml [Oc, T, N])."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DTensor
from .ops import _out, _p, _s

SOLVERS = {"euler": 0, "dpm3m": 1}
ALL_SOLVERS = ("euler", "sde", "dpm3m", "stork4")  # solvers/solver-registry.h:30-33
INJECTS_NOISE = {"sde"}
DCW_MODES = {"low": 0, "high": 1, "double": 2, "pix": 3}


def apg_buffer(cond) -> DTensor:
    n = ctypes.c_size_t(0)
    _lib.call("mi_apg_buffer_bytes", _p(cond), ctypes.byref(n))
    return DTensor.empty((max(int(n.value), 8),), "u8")


def apg_forward(cond, uncond, guidance_scale: float, mbuf: DTensor, first: bool, momentum: float = -0.75,
                norm_threshold: float = 2.5, out=None, stream=None):
    y = _out(out, cond.shape, "f32")
    _lib.call("mi_apg_forward", _p(cond), _p(uncond), guidance_scale, momentum, norm_threshold,
              ctypes.c_void_p(mbuf.ptr), mbuf.numel() * mbuf.es, int(bool(first)), _p(y), _s(stream))
    return y


def flow_step(solver: str, vt, xt, t_curr: float, t_next: float, history: int = 0, prev=None, prev2=None,
              stream=None):
    _lib.call("mi_flow_step", SOLVERS[solver], _p(vt), _p(xt), t_curr, t_next, history, _p(prev), _p(prev2),
              _s(stream))


def sde_step(vt, xt, noise, t_curr: float, t_next: float, stream=None):
    """SDE ancestral step in place on xt with the step's N(0,1) draws (solver-sde.h:17-38)."""
    _lib.call("mi_flow_step_sde", _p(vt), _p(xt), _p(noise), t_curr, t_next, _s(stream))


class Rock4Tables:
    """ROCK4 coefficient tables for STORK4, host memory (the reference's
    solver-stork4-constants.h: degrees ms, finishing fpa [len(ms)][6] and
    fpb [len(ms)][4], recurrence recf)."""

    def __init__(self, ms, fpa, fpb, recf):
        self.ms = np.ascontiguousarray(ms, np.int32)
        self.fpa = np.ascontiguousarray(fpa, np.float64).reshape(len(self.ms), 6)
        self.fpb = np.ascontiguousarray(fpb, np.float64).reshape(len(self.ms), 4)
        self.recf = np.ascontiguousarray(recf, np.float64)
        dp = ctypes.POINTER(ctypes.c_double)
        self.c = _lib.MiRock4Tables(self.ms.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                    self.fpa.ctypes.data_as(dp), self.fpb.ctypes.data_as(dp),
                                    self.recf.ctypes.data_as(dp), len(self.ms), len(self.recf))


def stork4_workspace(xt) -> DTensor:
    n = ctypes.c_size_t(0)
    _lib.call("mi_stork4_workspace", _p(xt), ctypes.byref(n))
    return DTensor.zeros((int(n.value),), "u8")


def stork4_step(vt, xt, t_curr: float, t_next: float, history: int, h_prev: float, h_prev2: float, prev, prev2,
                tables: Rock4Tables, workspace: DTensor, substeps: int = 10, stream=None):
    """One STORK4 step in place on xt; rotates prev2 <- prev, prev <- vt (solver-stork.h:269-323)."""
    _lib.call("mi_stork4_step", _p(vt), _p(xt), t_curr, t_next, history, h_prev, h_prev2, _p(prev), _p(prev2),
              substeps, ctypes.byref(tables.c), ctypes.c_void_p(workspace.ptr), workspace.numel(), _s(stream))


def stork4_status(workspace: DTensor) -> tuple:
    """(Euler fallbacks since the bootstrap step, last derivative order, last accepted degree); synchronizes."""
    w = workspace.numpy()[:16].view(np.uint32)
    return int(w[0]), int(w[1]), int(w[2])


def dcw(mode: str, xt, vt, t_curr: float, t_next: float, scaler: float, high_scaler: float = 0.0, stream=None):
    """DCW correction in place on xt after a solver step (dit-sampler.h:613-667); unknown modes act as "low"."""
    _lib.call("mi_dcw", DCW_MODES.get(mode, 0), _p(xt), _p(vt), t_curr, t_next, scaler, high_scaler, _s(stream))


def flow_final(xt, vt, t: float, out=None, stream=None):
    y = _out(out, xt.shape, "f32")
    _lib.call("mi_flow_final", _p(xt), _p(vt), t, _p(y), _s(stream))
    return y


class DeviceSampler:
    """dit_ggml_generate's step loop for one generation of N samples."""

    def __init__(self, noise: DTensor, schedule, guidance_scale: float = 1.0, solver: str = "euler",
                 momentum: float = -0.75, norm_threshold: float = 2.5, stream=None, noise_fn=None,
                 rock4: Rock4Tables | None = None, stork_substeps: int = 10, dcw_scaler: float = 0.0,
                 dcw_high_scaler: float = 0.0, dcw_mode: str = "low"):
        """noise_fn(step) -> DTensor of N(0,1) draws shaped like noise (the sde solver's renoise);
        rock4: the STORK4 coefficient tables."""
        if solver not in ALL_SOLVERS:
            raise ValueError(f"solver {solver!r}: the device loop has {list(ALL_SOLVERS)}")
        if solver == "sde" and noise_fn is None:
            raise ValueError("the sde solver needs noise_fn(step) -> the step's N(0,1) draws")
        if solver == "stork4" and rock4 is None:
            raise ValueError("the stork4 solver needs its ROCK4 tables (rock4=Rock4Tables(...))")
        self.xt = DTensor.empty(noise.shape, "f32")
        _lib.call("mi_cpy", _p(noise), _p(self.xt), _s(stream))
        self.schedule = [float(t) for t in schedule]
        self.scale = float(guidance_scale)
        self.solver = solver
        self.momentum, self.threshold = momentum, norm_threshold
        self.stream = stream
        self.noise_fn, self.rock4, self.substeps = noise_fn, rock4, int(stork_substeps)
        self.dcw = (dcw_mode, float(dcw_scaler), float(dcw_high_scaler))
        self.dcw_active = (dcw_scaler > 0.0 or dcw_high_scaler > 0.0) and solver not in INJECTS_NOISE
        self.do_cfg = self.scale > 1.0
        self.mbuf = apg_buffer(noise) if self.do_cfg else None
        self.vt = DTensor.empty(noise.shape, "f32")
        hist = solver in ("dpm3m", "stork4")
        self.prev = DTensor.zeros(noise.shape, "f32") if hist else None
        self.prev2 = DTensor.zeros(noise.shape, "f32") if hist else None
        self.ws = stork4_workspace(self.xt) if solver == "stork4" else None

    def run(self, model_fn) -> DTensor:
        """model_fn(xt, t) -> (v_cond, v_uncond) device tensors (v_uncond ignored without CFG)."""
        n = len(self.schedule)
        hist = 0
        h1 = h2 = 0.0
        out = None
        for step in range(n):
            t = self.schedule[step]
            vc, vu = model_fn(self.xt, t)
            vt = apg_forward(vc, vu, self.scale, self.mbuf, step == 0, self.momentum, self.threshold, out=self.vt,
                             stream=self.stream) if self.do_cfg else vc
            if step == n - 1:
                out = flow_final(self.xt, vt, t, stream=self.stream)
                break
            t_next = self.schedule[step + 1]
            if self.solver == "sde":
                sde_step(vt, self.xt, self.noise_fn(step), t, t_next, stream=self.stream)
            elif self.solver == "stork4":
                stork4_step(vt, self.xt, t, t_next, hist, h1, h2, self.prev, self.prev2, self.rock4, self.ws,
                            self.substeps, stream=self.stream)
                h2, h1 = h1, float(np.float32(t) - np.float32(t_next))
            else:
                flow_step(self.solver, vt, self.xt, t, t_next, hist, self.prev, self.prev2, stream=self.stream)
            hist = min(hist + 1, 2)
            if self.dcw_active:
                mode, s_lo, s_hi = self.dcw
                dcw(mode, self.xt, vt, t, t_next, s_lo, s_hi, stream=self.stream)
        return out
