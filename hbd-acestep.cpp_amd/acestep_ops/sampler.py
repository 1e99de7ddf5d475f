"""The DiT flow-matching loop with the latents resident on the device
(reference: dit_ggml_generate, dit-sampler.h:408-640). Per step: the model's
conditional and unconditional velocities (a callable returning device
tensors), APG when guidance_scale > 1 (dit-sampler.h:172, 536-590), then the
solver step (solvers/) or, at the last step, the x0 prediction
(dit-sampler.h:601-605) -- no host round trip between steps. Latents and
velocities are F32 DTensors of shape (N, T, Oc) (ggml [Oc, T, N])."""
from __future__ import annotations

import ctypes

from . import _lib
from .device import DTensor
from .ops import _out, _p, _s

SOLVERS = {"euler": 0, "dpm3m": 1}


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


def flow_final(xt, vt, t: float, out=None, stream=None):
    y = _out(out, xt.shape, "f32")
    _lib.call("mi_flow_final", _p(xt), _p(vt), t, _p(y), _s(stream))
    return y


class DeviceSampler:
    """dit_ggml_generate's step loop for one generation of N samples."""

    def __init__(self, noise: DTensor, schedule, guidance_scale: float = 1.0, solver: str = "euler",
                 momentum: float = -0.75, norm_threshold: float = 2.5, stream=None):
        if solver not in SOLVERS:
            raise ValueError(f"solver {solver!r}: the device loop has {sorted(SOLVERS)}")
        self.xt = DTensor.empty(noise.shape, "f32")
        _lib.call("mi_cpy", _p(noise), _p(self.xt), _s(stream))
        self.schedule = [float(t) for t in schedule]
        self.scale = float(guidance_scale)
        self.solver = solver
        self.momentum, self.threshold = momentum, norm_threshold
        self.stream = stream
        self.do_cfg = self.scale > 1.0
        self.mbuf = apg_buffer(noise) if self.do_cfg else None
        self.vt = DTensor.empty(noise.shape, "f32")
        self.prev = DTensor.zeros(noise.shape, "f32") if solver == "dpm3m" else None
        self.prev2 = DTensor.zeros(noise.shape, "f32") if solver == "dpm3m" else None

    def run(self, model_fn) -> DTensor:
        """model_fn(xt, t) -> (v_cond, v_uncond) device tensors (v_uncond ignored without CFG)."""
        n = len(self.schedule)
        hist = 0
        out = None
        for step in range(n):
            t = self.schedule[step]
            vc, vu = model_fn(self.xt, t)
            vt = apg_forward(vc, vu, self.scale, self.mbuf, step == 0, self.momentum, self.threshold, out=self.vt,
                             stream=self.stream) if self.do_cfg else vc
            if step == n - 1:
                out = flow_final(self.xt, vt, t, stream=self.stream)
            else:
                flow_step(self.solver, vt, self.xt, t, self.schedule[step + 1], hist, self.prev, self.prev2,
                          stream=self.stream)
                hist = min(hist + 1, 2)
        return out
