"""HIP-event timing for the benchmark, through the HIP runtime directly.

Events are created with hipEventCreate and recorded either here (around a
whole timed region, on torch's current stream) or by libhsattn itself
(hs_profile_next_launch brackets one kernel on the stream it launches on).
"""

from __future__ import annotations

import ctypes
import ctypes.util
from typing import Callable, List, Tuple

_hip = None


def _rt():
    global _hip
    if _hip is None:
        name = ctypes.util.find_library("amdhip64") or "libamdhip64.so"
        _hip = ctypes.CDLL(name)
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                             ctypes.c_void_p]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return _hip


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with HIP error {rc}")


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        _ok(_rt().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream: int) -> None:
        _ok(_rt().hipEventRecord(self.handle, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, end: "Event") -> float:
        _ok(_rt().hipEventSynchronize(end.handle), "hipEventSynchronize")
        ms = ctypes.c_float()
        _ok(_rt().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
            "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        if _hip is not None and self.handle:
            _hip.hipEventDestroy(self.handle)


def time_steps(step: Callable[[], None], steps: int, warmup: int, stream: int,
               arm: Callable[[Event, Event], None],
               warm_ms: float = 0.0) -> Tuple[float, List[float], float]:
    """Run `warmup` untimed steps (more, when they took less than `warm_ms`
    of wall time: after a host-only phase the GPU's clocks need tens of
    milliseconds of work to come back up), then `steps` timed ones back to
    back, then `steps` more with each step's main kernel bracketed by events.

    The timed region holds the steps only: a pair of event records between
    kernels adds a few microseconds of queue work per step, so the kernel
    times come from the second pass, where `arm(start, stop)` asks libhsattn
    to bracket each step's main kernel.  Returns (mean step ms over the timed
    region, per-step kernel ms of the second pass, host wall seconds of the
    timed region).
    """
    import time

    import torch

    t_w = time.perf_counter()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    spent = time.perf_counter() - t_w
    if warm_ms > 0 and spent * 1e3 < warm_ms:
        per = spent / max(warmup, 1)
        for _ in range(min(500, int((warm_ms * 1e-3 - spent) / max(per, 1e-6)) + 1)):
            step()
        torch.cuda.synchronize()
    region0, region1 = Event(), Event()
    t0 = time.perf_counter()
    region0.record(stream)
    for _ in range(steps):
        step()
    region1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = region0.elapsed_ms(region1) / max(steps, 1)
    pairs = [(Event(), Event()) for _ in range(steps)]
    for s, e in pairs:
        arm(s, e)
        step()
    torch.cuda.synchronize()
    kernel_ms = [s.elapsed_ms(e) for s, e in pairs]
    return step_ms, kernel_ms, wall
