"""ctypes binding of libgsraster.so (C ABI declared in include/gs_rasterizer.h)."""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgsraster.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_PSZ = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes (all functions return int status)
SIGNATURES = {
    "gs_tile_schedule_size": [_I32, _P],
    "gs_abi_version": [],
    "gs_host_device_pointer": [_P, ctypes.POINTER(ctypes.c_void_p)],
    "gs_project_points": [_P] * 6 + [_I64, _F, _F, _F, _F, _F, _I32, _I32] + [_P] * 6 + [_P],
    "gs_project_points_backward": [_P] * 8 + [_I64, _I32, _I32] + [_P] * 5 + [_P],
    "gs_evaluate_sh": [_P] * 5 + [_I64, _I32, _P, _P],
    "gs_evaluate_sh_backward": [_P] * 7 + [_I64, _I32] + [_P] * 3 + [_P],
    "gs_bin_count_workspace_size": [_I64, _PSZ],
    "gs_bin_count": [_P] * 4 + [_I64, _I32, _I32, _I32, _P, _SZ, _P, _P],
    "gs_bin_count_begin": [_P] * 4 + [_I64, _I32, _I32, _I32, _P, _SZ, _P, _P],
    "gs_bin_count_finish": [_P] * 4 + [_I64, _I32, _I32, _I32, _P, _SZ, _P, _P],
    "gs_bin_count_begin_hinted": [_P] * 4 + [_I64, _I32, _I32, _I32, _P, _SZ, ctypes.c_uint32,
                                            _I32, _P, _P],
    "gs_bin_sort_workspace_size": [_I64, _I64, _I64, _I32, _I32, _I32, _PSZ],
    "gs_bin_sort": [_P] * 3 + [_I64, _I32, _I32, _I32, _I64, _I64, _P, _P, _SZ] + [_P] * 4 + [_P],
    "gs_bin_sort_ordered": [_P] * 3 + [_I64, _I32, _I32, _I32, _I64, _I64, _P, _P, _SZ]
    + [_P] * 5 + [_P],
    "gs_bin_sort_capped": [_P] * 3 + [_I64, _I32, _I32, _I32, _I64, _I64, _P, _P, _SZ]
    + [_P] * 3 + [_P],
    "gs_rasterize": [_P, _P, _I32, _I64] + [_P] * 4 + [_I64, _I32, _I32, _I32, _F, _F, _F, _P, _P],
    "gs_rasterize_work": [_P, _P, _I32, _I64] + [_P] * 3 + [_I64, _I32, _I32, _I32, _F, _F, _F]
    + [_P, _P, _P],
    "gs_evaluate_sh_render": [_P] * 5 + [_I64, _P, _P],
    "gs_evaluate_sh_render_beside": [_P] * 5 + [_I64, _P, _P],
    "gs_evaluate_sh_render_cache": [_P] * 5 + [_I64, _I32, _P, _P, _P],
    "gs_evaluate_sh_render_backward": [_P] * 6 + [_I64, _I32] + [_P] * 3 + [_P],
    "gs_activate": [_P] * 3 + [_I64] + [_P] * 3 + [_P],
    "gs_preprocess_forward": [_P] * 8 + [_I64, _F, _F, _F, _F, _F, _I32, _I32] + [_P] * 9 + [_P],
    "gs_preprocess_backward": [_P] * 14 + [_I64, _I32, _I32] + [_P] * 7 + [_P],
    "gs_render_preprocess_backward": [_P] * 12 + [_I64, _I32, _I32] + [_P] * 6 + [_P],
    "gs_activate_backward": [_P] * 6 + [_I64] + [_P] * 3 + [_P],
    "gs_rasterize_display_l1": [_P, _P, _I32, _I64] + [_P] * 4
    + [_I64, _I32, _I32, _I32, _F, _F, _F] + [_P] * 7 + [_I64, _P, _P],
    "gs_l1_finish": [_P, _I32, _I64, _P, _P],
    "gs_set_blend_waves": [_I32],
    "gs_rasterize_l1_backward": [_P] * 5 + [_I32, _I64] + [_P] * 4
    + [_I64, _I32, _I32, _I32, _F, _F, _F] + [_P] * 4 + [_I32, _F, _P, _P, _P],
    "gs_rasterize_display": [_P, _P, _I32, _I64] + [_P] * 4
    + [_I64, _I32, _I32, _I32, _F, _F, _F, _P, _P, _P, _P, _P],
    "gs_rasterize_display_backward": [_P] * 4 + [_I32, _I64] + [_P] * 4
    + [_I64, _I32, _I32, _I32, _F, _F, _F]
    + [_P] * 4
    + [_I32, _P, _P],
    "gs_rasterize_backward": [_P] * 4 + [_I32, _I64] + [_P] * 4
    + [_I64, _I32, _I32, _I32, _F, _F, _F]
    + [_P] * 4
    + [_I32, _P],
}

class GsAdamTensor(ctypes.Structure):
    """include/gs_rasterizer.h GsAdamTensor."""

    _fields_ = [("param", _P), ("grad", _P), ("exp_avg", _P), ("exp_avg_sq", _P),
                ("count", _I64), ("step_size", _F), ("bias_correction2_sqrt", _F)]


class GsGatherTensor(ctypes.Structure):
    """include/gs_rasterizer.h GsGatherTensor."""

    _fields_ = [("src", _P), ("dst", _P), ("delta", _P), ("width", _I32), ("zero_fresh", _I32)]


SIGNATURES.update({
    "gs_adam_step": [ctypes.POINTER(GsAdamTensor), _I32, ctypes.c_double, ctypes.c_double,
                     ctypes.c_double, _P],
    "gs_accumulate_grad2d": [_P, _P, _I64, _I32, _I32, _P, _P, _P],
    "gs_gather_rows": [_I64, _P, _P, ctypes.POINTER(GsGatherTensor), _I32, _P],
    "gs_ssim_workspace_size": [_I32, _I32, _I32, _I32, _PSZ],
    "gs_ssim_forward": [_P] * 4 + [_I32] * 5 + [_F] + [_P] * 5 + [_F, _P, _P, _SZ, _P],
    "gs_ssim_forward_noalloc": [_P] * 4 + [_I32] * 5 + [_F] + [_P] * 5 + [_F, _P, _P],
    "gs_ssim_backward": [_P] * 5 + [_I32] * 4 + [_F] + [_P] * 3 + [_F, _P, _P, _P],
})

_lib = None


class RasterizerError(RuntimeError):
    """A gs_* entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"cuda_rasterizer: HIP library not found at {LIB_PATH}; build it with "
            "`python 3dgs_from_scratch_amd/build_lib.py` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.gs_status_string.argtypes = [ctypes.c_int]
    lib.gs_status_string.restype = ctypes.c_char_p
    _lib = lib
    return lib


class StageTimer:
    """Opt-in HIP-event timing of entry points on the stream they launch on.

    While enabled, each instrumented call records a (start, end) event pair on
    the device's current stream around the library call (only the stages in
    `only`, when set); `summary()` returns {stage: (calls, total_ms)} after
    synchronising.  Events come from a pool that reset() rewinds, so timing
    adds two event records per timed call and no event creation.
    """

    def __init__(self):
        self.enabled = False
        self.only = None
        self.events: dict = {}
        self._pool: list = []
        self._used = 0

    def reset(self):
        self.events = {}
        self._used = 0

    def _event(self):
        import torch

        if self._used == len(self._pool):
            self._pool.append(torch.cuda.Event(enable_timing=True))
        ev = self._pool[self._used]
        self._used += 1
        return ev

    def record(self, stage: str, device, stream=None):
        import torch

        if not self.enabled or (self.only is not None and stage not in self.only):
            return None
        ev = (self._event(), self._event())
        ev[0].record(stream if stream is not None else torch.cuda.current_stream(device))
        self.events.setdefault(stage, []).append(ev)
        return ev

    def stop(self, ev, device, stream=None):
        import torch

        if ev is not None:
            ev[1].record(stream if stream is not None else torch.cuda.current_stream(device))

    def summary(self) -> dict:
        import torch

        torch.cuda.synchronize()
        return {k: (len(v), sum(a.elapsed_time(b) for a, b in v)) for k, v in self.events.items()}


timer = StageTimer()


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().gs_status_string(status).decode()
        raise RasterizerError(f"{what} failed: {msg} (status {status})")
