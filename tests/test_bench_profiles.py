"""CPU checks of bench.py's reading of the committed rocprofv3 summaries: the
dominant kernel's HBM traffic and the step roofline's per-kernel bounds must be
found for the kernel names the profiles hold (the blend kernels carry a
waves-per-tile template argument there)."""

from __future__ import annotations

import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_kernel_base_names():
    b = load_bench()
    assert b.kernel_base("blend_forward_kernel<1>") == "blend_forward_kernel"
    assert b.kernel_base("blend_forward_kernel<4>") == "blend_forward_kernel"
    assert b.kernel_base("blend_backward_kernel<2, 1>") == "blend_backward_kernel<2>"
    assert b.kernel_base("blend_backward_kernel<0, 4>") == "blend_backward_kernel<0>"
    assert b.kernel_base("l2_scatter_kernel<true>") == "l2_scatter_kernel<true>"


def test_committed_profile_feeds_the_bench_line():
    b = load_bench()
    traffic = b.profiled_traffic("rasterize_l1_backward", "config3")
    assert traffic is not None and traffic > 1e8
    assert b.profiled_traffic("preprocess_forward", "config3") > 5e7
    res = {"visited": 261_421_531, "ms": 0.73}
    sr = b.step_roofline(res, "config3")
    assert sr is not None and sr["kernels"] >= 10
    # both blend kernels are priced by their flops as well as their bytes
    assert sr["valu_ms"] > 0.1 and sr["bound_ms"] > sr["hbm_ms"]
