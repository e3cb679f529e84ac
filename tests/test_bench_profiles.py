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


def _fake_result(steps=20):
    # per-step stage times (ms) as run_gpu returns them: (calls, ms per step)
    stages = {"preprocess_project": (steps, 0.025), "bin_count": (steps, 0.110),
              "bin_sort": (steps, 0.069), "rasterize_display_l1": (steps, 0.137),
              "rasterize_l1_backward": (steps, 0.250), "preprocess_backward": (steps, 0.067)}
    return {"n": 1_000_000, "keys": 22_671_735, "n_tiles": 8160, "width": 1920,
            "height": 1080, "steps": steps, "stages": stages, "visited": 261_421_531}


def test_roofline_takes_the_sampled_launch_time():
    # the timed loop carries events around the dominant kernel on every other step:
    # its average over the sampled launches is the launch time, whatever the count
    b = load_bench()
    res = _fake_result()
    res["main_launch_ms"] = {"rasterize_l1_backward": 0.2440}
    rl = b.roofline(res, "config3")["roofline"]
    assert rl["kernel"] == "rasterize_l1_backward" and rl["launch_ms"] == 0.244
    flops = 261_421_531 * 70.0
    assert abs(rl["achieved"] - flops / 0.244e-3 / 1e12) < 1e-3
    assert abs(rl["frac"] - rl["achieved"] / 157.3) < 1e-4
    # without the timed loop's events: the breakdown's per-step time of one launch
    del res["main_launch_ms"]
    assert b.roofline(res, "config3")["roofline"]["launch_ms"] == 0.25


def test_hbm_stages_window_excludes_the_colours_beside_binning():
    b = load_bench()
    res = _fake_result()
    res["stages"]["evaluate_sh_render"] = (20, 0.111)  # on the second stream
    hbm = b.roofline(res, "config3")["hbm_stages"]
    assert hbm["beside_binning"] == ["evaluate_sh_render"]
    assert abs(hbm["ms"] - (0.025 + 0.110 + 0.069 + 0.067)) < 1e-9
    # its bytes count (a window that both stages' traffic passes through)
    with_sh = hbm["bytes"]
    del res["stages"]["evaluate_sh_render"]
    assert b.roofline(res, "config3")["hbm_stages"]["bytes"] < with_sh
