"""bench.py's host logic on the CPU with a fake backend: the routing check
runs only after every layer slot has run (the driver's `--warmup 5` over 48
rotated layers), and an optional section that raises leaves the headline in
place."""
import numpy as np
import pytest

import bench

E, K = 512, 10


class FakeBackend:
    """Holds each slot's ids/y as host arrays; `read` returns them."""

    def __init__(self):
        self.synced = 0

    def read(self, buf):
        return buf

    def sync(self):
        self.synced += 1


def make_slots(L):
    # zero-filled, as Backend.alloc leaves a fresh buffer
    return [{"ids": np.zeros(K, np.int32), "y": np.zeros(4, np.float32)} for _ in range(L)]


def make_step(slots, skip=()):
    def step(i):
        if i in skip:
            return
        slots[i]["ids"][:] = (np.arange(K) * 37 + i) % E
        slots[i]["y"][:] = 1.0
    return step


def graph_capture(fn):
    return fn  # the fake "graph" replays by calling the same launches


def graph_replay(g):
    g()


@pytest.mark.parametrize("warmup", [0, 5, 47, 96])
def test_check_runs_after_every_slot_ran(warmup):
    L = 48
    slots = make_slots(L)
    be = FakeBackend()
    g = bench.warm_and_check(be, make_step(slots), slots, warmup, graph_capture, graph_replay, E, K, np)
    assert callable(g)
    assert bench.routing_problems(be, slots, E, K, np) == []


def test_check_names_a_slot_that_never_routes():
    L = 48
    slots = make_slots(L)
    with pytest.raises(RuntimeError, match=r"slots \[7\]"):
        bench.warm_and_check(FakeBackend(), make_step(slots, skip={7}), slots, 5, graph_capture, graph_replay, E, K,
                             np)


def test_non_finite_output_is_flagged():
    slots = make_slots(3)
    make_step(slots)(0)
    make_step(slots)(1)
    make_step(slots)(2)
    slots[1]["y"][2] = np.nan
    assert bench.routing_problems(FakeBackend(), slots, E, K, np) == [1]


def test_guarded_section_keeps_the_rest():
    out = {"value": 1.0}

    def boom():
        raise RuntimeError("bench_prompt.js failed")

    bench.guarded(out, "prompt", boom)
    bench.guarded(out, "stack", lambda: {"ok": True})
    assert out["value"] == 1.0
    assert out["prompt"]["error"].startswith("RuntimeError: bench_prompt.js failed")
    assert out["stack"] == {"ok": True}


def test_gpus_other_than_one_exit_with_a_message(capsys, monkeypatch):
    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "one GPU" in capsys.readouterr().err


def test_profiler_detection():
    assert bench.under_profiler({"LD_PRELOAD": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"})
    assert bench.under_profiler({"ROCPROF_KERNEL_TRACE": "1"})
    assert not bench.under_profiler({"LD_PRELOAD": "", "PATH": "/usr/bin"})


def test_graph_replays_refused_under_profiler(capsys, monkeypatch):
    # Graph-replayed runs are not profiled (the profiler crashed inside
    # hipGraphLaunch on them); --eager issues the same steps directly.
    monkeypatch.setattr("sys.argv", ["bench.py", "--steps", "4"])
    monkeypatch.setenv("ROCPROF_KERNEL_TRACE", "1")
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "--eager" in capsys.readouterr().err


def test_flat_prefill_is_scalars_only():
    r = {"tokens_per_s": 1.75e6, "ms_per_layer": 0.2925, "distinct_experts": 512,
         "stage_us": {"prefill_route": 60.0, "prefill_dispatch": 24.0, "prefill_gate_up_gemm": 135.0,
                      "prefill_down_gemm": 78.0, "prefill_combine": 14.0},
         "hbm": {"bytes": 466460672, "achieved_GBs": 1594.7, "frac": 0.1993},
         "mfma": {"layer_flops": 36.5e9, "layer_frac": 0.05}}
    f = bench.flat_prefill("T=512", r, 2048, 512, 512, 10)
    assert all(not isinstance(v, (dict, list)) for v in f.values())
    assert f["roofline_bound"] == "hbm" and f["roofline_frac"] == 0.1993 and f["route_us"] == 60.0
    assert "route_fallback_tokens" not in f
    z = bench.flat_prefill("T=2048 zipf", dict(r, ms_per_layer=0.5, router="certified", route_fallback_tokens=0,
                                               route_candidates_per_token=11.3), 2048, 512, 512, 10)
    assert z["route_fallback_tokens"] == 0 and z["route_candidates_per_token"] == 11.3
    assert z["roofline_bound"] == "mfma" and z["roofline_unit"] == "TFLOP/s"
    assert abs(z["roofline_achieved"] - 36.5e9 / 0.5e-3 / 1e12) < 0.1
