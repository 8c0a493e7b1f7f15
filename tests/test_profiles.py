"""Integrity of the committed rocprofv3 summaries that bench.py reports from (the
reference's report-file check, tests/test_phase1_task13_bandwidth_saturation.py:87-156):
the in-graph kernel table and the gate/up HBM-traffic record are complete, internally
consistent with the algorithmic bytes bench.py computes, and name the commit and commands
they were measured with; and the trace summarizer recognises every decode kernel under
both of the names the profiler prints for it."""

import csv
import os
import re

import pytest

import bench

PROFILES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles")
LAYER_KERNELS = ("qkv", "attention", "o", "gate_up", "down")


def test_in_graph_kernel_table_is_complete_and_consistent():
    js = bench.in_graph_profile(128)
    assert js is not None, "profiles/decode_7b_q4_g128_kernel_stats.json is missing"
    assert re.fullmatch(r"[0-9a-f]{7,40}", js["measured_at_commit"])
    assert "rocprofv3 --kernel-trace" in js["command"]
    k = js["kernels"]
    assert set(k) == set(LAYER_KERNELS) | {"lm_head", "set_params"}
    steps = js["decode_steps"]
    nb = bench.kernel_bytes(bench.CFG_7B, 128 + 28, 128)
    for name, e in k.items():
        assert 0 < e["min_us"] <= e["avg_us"] <= e["max_us"], name
        want_calls = steps * (1 if name in ("lm_head", "set_params") else bench.CFG_7B["n_layer"])
        assert e["calls"] == want_calls, name
        if name in nb:
            assert e["algorithmic_bytes"] == nb[name], name
            frac = e["algorithmic_bytes"] / (e["avg_us"] * 1e-6) / 1e9 / bench.HBM_PEAK_GBS
            assert e["frac"] == pytest.approx(frac, abs=1e-4), name
    per_layer = sum(k[n]["avg_us"] for n in LAYER_KERNELS)
    assert js["per_layer_us"] == pytest.approx(per_layer, abs=0.01)
    tok = bench.CFG_7B["n_layer"] * per_layer + k["lm_head"]["avg_us"] + k["set_params"]["avg_us"]
    assert js["kernel_us_per_token"] == pytest.approx(tok, abs=0.1)
    with open(os.path.join(PROFILES, "decode_7b_q4_g128_kernel_stats.txt")) as f:
        txt = f.read()
    assert js["measured_at_commit"] in txt and "rocprofv3 --kernel-trace" in txt


def test_gate_up_traffic_record_is_consistent():
    hbm, prov = bench.gate_up_traffic(128)
    assert hbm is not None, "profiles/gate_up_g128_traffic.json is missing"
    import json

    with open(os.path.join(PROFILES, "gate_up_g128_traffic.json")) as f:
        j = json.load(f)
    fs = j["calibration_copy_bytes"] / 1024.0 / j["calibration_fetch_size_kib"]
    ws = j["calibration_copy_bytes"] / 1024.0 / j["calibration_write_size_kib"]
    assert j["fetch_scale"] == pytest.approx(fs, abs=1e-4) and j["write_scale"] == pytest.approx(ws, abs=1e-4)
    want = j["fetch_size_kib_per_dispatch"] * 1024 * j["fetch_scale"] + j["write_size_kib_per_dispatch"] * 1024 * j[
        "write_scale"]
    assert hbm == pytest.approx(want, rel=1e-5)
    alg = bench.kernel_bytes(bench.CFG_7B, 129, 128)["gate_up"]
    assert j["algorithmic_bytes_per_launch"] == alg
    assert j["traffic_over_algorithmic"] == pytest.approx(hbm / alg, abs=1e-4)
    assert 1.0 <= hbm / alg < 1.1  # the kernel reads its weights once
    assert sum("--pmc FETCH_SIZE" in c for c in prov["commands"]) == 2  # the kernel run and the calibration
    assert sum("--pmc WRITE_SIZE" in c for c in prov["commands"]) == 2
    assert prov["measured_at_commit"] == bench.in_graph_profile(128)["measured_at_commit"]


def test_summarize_trace_matches_both_name_forms(tmp_path):
    """One decode step of a two-layer model, half of the GEMV launches under demangled and
    half under mangled names (the profiler prints kernels with fp16 pointer arguments
    mangled); the stand-alone launches after the step are left out of the averages."""
    names = {
        "qkv": ("void (anonymous namespace)::t16_gemv_kernel<1, 1, 3, 12, 2, true, 256>(T16Args)",
                "_ZN12_GLOBAL__N_115t16_gemv_kernelILi1ELi1ELi3ELi12ELi2ELb1ELi256EEEvPKDF16_S2_7T16Args"),
        "attention": ("void (anonymous namespace)::attn_split_kernel<0, 1, false, 4, 4>(AttnParams)",) * 2,
        "o": ("void (anonymous namespace)::t16_gemv_kernel<1, 1, 16, 12, 2, true, 512>(T16Args)",
              "_ZN12_GLOBAL__N_115t16_gemv_kernelILi1ELi1ELi16ELi12ELi2ELb1ELi512EEEvPKDF16_S2_7T16Args"),
        "gate_up": ("void (anonymous namespace)::t16_gemv_kernel<1, 2, 2, 12, 2, true, 256>(T16Args)",
                    "_ZN12_GLOBAL__N_115t16_gemv_kernelILi1ELi2ELi2ELi12ELi2ELb1ELi256EEEvPKDF16_S2_7T16Args"),
        "down": ("void (anonymous namespace)::t16_gemv_kernel<1, 1, 1, 12, 2, true, 512>(T16Args)",
                 "_ZN12_GLOBAL__N_115t16_gemv_kernelILi1ELi1ELi1ELi12ELi2ELb1ELi512EEEvPKDF16_S2_7T16Args"),
    }
    rows, t = [], 0
    durations = {"qkv": 8.0, "attention": 5.0, "o": 6.0, "gate_up": 11.0, "down": 8.5}

    def add(name, us):
        nonlocal t
        rows.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += int(us * 1000) + 500

    add("set_params_kernel(int*, long const*)", 4.0)
    for layer in range(2):
        for key, us in durations.items():
            add(names[key][layer], us + layer)  # layer 0 demangled, layer 1 mangled
    add("_ZN12_GLOBAL__N_115t16_gemv_kernelILi1ELi1ELi0ELi12ELi2ELb1ELi512EEEvPKDF16_S2_7T16Args", 13.0)
    for key in durations:  # stand-alone launches after the step: excluded
        add(names[key][1], 100.0)
    path = tmp_path / "trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)
    out = bench.summarize_trace(str(path), n_steps=1, n_layer=2)
    assert set(out) == set(durations) | {"lm_head", "set_params"}
    for key, us in durations.items():
        assert out[key]["avg_us"] == pytest.approx(us + 0.5) and out[key]["calls"] == 2
    assert out["lm_head"]["avg_us"] == pytest.approx(13.0) and out["set_params"]["avg_us"] == pytest.approx(4.0)
