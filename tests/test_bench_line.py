"""The benchmark's stdout JSON line stays short enough to be read back from a
bounded output tail, and keeps the fields the benchmark contract names."""

import json

import bench


def _big_leg(i: int) -> dict:
    sub = {f"case_{j}": {"us_per_call": 10.0 + j, "reference_us_per_call": 20.0 + j, "gbps": 1000.0 + j,
                         "samples": list(range(50)), "note": "x" * 200} for j in range(20)}
    return dict(sub, workload=f"leg{i}", us_per_layer_call=12.345678, hbm_gbps=4321.0, hbm_frac=0.54,
                frac_of_gather_floor=0.9, spread={"p10": 1.0, "p90": 2.0, "list": list(range(500))},
                kv_gather_floor={"us_per_layer_call": 11.1, "gbps": 5000.0, "spread": list(range(100)),
                                 "best": {"mechanism": "registers", "us_per_layer_call": 11.1},
                                 "mechanisms": {f"mech_{j}": {"us_per_layer_call": 11.1 + j, "workgroups": 512,
                                                              "gbps": 5000.0} for j in range(6)}},
                cpu_baseline={"value": 1.5e5, "unit": "us/layer-call", "cores": 16, "kind": "port",
                              "sample": "y" * 300, "cpu_model": "z" * 50},
                throughput={"native": {"decode_tokens_per_s": 2800.0, "wall_s": 10.0}},
                prompts=list(range(400)))


def _line() -> dict:
    return {
        "metric": "verify/decode attn µs per layer + HBM GB/s (% peak), Qwen3-8B B=16 q_len=5",
        "value": 37.8, "unit": "us/layer-call", "n_gpus": 1, "steps": 20, "warmup": 5, "ms_per_step": 1.36,
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "target_verify: ...", "batch": 16, "q_len": 5, "seed": 0},
        "roofline": {"bound": "hbm", "achieved": 4200.0, "peak": 8000.0, "unit": "GB/s", "frac": 0.52,
                     "traffic": 1.6e8},
        "cpu_baseline": {"value": 7.8e4, "unit": "us/layer-call", "cores": 16, "kind": "port",
                         "sample": "20 layer calls"},
        "probes": bench._compact_probes({"copy_gbps": 5000.0,
                                         "empty_launch_in_graph": {"one_workgroup": 1.8, "two_per_cu": 1.9,
                                                                   "us_per_launch": 1.9},
                                         "stream_read": {"gbps": 6100.0, "us": 700.0,
                                                         "sweep": [{"gbps": 1.0}] * 100,
                                                         "best": {"gbps": 6200.0, "grid": 1024, "unroll": 8}}}),
    }


def test_stdout_line_fits_and_parses():
    secondary = {f"leg{i}": _big_leg(i) for i in range(12)}
    text = bench.stdout_line(_line(), secondary)
    assert len(text.encode()) <= bench.LINE_MAX_BYTES
    parsed = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in parsed
    assert parsed["roofline"]["traffic"] == 1.6e8
    assert parsed["probes"]["stream_read"]["best"]["grid"] == 1024
    assert "sweep" not in parsed["probes"]["stream_read"]
    assert parsed["probes"]["empty_launch_in_graph"]["us_per_launch"] == 1.9


def test_compact_leg_keeps_headline_figures():
    leg = bench.compact_leg(_big_leg(0))
    assert leg["us_per_layer_call"] == 12.346
    assert leg["frac_of_gather_floor"] == 0.9
    assert leg["kv_gather_floor"]["us_per_layer_call"] == 11.1
    assert leg["kv_gather_floor"]["best"] == "registers"
    assert leg["kv_gather_floor"]["mechanisms_us"]["mech_5"] == 16.1
    assert leg["cpu_baseline"] == {"value": 1.5e5, "unit": "us/layer-call", "cores": 16, "kind": "port"}
    assert leg["throughput"]["native"]["decode_tokens_per_s"] == 2800.0
    assert "prompts" not in leg and "spread" not in leg


def test_few_legs_keep_their_detail():
    text = bench.stdout_line(_line(), {"a": {"us_per_layer_call": 1.0, "x": {"us_per_call": 2.0}}})
    assert json.loads(text)["secondary"]["a"]["x"]["us_per_call"] == 2.0
