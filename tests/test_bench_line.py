"""The line `bench.py` prints for the driver, built from synthetic records of
every workload the default run times: one JSON object, short enough for the
driver's record to keep it whole (the reference harness prints one compact
row per case, benches/nn_ops.rs:185-252)."""

import json

import bench
from bench import Timing


def _workloads():
    t = Timing.of(0.0123456, [0.0123456 + 1e-4 * i for i in range(15)])
    lines = []
    cpu = {"value": 0.0190123, "unit": "TFLOP/s", "cores": 1, "kind": "port", "sample": "s" * 200,
           "cpu": "AMD EPYC 9575F 64-Core Processor", "nproc": 128}
    for kind, shape in (("f32", "4096x4096x4096"), ("f16", "16384x1024x4096")):
        lines.append({"workload": f"{kind} GEMM {shape}", "key": f"gemm {kind} {shape}", "value": 129.123456,
                      "unit": "TFLOP/s", "ms": t, "spread": bench.spread(t), "cpu_baseline": cpu,
                      "roofline": {"bound": "mfma", "achieved": 129.1, "peak": 157.3, "unit": "TFLOP/s",
                                   "frac": 0.8212345, "traffic": 8.246e8, "bytes": 2.01e8}})
    for size in ("32M", "512M"):
        for name in ("sum[2]", "max[2]", "min[2]", "mean[2]", "var[2]", "sum[0,1]", "max[0,1]", "var[0,1]",
                     "argmax[1]", "argmin[1]"):
            lines.append(bench.with_cpu(bench.hbm_line("a long descriptive workload name " * 3, 3.4e7, t,
                                                       f"{name} {size}"), cpu))
    keys = ["x*y", "t+z", "permute", "slice", "concat", "add", "matvec", "vecmat", "dot", "transpose", "adam",
            "layernorm 1 kernel", "layernorm composed", "launch floor", "mlp step"]
    keys += [f"dense {kind} {shape} {form}" for kind, shape in (("f32", "4096x1024x4096"), ("bf16", "8192x8192x8192"))
             for form in ("epilogue", "unfused", "product")]
    for key in keys:
        lines.append(bench.with_cpu(bench.hbm_line("another long workload name " * 3, 5.4e8, t, key), cpu))
    return lines


def test_the_driver_line_is_compact_and_complete():
    workloads = _workloads()
    head = {"value": 1514.0123456, "ms": 0.726123456, "spread": bench.spread(Timing.of(0.726, [0.726] * 20)),
            "roofline": {"bound": "mfma", "achieved": 1514.0, "peak": 2516.6, "unit": "TFLOP/s", "frac": 0.6016,
                         "traffic": None, "kernel_ms": 0.726, "bytes": 4.03e8}}
    cpu = {"value": 0.0145, "unit": "TFLOP/s", "cores": 1, "kind": "port", "sample": "rows " * 40,
           "cpu": "AMD EPYC 9575F 64-Core Processor", "nproc": 128}
    line = bench.headline_line(head, cpu, workloads, 20, 30, "AMD Instinct MI355X gfx950")
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) < 4000, len(text)
    back = json.loads(text)
    for field in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                  "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert field in back, field
    assert back["roofline"]["traffic"] == bench.HEADLINE_TRAFFIC
    assert back["roofline"]["peak"] == 2516.6
    assert back["cpu_baseline"]["cores"] == 1 and back["cpu_baseline"]["nproc"] == 128
    assert back["spread"]["samples"] == 20
    # Every workload keeps its own row, under a distinct key.
    assert len(back["workloads"]) == len(workloads)
    row = back["workloads"]["gemm f32 4096x4096x4096"]
    assert dict(zip(back["workload_fields"], row))["traffic_ratio"] == round(8.246e8 / 2.01e8, 2)


def test_timing_statistics_follow_the_reference_harness():
    # Median, minimum and the median absolute deviation over the median
    # (benches/nn_ops.rs:239-251).
    t = Timing.of(2.0, [1.0, 2.0, 3.0, 10.0, 2.0])
    assert float(t) == 2.0 and t.median == 2.0 and t.low == 1.0
    assert t.mad == 0.5  # deviations 1, 0, 1, 8, 0 -> median 1, over 2
    assert t.samples == 5
