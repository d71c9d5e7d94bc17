"""bench.py's contract on the CPU: one GPU only (a clear refusal otherwise),
the algorithmic work it divides by, and the counted traffic it reports from
the committed rocprofv3 summary."""
import json
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout.strip()


def test_step_flops_and_compulsory_bytes():
    # forward 2·B·Σ din·dout, dW the same, dX for layers 1..: 17.31 GF at batch 2048
    d, b = bench.DIMS, bench.BATCH
    fwd = sum(2 * b * d[l] * d[l + 1] for l in range(len(d) - 1))
    dx = sum(2 * b * d[l] * d[l + 1] for l in range(1, len(d) - 1))
    assert bench.step_flops(d, b) == 2 * fwd + dx == 17_305_698_304
    # batch-32 SGD step: W read by the forward and by dX (layers 1, 2), dW
    # written, θ and g read and θ written (20 B per parameter)
    w = sum(d[l] * d[l + 1] for l in range(len(d) - 1))
    p = w + sum(d[1:])
    assert bench.c1_bytes(d) == 20 * p + 4 * (d[1] * d[2] + d[2] * d[3]) == 35_938_504
    # per-launch FLOPs of the plan's labels
    assert bench.label_flops("dwdx_l1", d, b) == 2 * 2 * b * 1024 * 1024
    assert bench.label_flops("fwd_l0", d, b) == 2 * b * 512 * 1024
    assert bench.label_flops("optimizer", d, b) == 0


def test_reported_traffic_comes_from_the_committed_counts():
    with open(os.path.join(ROOT, "profiles", "pmc_traffic.json")) as f:
        doc = json.load(f)
    for label in ("fwd_l0", "fwd_l1", "head_xent", "dwdx_l2", "dwdx_l1", "dw_l0", "optimizer"):
        row = doc[label]
        assert bench.traffic_for(label) == row["bytes_per_launch"] > 0
        # the scaled counters add up to the reported bytes (FETCH_SIZE counts
        # half of what a copy of known size reads, WRITE_SIZE all it writes)
        assert abs(row["fetch_kib"] * 1024 * 2 + row["write_kib"] * 1024 - row["bytes_per_launch"]) \
            <= 1e-3 * row["bytes_per_launch"]
    sb = doc["small_batch"]
    per_step = sum(v["bytes_per_launch"] for k, v in sb.items() if isinstance(v, dict))
    assert bench.traffic_for(None, "small_batch", "bytes_per_step") == sb["bytes_per_step"] == per_step
    assert sb["algorithmic_bytes_per_step"] == bench.c1_bytes(bench.DIMS)
