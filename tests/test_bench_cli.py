"""bench.py's contract on the host: a request for more than one GPU exits with a message (this path is measured on
one GPU), and the committed HBM-traffic summary that the bench line's `roofline.traffic` is read from stays
parseable and calibrated. No GPU is touched."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_traffic_summary_is_parseable_and_calibrated():
    sys.path.insert(0, ROOT)
    import bench

    traffic = bench.measured_traffic()
    assert "swiglu_bias" in traffic
    import workloads as W

    # the workload kernel's measured HBM bytes sit within 1% of its algorithmic bytes
    assert abs(traffic["swiglu_bias"] / W.ALGO_BYTES["swiglu_bias"] - 1.0) < 0.01
    text = open(os.path.join(ROOT, "profiles", "hbm_traffic_per_op.md")).read()
    block = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    assert 1.9 < block["fetch_scale"] < 2.1 and 0.95 < block["write_scale"] < 1.05
    # every op of the bench has its own measured traffic, and none reads below its algorithmic bytes
    same = {"rmsnorm_residual_separate": "rmsnorm_residual", "rope_qk_separate": "rope_qk", "argmax_topk_k1": "argmax"}
    for name, t in traffic.items():
        algo = W.ALGO_BYTES.get(same.get(name, name))
        if algo is not None:
            assert t >= 0.99 * algo, name
