"""CPU checks of bench.py's bookkeeping: the algorithmic work it prices the
rooflines with, the counter-file reader of its HBM traffic passes, and the
refusal of a multi-GPU run."""

from __future__ import annotations

import dataclasses
import subprocess
import sys
from pathlib import Path

import bench
from cutriton_amd import workloads

ROOT = Path(__file__).resolve().parents[1]


def test_conv_family_bytes_and_flops_at_batch_32():
    # The profile engine's graph is declared at batch 1; bench resolves it
    # at the run batch. 53 fused conv nodes, 3587.7 MB and 261.7 GFLOP of
    # conv + classifier work per bs32 step.
    g = workloads.resnet50(1)
    at32 = dataclasses.replace(g, inputs={"input": ((32, 3, 224, 224), "float32", "NCHW")})
    total, launches = bench.conv_family_bytes(at32)
    assert launches == 53
    assert abs(total / 1e6 - 3587.67) < 0.01
    assert abs(sum(workloads.node_flops(at32).values()) / 1e9 - 261.708) < 0.001
    # Linear in the batch for activations, constant for weights.
    total1, _ = bench.conv_family_bytes(g)
    weights = sum(4 * arr.size for name, (arr, _) in g.constants.items()
                  if any(n.op_type == "Conv" and n.inputs[1] == name for n in g.nodes))
    assert total - weights == 32 * (total1 - weights)


def test_ffn_gemm_bytes():
    gelu, gemm = bench.ffn_gemm_bytes(4096, 1024, 4096)
    # X, W1, b1 in and [M, I] out; [M, I], W2, b2 in and [M, H] out; FP16.
    assert gelu == 2 * (4096 * 1024 + 1024 * 4096 + 4096 + 4096 * 4096)
    assert gemm == 2 * (4096 * 4096 + 4096 * 1024 + 1024 + 4096 * 1024)


def test_counter_file_sums_instances_per_dispatch(tmp_path):
    path = tmp_path / "run_counter_collection.csv"
    rows = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"]
    # two dispatches of one kernel, each reported over three instances
    for dispatch, values in ((1, (10, 20, 30)), (2, (1, 2, 3))):
        rows += [f"{dispatch},relu_fp32,FETCH_SIZE,{v}" for v in values]
    rows.append("3,conv_bn_relu_fp32_m64n64,FETCH_SIZE,7.5")
    path.write_text("\n".join(rows) + "\n")
    got = bench._read_counter(str(path))
    assert sorted(got["relu_fp32"]) == [6.0, 60.0]
    assert got["conv_bn_relu_fp32_m64n64"] == [7.5]


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         cwd=ROOT, timeout=120)
    assert run.returncode == 2
    assert "one GPU" in run.stderr
