"""CPU checks of bench.py's accounting: algorithmic byte counts per activation
storage type, the profile-traffic lookup's coverage, and the one-GPU guard."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_attention_bytes_split_by_activation_type():
    N, E = 7, 53
    # fp32: every term at 4 bytes, counted tensor by tensor
    fwd32 = 4 * (N * 128 * 8 * 2 + N * 9 * 256 + N * 20 * 256 + N * 3 * 128 + E * 256 + E * 5 + N + 1)
    assert bench.attn_fwd_bytes(N, E) == fwd32
    row32 = 4 * (N * 20 * 256 * 2 + N * 1024 * 3 + N * 9 * 256 + N * 3 * 128 + E * (256 + 5 + 256 + 4 + 256))
    col32 = 4 * (N * 20 * 256 + N * 1024 * 2 + N * 9 * 256 + 2 * N + E * (256 + 5))
    assert bench.attn_bwd_bytes(N, E) == row32 + col32
    # bf16 storage halves exactly the activation terms: q, k, v, out, grad
    act_fwd = N * (128 * 8 * 2 + 9 * 256 + 20 * 256)
    assert fwd32 - bench.attn_fwd_bytes(N, E, 2) == 2 * act_fwd
    act_bwd = N * (2 * 20 * 256 + 2 * 1024 + 9 * 256) + N * (20 * 256 + 1024)
    assert row32 + col32 - bench.attn_bwd_bytes(N, E, 2) == 2 * act_bwd
    # the degree kernels read and write fp32 in both modes
    assert bench.deg_fwd_bytes(N, E, 2) == bench.deg_fwd_bytes(N, E)


def test_profile_traffic_only_for_the_profiled_workload():
    t = bench.traffic_from_profile("e2v2_attn_bwd")
    assert t is not None and t > 1e9
    assert bench.traffic_from_profile("e2v2_attn_bwd", bf16=True) is None
    assert bench.traffic_from_profile("e2v2_attn_bwd", False, 5) is None
    assert bench.traffic_from_profile("e2v2_not_an_entry") is None


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]
