"""CPU checks of bench.py's contract: one GPU only (--gpus N > 1 exits with a
message, before touching a device), and the per-unit figures behind the
roofline line (algorithmic flops and bytes of the C2 launch)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and r.stdout == ""


def test_c2_roofline_units():
    """4*hd flops per kept (query, key, head) triple; C2 keeps 1,223,168
    (query, key) pairs x 12 heads = 14,678,016 triples -> 3.758 GFLOP per
    launch; algorithmic bytes = qkv read once + out written once + the packed
    keep words."""
    import bench
    from tenferro_ext.workloads import laya_config

    w = laya_config(2)
    pairs = w.kept_pairs()
    assert pairs == 1_223_168
    assert 4 * w.head_dim * pairs * w.heads == 3_757_572_096
    words = 4 * w.length * w.batch * ((w.length + 31) // 32)
    assert bench.laya_bytes(w) == 4 * 3 * 768 * 512 * 8 + 4 * 768 * 512 * 8 + words
