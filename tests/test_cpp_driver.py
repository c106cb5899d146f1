"""The C++ host of the C ABI (tenferro-decision-rs_amd/drivers/tfd_driver.cpp):
a program that links libtfd_attention.so directly, without Python or torch,
as an engine would. CPU: it is built, reports the ABI, and validates
arguments without a device. GPU: its closed-form checks of both drop-in ops
pass through host and device pointers, and its C2 timing runs."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tenferro-decision-rs_amd", "_build", "tfd_driver")


def run(mode, timeout=120):
    return subprocess.run([DRIVER, mode], capture_output=True, text=True, timeout=timeout)


def test_driver_reports_the_abi():
    assert os.path.exists(DRIVER), "build the library first (make -C tenferro-decision-rs_amd)"
    r = run("abi")
    assert r.returncode == 0
    assert r.stdout.split() == ["abi", "2", "tenferro-decision.laya_attention_block.v1",
                                "tenferro-decision.jeff_full_attention.v1"]


def test_driver_without_gpu_validates_and_refuses_compute():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = run("check")
    assert r.returncode == 77, r.stdout + r.stderr
    assert "validation works" in r.stdout and "attention block expects (3d, L, B)" in r.stdout


@pytest.mark.gpu
def test_driver_closed_form_checks_gpu():
    print("[driver] check", flush=True)
    r = run("check")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout and r.stdout.count("PASS") == 9
    assert "0 failure(s)" in r.stdout


@pytest.mark.gpu
def test_driver_bench_gpu():
    print("[driver] bench", flush=True)
    r = run("bench")
    assert r.returncode == 0, r.stdout + r.stderr
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["tflops"] > 10.0
