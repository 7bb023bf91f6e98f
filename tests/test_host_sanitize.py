"""The runtime's host code under AddressSanitizer and UndefinedBehaviorSanitizer: tests/native/
host_sanitize (built by brimkern_amd/build.py from host_sanitize.cpp and the runtime sources, host
code instrumented, kernels the ordinary code object) drives every C-ABI entry point. Without a device
it checks argument validation and error codes; on the GPU it runs contexts, copies, the pinned upload
ring, every matmul path, plans (the GLU pair and a pre-staged plan included), graphs, fences, top-k,
MoE, convolution, f16 weights and the encoders. A sanitizer report aborts the driver (non-zero exit)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "tests", "native", "host_sanitize")


def run(*args, timeout):
    assert os.path.exists(DRIVER), f"{DRIVER} is missing: run `python -m brimkern_amd.build`"
    p = subprocess.run([DRIVER, *args], capture_output=True, text=True, timeout=timeout)
    out = p.stdout + p.stderr
    print(out[-4000:], flush=True)
    return p.returncode, out


def test_host_paths_without_a_device():
    rc, out = run("nodev", timeout=120)
    assert rc == 0, out[-4000:]
    assert "host checks only (no device): 0 failure(s)" in out
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out


@pytest.mark.gpu
def test_every_entry_point_under_sanitizers_on_the_gpu():
    print("host_sanitize: device run", flush=True)
    rc, out = run(timeout=300)
    assert rc == 0, out[-4000:]
    assert "device checks done: 0 failure(s)" in out
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out
