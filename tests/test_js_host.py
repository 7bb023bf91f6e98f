"""The JavaScript host (brimkern_amd/js over the N-API addon brik.node).

CPU: the addon loads under this image's Node, exports every entry point the facade uses, the facade's
layout helpers agree with the Python layout module, and with no GPU present context creation fails
loudly with BRIK_ENODEV (there is no CPU fallback).
GPU: tests/js/engine_parity.js checks the reference-shaped readback ops on the golden fixtures, dequant
bit-exactness, a seeded Qwen3-4B-shaped q4 GEMV against the JavaScript CPU reference, the recMM form,
a grouped plan and the error codes.
"""
import json
import os
import shutil
import subprocess

import pytest

from brimkern_amd import layout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "brimkern_amd", "js", "brik.node")
NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node not installed")

EXPORTS = ["deviceCount", "createContext", "alloc", "free", "h2d", "d2h", "sync", "setOption", "timerBegin",
           "timerEnd", "matmulQ8", "matmulQ4", "matmulQ3", "moeMatmulQ4", "dequantQ8", "dequantQ4", "dequantQ3",
           "gemvPlanCreate", "gemvPlanCreateGlu", "gemvPlanRun", "gemvPlanDestroy", "logitsTopK", "lmHeadTopK", "quantize",
           "f16ToF32", "conv2d", "matmulF16W", "allocBuffer", "bufferPtr", "freeBuffer", "liveBuffers",
           "readbackAsync", "selfValidate", "moeMatmulQ4x2", "h2dAsync", "graphBegin", "graphEnd", "graphLaunch",
           "graphDestroy"]


def node(script, timeout=120):
    return subprocess.run([NODE, "-e", script], cwd=ROOT, capture_output=True, text=True, timeout=timeout)


def test_addon_exports():
    assert os.path.exists(ADDON), "brik.node is not built (python -m brimkern_amd.build)"
    r = node("console.log(JSON.stringify(Object.keys(require('./brimkern_amd/js/brik.node'))))")
    assert r.returncode == 0, r.stderr
    assert sorted(json.loads(r.stdout)) == sorted(EXPORTS)


def test_js_plane_offsets_match_python():
    cases = [(f, n) for f in ("q8", "q4", "q3") for n in (32, 96, 2560 * 4096)]
    r = node("const p = require('./brimkern_amd/js/planes'); console.log(JSON.stringify(" +
             json.dumps(cases) + ".map(c => [p.byteLength(c[0], c[1]), p.planeOffsets(c[0], c[1])])))")
    assert r.returncode == 0, r.stderr
    for (fmt, n), (blen, offs) in zip(cases, json.loads(r.stdout)):
        assert blen == layout.byte_length(fmt, n)
        assert {k: tuple(v) for k, v in offs.items()} == layout.plane_offsets(fmt, n)


def test_no_device_fails_loudly():
    r = node("const b = require('./brimkern_amd/js'); if (b.Engine.deviceCount() > 0) { console.log('gpu'); }"
             " else { try { new b.Engine(0); console.log('created'); } catch (e) { console.log(e.code); } }")
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() in ("gpu", "BRIK_ENODEV")


@pytest.mark.gpu
def test_js_engine_parity_on_gpu():
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "engine_parity.js")], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["failed"] == 0 and res["checks"] >= 20


@pytest.mark.gpu
def test_js_engine_async_and_lifetime_on_gpu():
    """Readbacks through fences off the JS thread, rejection instead of throwing, finalizers freeing
    dropped device buffers (and keeping their context alive), selfValidate passing, the scratch pool and
    recMM's pooled outputs, recorded launches, readback ops issued behind a long queue returning at once."""
    r = subprocess.run([NODE, "--expose-gc", os.path.join(ROOT, "tests", "js", "engine_async.js")], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["failed"] == 0 and res["checks"] >= 30
