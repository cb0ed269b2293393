"""loom_hip_flash_decode_noalloc on the GPU, through the C ABI: the
allocation-free form (split partials in the library's static per-device
scratch) gives bit-identical results to loom_hip_flash_decode with a caller
workspace -- the same kernels and the same splits -- on two calls in a row,
the second smaller than the first (the scratch keeps the first call's
partials, which the second must not read), and matches the CPU oracle."""
import ctypes
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _abi(lh, name, *args):
    err = ctypes.create_string_buffer(512)
    rc = getattr(lh._lib, name)(*args, err, len(err))
    assert rc == 0, (name, rc, err.value.decode())


def _inputs(B, H, D, S, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, D, S), generator=g).to(torch.bfloat16).cuda()
    v = torch.randn((B, S, D), generator=g).to(torch.bfloat16).cuda()
    q = torch.randn((B, H, D), generator=g).to(torch.bfloat16).cuda()
    return k, v, q


@pytest.mark.parametrize("calls", [((32, 32, 128, 8192, 1024), (2, 8, 64, 1000, 128),
                                     (3, 32, 128, 1001, 256))])
def test_noalloc_matches_workspace_form(lh, calls):
    """Three calls in a row, each smaller than the first; the last has S not a
    multiple of 8, so it takes the register-load split kernel."""
    stream = torch.cuda.current_stream().cuda_stream
    for B, H, D, S, ts in calls:
        print(f"noalloc B{B} H{H} D{D} S{S} tile_s{ts}", flush=True)
        k, v, q = _inputs(B, H, D, S, seed=B * 1000 + S)
        scale = 1.0 / math.sqrt(D)
        out_na = torch.full((B, H, D), float("nan"), dtype=torch.bfloat16, device="cuda")
        _abi(lh, "loom_hip_flash_decode_noalloc", k.data_ptr(), v.data_ptr(), q.data_ptr(),
             out_na.data_ptr(), B, H, D, S, ctypes.c_float(scale), 1, ts, min(ts, 128), stream)
        ws_bytes = lh.flash_decode_workspace_bytes(B, H, D, S, ts)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        out_ws = torch.empty((B, H, D), dtype=torch.bfloat16, device="cuda")
        _abi(lh, "loom_hip_flash_decode", k.data_ptr(), v.data_ptr(), q.data_ptr(),
             out_ws.data_ptr(), ws.data_ptr(), ws_bytes, B, H, D, S, ctypes.c_float(scale), 1, ts,
             min(ts, 128), stream)
        torch.cuda.synchronize()
        assert torch.equal(out_na.view(torch.int16), out_ws.view(torch.int16)), (B, H, D, S, ts)
        hk, hv, hq = (t.view(torch.int16).cpu().numpy().view(np.uint16) for t in (k, v, q))
        ref = oracle.flash_decode(hk, hv, hq, scale, 1, ts, 128)[0]
        got = out_na.view(torch.int16).cpu().numpy().view(np.uint16)
        assert_close(from_bf16(got), from_bf16(ref), atol=2e-2, rtol=1e-2,
                     what=f"noalloc B{B} S{S}")


CAPTURE_SCRIPT = r"""
import ctypes, math, sys
import torch
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/loom-dataflow_amd"]
import loom_hip
B, H, D, S, ts = 2, 32, 128, 2048, 512
g = torch.Generator().manual_seed(7)
k = torch.randn((B, D, S), generator=g).to(torch.bfloat16).cuda()
v = torch.randn((B, S, D), generator=g).to(torch.bfloat16).cuda()
q = torch.randn((B, H, D), generator=g).to(torch.bfloat16).cuda()
scale = ctypes.c_float(1.0 / math.sqrt(D))
def call(out):
    err = ctypes.create_string_buffer(512)
    rc = loom_hip._lib.loom_hip_flash_decode_noalloc(
        k.data_ptr(), v.data_ptr(), q.data_ptr(), out.data_ptr(), B, H, D, S, scale, 1, ts, 128,
        torch.cuda.current_stream().cuda_stream, err, len(err))
    return rc, err.value.decode()
side = torch.cuda.Stream()
out_g = torch.zeros((B, H, D), dtype=torch.bfloat16, device="cuda")
torch.cuda.synchronize()
# first call of the process, under capture: refused, nothing recorded
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    graph.capture_begin()
    rc, msg = call(out_g)
    graph.capture_end()
print("captured-first", rc, msg, flush=True)
assert rc == 1 and "outside graph capture" in msg, (rc, msg)
# one call outside capture resolves the scratch; a captured call then runs
out_e = torch.empty((B, H, D), dtype=torch.bfloat16, device="cuda")
rc, msg = call(out_e)
assert rc == 0, msg
torch.cuda.synchronize()
graph2 = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    graph2.capture_begin()
    rc, msg = call(out_g)
    graph2.capture_end()
assert rc == 0, msg
for rep in range(3):
    out_g.zero_()
    graph2.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16)), rep
print("capture-ok", flush=True)
"""


def test_noalloc_first_call_under_capture(lh):
    """In a fresh process: a first call made while its stream is being
    captured is refused with a clear message (the scratch address lookup is
    not made under capture), and after one eager call the captured call
    replays bit-identical to the eager result."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", CAPTURE_SCRIPT, root], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "capture-ok" in r.stdout, r.stdout + r.stderr
