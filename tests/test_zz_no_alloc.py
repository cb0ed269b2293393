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


@pytest.mark.parametrize("first,second", [((32, 32, 128, 8192, 1024), (2, 8, 64, 1000, 128))])
def test_noalloc_matches_workspace_form(lh, first, second):
    stream = torch.cuda.current_stream().cuda_stream
    for B, H, D, S, ts in (first, second):
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
