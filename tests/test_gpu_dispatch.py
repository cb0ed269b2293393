"""By-name dispatch on the GPU: variant names produced by the materialization
contract, launched through loom_hip_dispatch, give bit-identical results to
the direct entry points (same kernels, same tiles), and one variant per
function is checked against the CPU oracle."""
import json

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, GEMM_TOL, _mamba_inputs, dev, devf, host, rng_bf16

pytestmark = pytest.mark.gpu

SOLVER_JSON = json.dumps({
    "matmul": [{"tile_m": 128, "tile_n": 128, "tile_k": 64},
               {"tile_m": 256, "tile_n": 256, "tile_k": 64}],
    "batch_matmul": {"tile_b": 1, "tile_m": 256, "tile_n": 256, "tile_k": 64},
    "split_k_matmul_gather": {"tile_m": 64, "tile_n": 64, "tile_k": 256},
    "attention": [{"tile_b": 1, "tile_m": 192, "tile_n": 64},
                  {"tile_b": 1, "tile_m": 64, "tile_n": 64}],
    "flash_decode": {"tile_b": 1, "tile_s": 256, "tile_n": 128},
    "helion_mamba2_chunk_scan_kernel": {"tile_b": 1, "tile_h": 1, "tile_c": 1, "tile_m": 128,
                                        "tile_n": 32, "tile_k": 64},
})


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


@pytest.fixture(scope="module")
def variants(lh):
    names = lh.materialize_variants(SOLVER_JSON)
    assert len(names) == 8
    return names


def _of(variants, func):
    return [v for v in variants if v.split("__")[0] == func]


def test_dispatch_gemms(lh, variants):
    rng = np.random.default_rng(31)
    x, y = rng_bf16(rng, (320, 192)), rng_bf16(rng, (192, 256))
    ref = oracle.matmul(x, y, 64, 64, 64)
    for v in _of(variants, "matmul"):
        _, t = lh.parse_variant(v)
        out = torch.empty((320, 256), dtype=torch.bfloat16, device="cuda")
        lh.dispatch(v, dev(x), dev(y), out)
        direct = lh.matmul(dev(x), dev(y), tile_m=t["tile_m"], tile_n=t["tile_n"],
                           tile_k=t["tile_k"])
        assert torch.equal(out, direct), v
        assert_close(from_bf16(host(out)), from_bf16(ref), **GEMM_TOL, what=v)

    a, b = rng_bf16(rng, (2, 256, 128)), rng_bf16(rng, (2, 128, 512))
    (v,) = _of(variants, "batch_matmul")
    out = torch.empty((2, 256, 512), dtype=torch.bfloat16, device="cuda")
    lh.dispatch(v, dev(a), dev(b), out)
    assert torch.equal(out, lh.batch_matmul(dev(a), dev(b), tile_m=256, tile_n=256))

    a = np.round(rng.uniform(-4, 4, (96, 640))).astype(np.float32)
    b = np.round(rng.uniform(-4, 4, (640, 128))).astype(np.float32)
    a16, b16 = oracle.to_bf16(a), oracle.to_bf16(b)
    (v,) = _of(variants, "split_k_matmul_gather")
    out = torch.empty((96, 128), dtype=torch.bfloat16, device="cuda")
    _, ws = lh.dispatch(v, dev(a16), dev(b16), out)
    parts = ws[:3 * 96 * 128 * 4].view(torch.float32).view(3, 96, 128).cpu().numpy()
    ref_out, ref_parts = oracle.split_k_matmul_gather(a16, b16, 32, 32, 256)
    np.testing.assert_array_equal(parts, ref_parts)
    np.testing.assert_array_equal(host(out), ref_out)


def test_dispatch_attention(lh, variants):
    rng = np.random.default_rng(32)
    BH, S, D = 2, 320, 128
    k = rng_bf16(rng, (BH, D, S))
    v_ = rng_bf16(rng, (BH, S, D))
    q = rng_bf16(rng, (BH, S, D))
    ref = oracle.attention(k, v_, q, 1.0 / np.sqrt(D), True)
    for name in _of(variants, "attention"):
        _, t = lh.parse_variant(name)
        out = torch.empty((BH, S, D), dtype=torch.bfloat16, device="cuda")
        lh.dispatch(name, dev(k), dev(v_), dev(q), out, causal=True)
        direct = lh.attention(dev(k), dev(v_), dev(q), causal=True, tile_m=t["tile_m"],
                              tile_n=t["tile_n"])
        assert torch.equal(out, direct), name
        assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=name)


def test_dispatch_decode(lh, variants):
    rng = np.random.default_rng(33)
    B, H, D, S = 2, 8, 128, 1000
    k = rng_bf16(rng, (B, D, S))
    v_ = rng_bf16(rng, (B, S, D))
    q = rng_bf16(rng, (B, H, D))
    (name,) = _of(variants, "flash_decode")
    out = torch.empty((B, H, D), dtype=torch.bfloat16, device="cuda")
    lh.dispatch(name, dev(k), dev(v_), dev(q), out)
    direct = lh.flash_decode(dev(k), dev(v_), dev(q), tile_s=256, tile_n=128)
    assert torch.equal(out, direct)
    ref = oracle.flash_decode(k, v_, q, 1.0 / np.sqrt(D), 1, 256, 128)[0]
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=name)


def test_dispatch_mamba(lh, variants):
    rng = np.random.default_rng(34)
    cb, x, dt, dA, C, Dh, prev = _mamba_inputs(rng, 1, 2, 4, 2, 128, 64, 64)
    (name,) = _of(variants, "helion_mamba2_chunk_scan_kernel")
    args = [dev(cb), dev(x), devf(dt), devf(dA), dev(C), devf(Dh), devf(prev)]
    out = torch.empty(x.shape, dtype=torch.bfloat16, device="cuda")
    lh.dispatch(name, *args, out)
    direct = lh.helion_mamba2_chunk_scan_kernel(*args, tile_m=128, tile_n=32)
    assert torch.equal(out, direct)
    ref = oracle.mamba_chunk_scan(cb, x, dt, dA, C, Dh, prev, 64, 64, 64)
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=name)


def test_dispatch_runs_every_aligned_binding(lh):
    """A binding with no workgroup tile of its own (tile_n 32 beside tile_m
    64, the pair the reference emits for split-K) runs on the smallest built
    tile covering it, bit-identical to that tile; a value that is neither a
    multiple of 16 nor the extent is rejected with LOOM_HIP_EINVAL."""
    rng = np.random.default_rng(35)
    x, y = rng_bf16(rng, (192, 320)), rng_bf16(rng, (320, 160))
    ref = oracle.matmul(x, y, 64, 64, 64)
    direct = lh.matmul(dev(x), dev(y), tile_m=64, tile_n=64, tile_k=64)
    for tm, tn in ((64, 32), (16, 48), (48, 160), (192, 112)):
        name = f"matmul__tile_k64__tile_m{tm}__tile_n{tn}"
        out = torch.empty((192, 160), dtype=torch.bfloat16, device="cuda")
        lh.dispatch(name, dev(x), dev(y), out)
        assert torch.equal(out, direct), name
        assert_close(from_bf16(host(out)), from_bf16(ref), **GEMM_TOL, what=name)
    out = torch.empty((192, 160), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError) as ei:
        lh.dispatch("matmul__tile_k64__tile_m64__tile_n40", dev(x), dev(y), out)
    assert ei.value.code == 1
