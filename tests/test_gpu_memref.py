"""The memref-descriptor entry points on the GPU.

Every argument lives inside a larger buffer at a nonzero element offset and
is passed as an MLIR ranked descriptor (aligned = the buffer, offset = the
view's element offset), the way a `_mlir_ciface_` caller holds it.  Each
argument carries its own seeded data (distinct per argument, so any swap or
wrong offset changes the result); the outputs must be bit-identical to the
pointer entry points on the same data and match the CPU oracle.  The
buffer regions around each output must stay untouched."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16, to_bf16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, GEMM_TOL, _mamba_inputs, dev, devf, host

pytestmark = pytest.mark.gpu

PAD = 24   # elements before (and after) each view inside its buffer: 48 bytes of bf16


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def embed(t, pad=PAD, fill=7.0):
    """A copy of t living at element offset `pad` of a larger buffer filled
    with `fill`: (view, buffer)."""
    buf = torch.full((t.numel() + 2 * pad,), fill, dtype=t.dtype, device=t.device)
    view = buf[pad:pad + t.numel()].view(t.shape)
    view.copy_(t)
    return view, buf


def guard_ok(view, buf, pad=PAD, fill=7.0):
    f = torch.tensor(fill, dtype=buf.dtype, device=buf.device)
    return bool((buf[:pad] == f).all()) and bool((buf[pad + view.numel():] == f).all())


def test_matmul_and_bmm_descriptors(lh):
    rng = np.random.default_rng(61)
    x, y = to_bf16(rng.integers(-4, 5, (200, 136)).astype(np.float32)), \
        to_bf16(rng.integers(-4, 5, (136, 264)).astype(np.float32))
    ref = oracle.matmul(x, y)
    xv, xb = embed(dev(x))
    yv, yb = embed(dev(y))
    ov, ob = embed(torch.zeros((200, 264), dtype=torch.bfloat16, device="cuda"))
    lh.ciface("matmul", lh.memref(xv, base=xb), lh.memref(yv, base=yb), lh.memref(ov, base=ob),
              tile_m=128, tile_n=128, tile_k=64)
    torch.cuda.synchronize()
    assert np.array_equal(host(ov), ref)
    assert guard_ok(ov, ob)
    # PAD = 24 elements is 16-byte aligned; an offset of one element is not:
    # the GEMM then runs its element-store kernel, with the same bits
    ov1, ob1 = embed(torch.zeros((200, 264), dtype=torch.bfloat16, device="cuda"), pad=PAD + 1)
    assert ov1.data_ptr() % 16 != 0
    lh.ciface("matmul", lh.memref(xv, base=xb), lh.memref(yv, base=yb), lh.memref(ov1, base=ob1),
              tile_m=128, tile_n=128, tile_k=64)
    torch.cuda.synchronize()
    assert np.array_equal(host(ov1), ref) and guard_ok(ov1, ob1, pad=PAD + 1)

    a = torch.from_numpy(rng.standard_normal((3, 256, 128)).astype(np.float32) * 0.1).to(
        torch.bfloat16).cuda()
    b = torch.from_numpy(rng.standard_normal((3, 128, 320)).astype(np.float32) * 0.1).to(
        torch.bfloat16).cuda()
    av, ab = embed(a)
    bv, bb = embed(b)
    cv, cb_ = embed(torch.zeros((3, 256, 320), dtype=torch.bfloat16, device="cuda"))
    lh.dispatch_memref("batch_matmul__tile_b1__tile_k64__tile_m256__tile_n256",
                       lh.memref(av, base=ab), lh.memref(bv, base=bb), lh.memref(cv, base=cb_))
    direct = lh.batch_matmul(a, b, tile_m=256, tile_n=256)
    torch.cuda.synchronize()
    assert torch.equal(cv, direct) and guard_ok(cv, cb_)


def test_split_k_descriptors(lh):
    rng = np.random.default_rng(62)
    a = to_bf16(rng.integers(-4, 5, (96, 2048)).astype(np.float32))
    b = to_bf16(rng.integers(-4, 5, (2048, 128)).astype(np.float32))
    o_ref, p_ref = oracle.split_k_matmul_gather(a, b, 32, 32, 512)
    av, ab = embed(dev(a))
    bv, bb = embed(dev(b))
    ov, ob = embed(torch.zeros((96, 128), dtype=torch.bfloat16, device="cuda"))
    parts = torch.empty((4, 96, 128), dtype=torch.float32, device="cuda")
    lh.ciface("split_k_matmul_gather", lh.memref(av, base=ab), lh.memref(bv, base=bb),
              lh.memref(ov, base=ob), workspace=parts.view(torch.uint8).view(-1), tile_m=64,
              tile_n=64, tile_k=512)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(parts.cpu().numpy(), p_ref)
    np.testing.assert_array_equal(host(ov), o_ref)
    assert guard_ok(ov, ob)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_descriptors(lh, causal):
    rng = np.random.default_rng(63)
    BH, S, D = 2, 320, 128
    k = to_bf16(rng.standard_normal((BH, D, S)).astype(np.float32))
    v = to_bf16(rng.standard_normal((BH, S, D)).astype(np.float32))
    q = to_bf16(rng.standard_normal((BH, S, D)).astype(np.float32))
    views = [embed(dev(t)) for t in (k, v, q)]
    ov, ob = embed(torch.zeros((BH, S, D), dtype=torch.bfloat16, device="cuda"))
    lh.ciface("attention", *[lh.memref(vw, base=bf) for vw, bf in views], lh.memref(ov, base=ob),
              scale=1 / math.sqrt(D), causal=causal, tile_b=1, tile_m=128, tile_n=64)
    direct = lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=128, tile_n=64)
    torch.cuda.synchronize()
    assert torch.equal(ov, direct) and guard_ok(ov, ob)
    ref = oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64)
    assert_close(from_bf16(host(ov)), from_bf16(ref), **ATTN_TOL, what="attention memref")


def test_decode_descriptors(lh):
    rng = np.random.default_rng(64)
    B, H, D, S = 3, 32, 128, 1000
    k = to_bf16(rng.standard_normal((B, D, S)).astype(np.float32))
    v = to_bf16(rng.standard_normal((B, S, D)).astype(np.float32))
    q = to_bf16(rng.standard_normal((B, H, D)).astype(np.float32))
    views = [embed(dev(t)) for t in (k, v, q)]
    ov, ob = embed(torch.zeros((B, H, D), dtype=torch.bfloat16, device="cuda"))
    ws = lh.flash_decode_workspace(B, H, D, S, 256, "cuda")
    lh.dispatch_memref("flash_decode__tile_b1__tile_n128__tile_s256",
                       *[lh.memref(vw, base=bf) for vw, bf in views], lh.memref(ov, base=ob),
                       workspace=ws, scale=1 / math.sqrt(D))
    direct = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=256, tile_n=128)
    torch.cuda.synchronize()
    assert torch.equal(ov, direct) and guard_ok(ov, ob)
    ref = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 256, 128)[0]
    assert_close(from_bf16(host(ov)), from_bf16(ref), **ATTN_TOL, what="decode memref")


def test_mamba_descriptors_bf16_and_f16(lh):
    rng = np.random.default_rng(65)
    cb, x, dt, dA, C, Dh, prev = _mamba_inputs(rng, 1, 2, 4, 2, 128, 64, 64)
    tensors = [dev(cb), dev(x), devf(dt), devf(dA), dev(C), devf(Dh), devf(prev)]
    views = [embed(t) for t in tensors]
    ov, ob = embed(torch.zeros(x.shape, dtype=torch.bfloat16, device="cuda"))
    tiles = dict(tile_b=1, tile_h=1, tile_c=1, tile_m=128, tile_n=32, tile_k=64)
    lh.ciface("helion_mamba2_chunk_scan_kernel", *[lh.memref(vw, base=bf) for vw, bf in views],
              lh.memref(ov, base=ob), **tiles)
    direct = lh.helion_mamba2_chunk_scan_kernel(*tensors, tile_m=128, tile_n=32)
    torch.cuda.synchronize()
    assert torch.equal(ov, direct) and guard_ok(ov, ob)
    ref = oracle.mamba_chunk_scan(cb, x, dt, dA, C, Dh, prev, 64, 64, 64)
    assert_close(from_bf16(host(ov)), from_bf16(ref), **ATTN_TOL, what="mamba memref")

    # the reference's own signature: every tensor f16 (dt, dA_cumsum, D, prev
    # included), through loom_hip_ciface_helion_mamba2_chunk_scan_kernel_f16
    h16 = lambda a: np.asarray(a, np.float32).astype(np.float16)  # noqa: E731
    b16 = lambda u: from_bf16(u).astype(np.float16)  # noqa: E731
    arrs = [b16(cb), b16(x), h16(dt), h16(dA), b16(C), h16(Dh), h16(prev)]
    t16 = [torch.from_numpy(a).cuda() for a in arrs]
    views = [embed(t) for t in t16]
    ov, ob = embed(torch.zeros(x.shape, dtype=torch.float16, device="cuda"))
    lh.ciface("helion_mamba2_chunk_scan_kernel", *[lh.memref(vw, base=bf) for vw, bf in views],
              lh.memref(ov, base=ob), f16=True, **tiles)
    torch.cuda.synchronize()
    assert guard_ok(ov, ob)
    with oracle.element_type("f16"):
        u = lambda a: np.ascontiguousarray(a).view(np.uint16)  # noqa: E731
        ref = oracle.mamba_chunk_scan(u(arrs[0]), u(arrs[1]), arrs[2].astype(np.float32),
                                      arrs[3].astype(np.float32), u(arrs[4]),
                                      arrs[5].astype(np.float32), arrs[6].astype(np.float32),
                                      64, 64, 64)
    got = ov.view(torch.int16).cpu().numpy().view(np.uint16)
    assert_close(oracle.from_f16(got), oracle.from_f16(ref), **ATTN_TOL, what="mamba f16 memref")
