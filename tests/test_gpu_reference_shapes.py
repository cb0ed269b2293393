"""f16 parity at the reference's own example signatures.

Each test runs one function at the exact shapes and element type of its
stage-00 MLIR signature (examples/<k>/IR/00_from_helion_frontend.mlir, f16
memrefs throughout), with the reference's own emitted tile binding where the
Materialize pass produced an in-bounds one (split-K and mqa_decode; the other
examples' committed variants carry placeholder sizes beyond their extents,
materialize.cpp:56-65).  The whole output is compared with the CPU oracle in
f16 mode (oracle.element_type("f16")); bars as elsewhere: GEMMs 1e-2 +
1e-2 |ref|, attention / decode 2e-2 + 1e-2 |ref|, split-K partials and output
bit-exact on integer-valued inputs.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import from_f16, to_f16
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

GEMM_TOL = dict(atol=1e-2, rtol=1e-2)
ATTN_TOL = dict(atol=2e-2, rtol=1e-2)
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


@pytest.fixture(autouse=True)
def f16_oracle():
    with oracle.element_type("f16"):
        yield


@pytest.fixture(scope="module")
def emitted():
    with open(os.path.join(GOLDEN, "variant_names.json")) as f:
        return json.load(f)


def dev(h):
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).view(torch.float16).cuda()


def host(t):
    assert t.dtype == torch.float16
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rnd(rng, shape, scale=1.0):
    return to_f16(rng.standard_normal(shape).astype(np.float32) * scale)


def ints(rng, shape):
    return to_f16(rng.integers(-4, 5, shape).astype(np.float32))


def _announce(what):
    print(f"reference shape: {what}", flush=True)


def test_mm_reference_signature(lh):
    """@matmul (x: 2048x256, y: 256x256, out: 2048x256 f16), EX(mm,00):2."""
    _announce("matmul f16 2048x256 . 256x256")
    rng = np.random.default_rng(301)
    x, y = rnd(rng, (2048, 256)), rnd(rng, (256, 256))
    ref = oracle.matmul(x, y)
    for tm, tn in ((64, 64), (128, 128), (256, 256), (2048, 256)):
        out = lh.matmul(dev(x), dev(y), tile_m=tm, tile_n=tn, tile_k=256)
        assert_close(from_f16(host(out)), from_f16(ref), **GEMM_TOL,
                     what=f"mm f16 2048x256x256 tiles {tm}x{tn}")
    xi, yi = ints(rng, (2048, 256)), ints(rng, (256, 256))
    np.testing.assert_array_equal(host(lh.matmul(dev(xi), dev(yi))), oracle.matmul(xi, yi))


def test_bmm_reference_signature(lh):
    """@batch_matmul (8x4096x512 . 8x512x4096 -> 8x4096x4096 f16),
    EX(bmm_2Dmesh,00):4; every element against the oracle."""
    _announce("batch_matmul f16 8x4096x512 . 8x512x4096")
    rng = np.random.default_rng(302)
    a, b = rnd(rng, (8, 4096, 512)), rnd(rng, (8, 512, 4096))
    out = host(lh.batch_matmul(dev(a), dev(b), tile_m=256, tile_n=256, tile_k=512))
    ref = oracle.batch_matmul(a, b)
    assert_close(from_f16(out), from_f16(ref), **GEMM_TOL, what="bmm f16 8x4096x4096x512")


def test_split_k_reference_variant_dispatch_bit_exact(lh, emitted):
    """@split_k_matmul_gather (a: 512x4096, b: 4096x512 f16),
    EX(split_k_mm_gather,00):2, launched by the name the reference's own
    Materialize pass emitted (tile_k512 tile_m64 tile_n32,
    examples/split_k_mm_gather/IR/06_after_canonicalize.mlir:23) through
    loom_hip_dispatch_f16: on integer-valued inputs every one of the 8 fp32
    partial slabs and the f16 output equal the oracle's bit for bit."""
    names = [n for n in emitted["split_k_mm_gather"]["variants"]
             if n.endswith("__tile_k512__tile_m64__tile_n32")]
    assert len(names) == 20
    name = names[0]
    _announce(f"split_k f16 512x4096x512 via {name}")
    rng = np.random.default_rng(303)
    a, b = ints(rng, (512, 4096)), ints(rng, (4096, 512))
    out = torch.empty((512, 512), dtype=torch.float16, device="cuda")
    _, ws = lh.dispatch(name, dev(a), dev(b), out)
    ref, ref_partials = oracle.split_k_matmul_gather(a, b, 64, 32, 512)
    assert ref_partials.shape == (8, 512, 512)
    partials = ws[: 8 * 512 * 512 * 4].view(torch.float32).view(8, 512, 512).cpu().numpy()
    np.testing.assert_array_equal(partials, ref_partials)
    np.testing.assert_array_equal(host(out), ref)
    # every emitted mapping variant names the same binding: same bits
    for other in names[1:4]:
        out2 = torch.empty_like(out)
        lh.dispatch(other, dev(a), dev(b), out2)
        assert torch.equal(out2, out), other
    # float inputs at the same binding against the oracle's tolerance
    af, bf = rnd(rng, (512, 4096), 0.1), rnd(rng, (4096, 512), 0.1)
    outf = torch.empty((512, 512), dtype=torch.float16, device="cuda")
    lh.dispatch(name, dev(af), dev(bf), outf)
    reff, _ = oracle.split_k_matmul_gather(af, bf, 64, 32, 512)
    assert_close(from_f16(host(outf)), from_f16(reff), **GEMM_TOL, what="split-K f16 reference")


def test_flashattn_reference_signature_noncausal(lh):
    """@attention (k: 32x128x4096, v, q, out: 32x4096x128 f16), non-causal as
    the reference, EX(flashattn,00):4; the reference's scale constant
    0.08837890625 (:10); every element against the oracle."""
    _announce("attention f16 BH32 S4096 D128 non-causal")
    rng = np.random.default_rng(304)
    BH, S, D = 32, 4096, 128
    k, v, q = rnd(rng, (BH, D, S)), rnd(rng, (BH, S, D)), rnd(rng, (BH, S, D))
    scale = 0.08837890625
    out = lh.attention(dev(k), dev(v), dev(q), scale=scale, causal=False, tile_m=256)
    ref = oracle.attention(k, v, q, scale, False)
    assert_close(from_f16(host(out)), from_f16(ref), **ATTN_TOL, what="flashattn f16 reference")


def test_mqa_decode_reference_variant(lh, emitted):
    """@flash_decode (k: 16x128x8192, v: 16x8192x128, q, out: 16x32x128 f16),
    EX(mqa_decode,00):6, by the name the reference emitted (tile_b1 tile_n512
    tile_s512) through loom_hip_dispatch_f16; output and the 16 splits'
    partials against the oracle."""
    names = emitted["mqa_decode"]["variants"]
    assert all("__tile_b1__tile_n512__tile_s512" in n for n in names)
    name = names[0]
    _announce(f"flash_decode f16 B16 H32 D128 S8192 via {name}")
    rng = np.random.default_rng(305)
    B, H, D, S = 16, 32, 128, 8192
    k, v, q = rnd(rng, (B, D, S)), rnd(rng, (B, S, D)), rnd(rng, (B, H, D))
    scale = 0.08837890625
    out = torch.empty((B, H, D), dtype=torch.float16, device="cuda")
    _, ws = lh.dispatch(name, dev(k), dev(v), dev(q), out, scale=scale)
    ref, ref_lse, ref_o = oracle.flash_decode(k, v, q, scale, 1, 512, 512)
    assert_close(from_f16(host(out)), from_f16(ref), **ATTN_TOL, what="mqa f16 reference")
    ns = S // 512
    lse_bytes = (ns * B * H * 4 + 255) // 256 * 256
    lse = ws[: ns * B * H * 4].view(torch.float32).view(ns, B, H).cpu().numpy()
    o = ws[lse_bytes: lse_bytes + ns * B * H * D * 4].view(torch.float32).view(ns, B, H, D)
    assert_close(lse, ref_lse, atol=1e-2, rtol=1e-3, what="mqa f16 lse_s")
    assert_close(o.cpu().numpy(), ref_o, **ATTN_TOL, what="mqa f16 o_s")
    direct = lh.flash_decode(dev(k), dev(v), dev(q), scale=scale, tile_s=512, tile_n=512)
    assert torch.equal(direct, out)
