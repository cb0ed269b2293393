"""GPU parity of the f16 entry points (the reference's own element type)
against the CPU oracle in f16 mode (oracle.element_type("f16"): inputs widen
from IEEE binary16, outputs round to it; the conversions are pinned against
numpy in tests/test_oracle.py).  Bars as for bf16: GEMMs 1e-2 + 1e-2 |ref|,
attention / decode / chunk scan 2e-2 + 1e-2 |ref|, split-K partials and
integer-valued GEMMs bit-exact."""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_f16, to_f16
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

GEMM_TOL = dict(atol=1e-2, rtol=1e-2)
ATTN_TOL = dict(atol=2e-2, rtol=1e-2)


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


def dev(h):
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).view(torch.float16).cuda()


def devf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    assert t.dtype == torch.float16
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rnd(rng, shape, scale=1.0):
    return to_f16(rng.standard_normal(shape).astype(np.float32) * scale)


@pytest.mark.parametrize("tile", [64, 128, 256])
def test_matmul_f16(lh, tile):
    rng = np.random.default_rng(51)
    x, y = rnd(rng, (320, 256)), rnd(rng, (256, 192))
    # tile_n bounded by N = 192 (natural_ub): 192 runs as the 256 tile
    out = lh.matmul(dev(x), dev(y), tile_m=tile, tile_n=min(tile, 192))
    assert out.dtype == torch.float16
    ref = oracle.matmul(x, y, 64, 64, 64)
    assert_close(from_f16(host(out)), from_f16(ref), **GEMM_TOL, what=f"matmul f16 {tile}")
    xi = to_f16(rng.integers(-4, 5, (256, 512)).astype(np.float32))
    yi = to_f16(rng.integers(-4, 5, (512, 256)).astype(np.float32))
    np.testing.assert_array_equal(host(lh.matmul(dev(xi), dev(yi), tile_m=tile, tile_n=tile)),
                                  oracle.matmul(xi, yi, 64, 64, 64))


def test_batch_matmul_f16_persistent_bit_exact(lh):
    """The f16 form of the persistent 256x256 kernel (16 x 2048^2 x 128: 1024
    tiles, four per CU on a 256-CU part) on integer-valued inputs: every
    output element exact."""
    rng = np.random.default_rng(53)
    a = to_f16(rng.integers(-4, 5, (16, 2048, 128)).astype(np.float32))
    b = to_f16(rng.integers(-4, 5, (16, 128, 2048)).astype(np.float32))
    out = host(lh.batch_matmul(dev(a), dev(b), tile_m=256, tile_n=256))
    with oracle.element_type("f16"):
        for z in (0, 7, 15):
            np.testing.assert_array_equal(out[z], oracle.matmul(a[z], b[z]), err_msg=str(z))


def test_batch_matmul_f16(lh):
    rng = np.random.default_rng(52)
    a, b = rnd(rng, (2, 256, 128)), rnd(rng, (2, 128, 512))
    out = host(lh.batch_matmul(dev(a), dev(b), tile_m=256, tile_n=256))
    ref = oracle.batch_matmul(a, b, 1, 64, 64, 64)
    assert_close(from_f16(out), from_f16(ref), **GEMM_TOL, what="bmm f16")


def test_split_k_f16_bit_exact(lh):
    rng = np.random.default_rng(53)
    a = to_f16(rng.integers(-4, 5, (96, 2048)).astype(np.float32))
    b = to_f16(rng.integers(-4, 5, (2048, 128)).astype(np.float32))
    out, parts = lh.split_k_matmul_gather(dev(a), dev(b), tile_m=64, tile_n=64, tile_k=512)
    o_ref, p_ref = oracle.split_k_matmul_gather(a, b, 32, 32, 512)
    np.testing.assert_array_equal(parts.cpu().numpy(), p_ref)
    np.testing.assert_array_equal(host(out), o_ref)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("tile_m", [64, 256])
def test_attention_f16(lh, causal, tile_m):
    rng = np.random.default_rng(54)
    BH, S, D = 3, 328, 128
    k, v, q = rnd(rng, (BH, D, S)), rnd(rng, (BH, S, D)), rnd(rng, (BH, S, D))
    out = host(lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=tile_m, tile_n=64))
    ref = oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64)
    assert_close(from_f16(out), from_f16(ref), **ATTN_TOL, what=f"attention f16 {causal} {tile_m}")


def test_flash_decode_f16(lh):
    rng = np.random.default_rng(55)
    B, H, D, S = 3, 32, 128, 1000
    k, v, q = rnd(rng, (B, D, S)), rnd(rng, (B, S, D)), rnd(rng, (B, H, D))
    out, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=256, tile_n=128,
                                  return_partials=True)
    ref, lse_r, o_r = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 256, 64)
    assert_close(from_f16(host(out)), from_f16(ref), **ATTN_TOL, what="decode f16")
    assert_close(lse.cpu().numpy(), lse_r, atol=1e-3, rtol=1e-4, what="decode f16 lse")


@pytest.mark.parametrize("S,ts", [(1024, 44), (2048, 256)])
def test_flash_decode_f16_d64_dma(lh, S, ts):
    """f16 at D = 64 with S a multiple of 8: the LDS-DMA split kernel's f16
    D = 64 instantiation, including splits that start off an 8-key boundary
    (tile_s 44); output, lse_s and o_s against the oracle."""
    rng = np.random.default_rng(S + ts)
    B, H, D = 2, 12, 64
    k, v, q = rnd(rng, (B, D, S)), rnd(rng, (B, S, D)), rnd(rng, (B, H, D))
    out, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=ts,
                                  return_partials=True)
    ref, lse_r, o_r = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, ts, ts)
    assert_close(from_f16(host(out)), from_f16(ref), **ATTN_TOL, what=f"decode f16 D64 S{S} ts{ts}")
    assert_close(lse.cpu().numpy(), lse_r, atol=1e-2, rtol=1e-3, what=f"decode f16 D64 lse ts{ts}")
    assert_close(o.cpu().numpy(), o_r, **ATTN_TOL, what=f"decode f16 D64 o_s ts{ts}")


@pytest.mark.parametrize("causal", [False, True])
def test_attention_f16_d64(lh, causal):
    """f16 attention at head_dim 64 (the D = 64 instantiations in f16)."""
    rng = np.random.default_rng(58 + causal)
    BH, S, D = 2, 456, 64
    k, v, q = rnd(rng, (BH, D, S)), rnd(rng, (BH, S, D)), rnd(rng, (BH, S, D))
    for tile_m in (64, 128, 192, 256):
        out = host(lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=tile_m))
        ref = oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64)
        assert_close(from_f16(out), from_f16(ref), **ATTN_TOL,
                     what=f"attention f16 D64 causal={causal} tile_m={tile_m}")


def _ssd_inputs(rng, b, H, G, L, P, N):
    x = rnd(rng, (b, H, L, P))
    Bm, C = rnd(rng, (b, G, L, N)), rnd(rng, (b, G, L, N))
    dt = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
    A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
    return x, dt, A, Bm, C


def test_ssd_prologue_f16_wide_units(lh):
    """P = 64, N = 128, Q = 256 in f16: the state kernel's 256-key form."""
    rng = np.random.default_rng(57)
    b, H, G, Q, nc, P, N = 1, 4, 1, 256, 3, 64, 128
    x, dt, A, Bm, C = _ssd_inputs(rng, b, H, G, nc * Q, P, N)
    _, dA, cb, prev = lh.ssd_prologue(dev(x), devf(dt), devf(A), dev(Bm), dev(C), Q)
    assert cb.dtype == torch.float16
    _, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, Q)
    cbg, cbr = from_f16(host(cb)), from_f16(cb_o)
    assert np.all(np.abs(cbg - cbr) <= 2.0 ** -10 * np.abs(cbr) + 1e-5), "cb f16"
    pg = prev.cpu().numpy()
    scale = 1e-2 * float(np.abs(prev_o).max())
    assert np.all(np.abs(pg - prev_o) <= 1e-3 * (np.abs(prev_o) + scale)), "prev_states f16"


def test_ssd_prologue_and_chunk_scan_f16(lh):
    """The whole Mamba-2 chain in f16 (the reference example's geometry)."""
    rng = np.random.default_rng(56)
    b, H, G, Q, nc, P, N = 1, 32, 4, 192, 2, 160, 128
    x, dt, A, Bm, C = _ssd_inputs(rng, b, H, G, nc * Q, P, N)
    Dh = rng.standard_normal(H).astype(np.float32)
    dt4, dA, cb, prev = lh.ssd_prologue(dev(x), devf(dt), devf(A), dev(Bm), dev(C), Q)
    assert cb.dtype == torch.float16
    _, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, Q)
    cbg, cbr = from_f16(host(cb)), from_f16(cb_o)
    assert np.all(np.abs(cbg - cbr) <= 2.0 ** -10 * np.abs(cbr) + 1e-5), "cb f16"
    pg = prev.cpu().numpy()
    scale = 1e-2 * float(np.abs(prev_o).max())
    assert np.all(np.abs(pg - prev_o) <= 1e-3 * (np.abs(prev_o) + scale)), "prev_states f16"
    # the chunk scan's f16 signature is the reference's own: every tensor f16,
    # dt, dA_cumsum, D and prev_states_T included
    # (examples/mamba_chunk_scan/IR/00_from_helion_frontend.mlir:4)
    h16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    dt_h, dA_h, D_h, prev_h = h16(dt.reshape(b, H, nc, Q)), h16(dA_o), h16(Dh), h16(prev_o)
    f16 = lambda a: torch.from_numpy(a).to(torch.float16).cuda()  # noqa: E731
    out = lh.helion_mamba2_chunk_scan_kernel(dev(cb_o), dev(x), f16(dt_h), f16(dA_h), dev(C),
                                             f16(D_h), f16(prev_h), tile_m=192, tile_n=64)
    assert out.dtype == torch.float16
    with oracle.element_type("f16"):
        ref = oracle.mamba_chunk_scan(cb_o, x, dt_h, dA_h, C, D_h, prev_h, 64, 64, 64)
    assert_close(from_f16(host(out)), from_f16(ref), **ATTN_TOL, what="chunk scan f16")
    # the fp32 side tensors are refused by the f16 signature before any launch
    with pytest.raises(TypeError):
        lh.helion_mamba2_chunk_scan_kernel(cb, dev(x), dt4.contiguous(), dA, dev(C), devf(Dh),
                                           prev, tile_m=192, tile_n=64)


def test_dispatch_f16(lh):
    rng = np.random.default_rng(57)
    x, y = rnd(rng, (256, 128)), rnd(rng, (128, 256))
    out = torch.empty((256, 256), dtype=torch.float16, device="cuda")
    lh.dispatch("matmul__tile_k64__tile_m128__tile_n128", dev(x), dev(y), out)
    assert torch.equal(out, lh.matmul(dev(x), dev(y), tile_m=128, tile_n=128))
    assert_close(from_f16(host(out)), from_f16(oracle.matmul(x, y, 64, 64, 64)), **GEMM_TOL,
                 what="dispatch f16")
