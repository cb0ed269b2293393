"""GPU parity: every HIP kernel against the CPU oracle and the golden fixtures.

Bars (from the task's tolerance statement):
  bf16 GEMMs            |gpu - ref| <= 1e-2 + 1e-2 |ref|
  attention / decode /
  chunk scan            |gpu - ref| <= 2e-2 + 1e-2 |ref|
  split-K partials      bit-exact on integer-valued inputs (and the output)
The oracle (oracle/oracle.c, fp32) is pinned against the fixtures by
tests/test_oracle.py; here it is the checker only.  Full BASELINE sizes are
checked against the oracle on full outputs where the oracle finishes in
seconds; where it does not (bmm, attention), the oracle checks exact
row/head subsets and a plain fp32 torch computation on the GPU checks every
element (both are floating-point kernels).  Each BASELINE-size test also
runs its kernel a second time on the same inputs and requires the same bits.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16, to_bf16
from tests.conftest import ATTN_TILES, GEMM_TILES, MAMBA_M_TILES, assert_close, tile_for

pytestmark = pytest.mark.gpu

GEMM_TOL = dict(atol=1e-2, rtol=1e-2)
ATTN_TOL = dict(atol=2e-2, rtol=1e-2)


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def dev(a_u16):
    """numpy bf16 bits -> torch bf16 on cuda:0."""
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).view(torch.bfloat16).cuda()


def devf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    """torch bf16 -> numpy bf16 bits."""
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rng_bf16(rng, shape, kind="normal", scale=1.0):
    if kind == "normal":
        return to_bf16(rng.standard_normal(shape, dtype=np.float32) * scale)
    return to_bf16(rng.uniform(-scale, scale, shape).astype(np.float32))


# ------------------------------------------------------------------- matmul

def gemm_bindings(M, N):
    """(T, tile_m, tile_n) for every square workgroup tile T a binding can
    name on an M x N output (tiles within their extents)."""
    out = []
    for T in GEMM_TILES:
        tm, tn = tile_for(T, M, GEMM_TILES), tile_for(T, N, GEMM_TILES)
        if tm is not None and tn is not None:
            out.append((T, tm, tn))
    assert out, (M, N)
    return out


@pytest.mark.parametrize("name", ["mm_tiles", "mm_ragged"])
def test_matmul_golden(lh, golden, name):
    g = golden(name)
    M, N = g["expected"].shape
    for T, tm, tn in gemm_bindings(M, N):
        out = host(lh.matmul(dev(g["x"]), dev(g["y"]), tile_m=tm, tile_n=tn, tile_k=32))
        assert_close(from_bf16(out), g["expected"], **GEMM_TOL, what=f"{name} T{T}")


def test_matmul_whole_extent_tiles(lh):
    """Tiles equal to short extents (below the smallest built tile) run as one
    covering tile: 48 x 40 output with tile_m = 48, tile_n = 40, tile_k = K."""
    rng = np.random.default_rng(14)
    x = to_bf16(rng.integers(-8, 9, (48, 24)).astype(np.float32))
    y = to_bf16(rng.integers(-8, 9, (24, 40)).astype(np.float32))
    got = host(lh.matmul(dev(x), dev(y), tile_m=48, tile_n=40, tile_k=24))
    assert np.array_equal(got, oracle.matmul(x, y))


def test_matmul_integer_bit_exact(lh):
    rng = np.random.default_rng(11)
    x = to_bf16(rng.integers(-8, 9, (200, 328)).astype(np.float32))
    y = to_bf16(rng.integers(-8, 9, (328, 136)).astype(np.float32))
    ref = oracle.matmul(x, y)
    assert len(gemm_bindings(200, 136)) == 3
    for T, tm, tn in gemm_bindings(200, 136):
        assert np.array_equal(host(lh.matmul(dev(x), dev(y), tile_m=tm, tile_n=tn)), ref), T


def test_matmul_pipelined_edge_tiles_bit_exact(lh):
    """K a multiple of the pipelined kernels' rounds (128 / 256 / 512), M and N not a
    multiple of the tile: clamped DMA rows/columns and the guarded epilogue."""
    rng = np.random.default_rng(12)
    for (M, N, K) in [(300, 264, 512), (520, 136, 768), (257, 520, 1024)]:
        x = to_bf16(rng.integers(-8, 9, (M, K)).astype(np.float32))
        y = to_bf16(rng.integers(-8, 9, (K, N)).astype(np.float32))
        ref = oracle.matmul(x, y)
        assert len(gemm_bindings(M, N)) == 3
        for T, tm, tn in gemm_bindings(M, N):
            got = host(lh.matmul(dev(x), dev(y), tile_m=tm, tile_n=tn))
            assert np.array_equal(got, ref), (M, N, K, T)


def test_matmul_tile64_whole_tiles_bit_exact(lh):
    """64x64 tiles on whole-tile shapes (the pipelined 64-tile kernel with its
    16-stage ring): integer-valued inputs, every element exact; also batched."""
    rng = np.random.default_rng(13)
    for (M, N, K) in [(1024, 1024, 1024), (512, 192, 2048), (64, 64, 512)]:
        x = to_bf16(rng.integers(-8, 9, (M, K)).astype(np.float32))
        y = to_bf16(rng.integers(-8, 9, (K, N)).astype(np.float32))
        got = host(lh.matmul(dev(x), dev(y), tile_m=64, tile_n=64))
        assert np.array_equal(got, oracle.matmul(x, y)), (M, N, K)
    a0 = to_bf16(rng.integers(-8, 9, (3, 256, 512)).astype(np.float32))
    a1 = to_bf16(rng.integers(-8, 9, (3, 512, 128)).astype(np.float32))
    out = host(lh.batch_matmul(dev(a0), dev(a1), tile_m=64, tile_n=64))
    for b in range(3):
        assert np.array_equal(out[b], oracle.matmul(a0[b], a1[b])), b


def test_matmul_baseline_1024(lh):
    rng = np.random.default_rng(1)
    x = rng_bf16(rng, (1024, 1024), "uniform")
    y = rng_bf16(rng, (1024, 1024), "uniform")
    ref = from_bf16(oracle.matmul(x, y, 128, 128, 64))
    for t in [(64, 64), (128, 128)]:
        out = lh.matmul(dev(x), dev(y), tile_m=t[0], tile_n=t[1])
        assert_close(from_bf16(host(out)), ref, **GEMM_TOL, what=f"mm 1024^3 {t}")
        again = lh.matmul(dev(x), dev(y), tile_m=t[0], tile_n=t[1])
        assert torch.equal(out.view(torch.int16), again.view(torch.int16)), t


# ------------------------------------------------------------- batch_matmul

def test_batch_matmul_golden(lh, golden):
    g = golden("bmm_small")
    _, M, N = g["expected"].shape
    for T, tm, tn in gemm_bindings(M, N):
        out = host(lh.batch_matmul(dev(g["arg0"]), dev(g["arg1"]), tile_m=tm, tile_n=tn))
        assert_close(from_bf16(out), g["expected"], **GEMM_TOL, what=f"bmm golden T{T}")


def test_batch_matmul_baseline(lh):
    """B16 x 2048^3 (the bench config): every element of every batch against
    the oracle, and a second run bit-identical to the first."""
    torch.manual_seed(0)
    a0 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
    a1 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
    dout = lh.batch_matmul(a0, a1, tile_m=256, tile_n=256)
    out = host(dout)
    ref = oracle.batch_matmul(host(a0), host(a1), 1, 256, 256, 64)
    assert_close(from_bf16(out), from_bf16(ref), **GEMM_TOL, what="bmm B16 2048^3 vs oracle")
    again = lh.batch_matmul(a0, a1, tile_m=256, tile_n=256)
    assert torch.equal(dout.view(torch.int16), again.view(torch.int16))


def test_batch_matmul_persistent_bit_exact(lh):
    """Shapes whose 256x256 tiles divide evenly over the CUs, two or more per CU (the
    persistent kernel on a 256-CU part): integer-valued inputs, every output element
    exact.  K 128 gives one DMA round per tile (the next tile's loads start in the
    tile's first round); K 512 four."""
    rng = np.random.default_rng(21)
    for (B, M, N, K) in [(16, 2048, 2048, 128), (8, 2048, 2048, 512), (4, 4096, 2048, 256)]:
        a0 = to_bf16(rng.integers(-4, 5, (B, M, K)).astype(np.float32))
        a1 = to_bf16(rng.integers(-4, 5, (B, K, N)).astype(np.float32))
        out = host(lh.batch_matmul(dev(a0), dev(a1), tile_m=256, tile_n=256))
        for b in range(B):
            assert np.array_equal(out[b], oracle.matmul(a0[b], a1[b])), (B, M, N, K, b)


def test_matmul_persistent_bit_exact(lh):
    """matmul 8192 x 4096 x 256 (512 tiles of 256x256): sampled rows exact."""
    rng = np.random.default_rng(22)
    x = to_bf16(rng.integers(-4, 5, (8192, 256)).astype(np.float32))
    y = to_bf16(rng.integers(-4, 5, (256, 4096)).astype(np.float32))
    out = host(lh.matmul(dev(x), dev(y), tile_m=256, tile_n=256))
    rows = np.sort(np.random.default_rng(6).choice(8192, 512, replace=False))
    assert np.array_equal(out[rows], oracle.matmul(np.ascontiguousarray(x[rows]), y))


# ------------------------------------------------------------------ split-K

def test_split_k_integer_partials_bit_exact(lh, golden):
    g = golden("splitk_int")
    out, parts = lh.split_k_matmul_gather(dev(g["a"]), dev(g["b"]), tile_m=64, tile_n=64,
                                          tile_k=int(g["tile_k"]))
    assert np.array_equal(parts.cpu().numpy().astype(np.float64), g["expected_partials"])
    assert np.array_equal(host(out), to_bf16(g["expected"].astype(np.float32)))


def test_split_k_float(lh, golden):
    g = golden("splitk_float")
    o_ref, p_ref = oracle.split_k_matmul_gather(g["a"], g["b"], 16, 32, int(g["tile_k"]))
    M, N = g["expected"].shape
    out, parts = lh.split_k_matmul_gather(dev(g["a"]), dev(g["b"]), tile_m=tile_for(64, M, GEMM_TILES),
                                          tile_n=tile_for(64, N, GEMM_TILES), tile_k=int(g["tile_k"]))
    assert_close(parts.cpu().numpy(), p_ref, atol=1e-4, rtol=1e-4, what="partials")
    assert_close(from_bf16(host(out)), g["expected"], **GEMM_TOL, what="split-K out")


def test_split_k_ragged_slab(lh, golden):
    """tile_k = 500 does not divide K = 768 and is not a multiple of 8."""
    g = golden("splitk_float")
    o_ref, p_ref = oracle.split_k_matmul_gather(g["a"], g["b"], 16, 32, 500)
    M, N = g["expected"].shape
    out, parts = lh.split_k_matmul_gather(dev(g["a"]), dev(g["b"]), tile_m=tile_for(64, M, GEMM_TILES),
                                          tile_n=tile_for(64, N, GEMM_TILES), tile_k=500)
    assert parts.shape[0] == 2
    assert_close(parts.cpu().numpy(), p_ref, atol=1e-4, rtol=1e-4, what="ragged partials")
    assert_close(from_bf16(host(out)), from_bf16(o_ref), **GEMM_TOL, what="ragged out")


def test_split_k_baseline_integer_bit_exact(lh):
    """512 x 512 x 16384, 16 slabs: partials and output bit-exact (integer inputs)."""
    rng = np.random.default_rng(7)
    ai = rng.integers(-4, 5, (512, 16384)).astype(np.float64)
    bi = rng.integers(-4, 5, (16384, 512)).astype(np.float64)
    out, parts = lh.split_k_matmul_gather(dev(to_bf16(ai.astype(np.float32))),
                                          dev(to_bf16(bi.astype(np.float32))),
                                          tile_m=64, tile_n=64, tile_k=1024)
    parts = parts.cpu().numpy()
    exp = np.stack([ai[:, s * 1024:(s + 1) * 1024] @ bi[s * 1024:(s + 1) * 1024] for s in range(16)])
    assert np.array_equal(parts.astype(np.float64), exp)
    assert np.array_equal(host(out), to_bf16(exp.sum(0).astype(np.float32)))


def test_split_k_pipelined_integer_bit_exact(lh):
    """Slabs that are whole rounds of the pipelined 128 and 256 tiles, with an
    edge tile in M: every fp32 partial and the output bit-exact."""
    rng = np.random.default_rng(9)
    ai = rng.integers(-4, 5, (384, 4096)).astype(np.float64)
    bi = rng.integers(-4, 5, (4096, 256)).astype(np.float64)
    exp = np.stack([ai[:, s * 1024:(s + 1) * 1024] @ bi[s * 1024:(s + 1) * 1024] for s in range(4)])
    for t in [(64, 64), (128, 128), (256, 256)]:
        out, parts = lh.split_k_matmul_gather(dev(to_bf16(ai.astype(np.float32))),
                                              dev(to_bf16(bi.astype(np.float32))),
                                              tile_m=t[0], tile_n=t[1], tile_k=1024)
        assert np.array_equal(parts.cpu().numpy().astype(np.float64), exp), t
        assert np.array_equal(host(out), to_bf16(exp.sum(0).astype(np.float32))), t


def test_split_k_baseline_float(lh):
    rng = np.random.default_rng(8)
    a = rng_bf16(rng, (512, 16384), scale=0.02)
    b = rng_bf16(rng, (16384, 512), scale=0.02)
    o_ref, p_ref = oracle.split_k_matmul_gather(a, b, 64, 64, 1024)
    for t in [(64, 64), (128, 128)]:
        out, parts = lh.split_k_matmul_gather(dev(a), dev(b), tile_m=t[0], tile_n=t[1],
                                              tile_k=1024)
        assert_close(parts.cpu().numpy(), p_ref, atol=1e-5, rtol=1e-4, what=f"partials {t}")
        assert_close(from_bf16(host(out)), from_bf16(o_ref), **GEMM_TOL, what=f"out {t}")
        out2, parts2 = lh.split_k_matmul_gather(dev(a), dev(b), tile_m=t[0], tile_n=t[1],
                                                tile_k=1024)
        assert torch.equal(parts2, parts) and torch.equal(out2.view(torch.int16),
                                                          out.view(torch.int16)), t


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("name", ["attention_noncausal", "attention_causal"])
def test_attention_golden(lh, golden, name):
    g = golden(name)
    Sq = g["q"].shape[1]
    ran = 0
    for T in ATTN_TILES:   # every query tile a binding can name for this Sq
        tm = tile_for(T, Sq, ATTN_TILES)
        if tm is None:
            continue
        out = lh.attention(dev(g["k"]), dev(g["v"]), dev(g["q"]), scale=float(g["scale"]),
                           causal=bool(g["causal"]), tile_m=tm, tile_n=32)
        assert_close(from_bf16(host(out)), g["expected"], **ATTN_TOL, what=f"{name} T{T}")
        ran += 1
    assert ran == 2


@pytest.mark.parametrize("causal", [False, True])
def test_attention_closed_forms(lh, causal):
    rng = np.random.default_rng(3)
    BH, S, D = 2, 200, 128
    k = rng_bf16(rng, (BH, D, S))
    q = rng_bf16(rng, (BH, S, D))
    row = rng_bf16(rng, (D,))
    v_same = np.ascontiguousarray(np.broadcast_to(row, (BH, S, D)))
    out = host(lh.attention(dev(k), dev(v_same), dev(q), scale=0.2, causal=causal))
    assert_close(from_bf16(out), np.broadcast_to(from_bf16(row), out.shape), atol=1e-2, rtol=1e-2,
                 what="identical V rows")
    v = rng_bf16(rng, (BH, S, D))
    zeros = np.zeros((BH, S, D), np.uint16)
    vf = from_bf16(v).astype(np.float64)
    out = from_bf16(host(lh.attention(dev(k), dev(v), dev(zeros), scale=0.2, causal=causal)))
    exp = (np.cumsum(vf, 1) / np.arange(1, S + 1)[None, :, None]) if causal else \
        np.broadcast_to(vf.mean(1, keepdims=True), vf.shape)
    assert_close(out, exp, **ATTN_TOL, what="Q=0")


def test_attention_vs_oracle_mid(lh):
    rng = np.random.default_rng(4)
    BH, S, D = 3, 1000, 128
    k, v, q = rng_bf16(rng, (BH, D, S)), rng_bf16(rng, (BH, S, D)), rng_bf16(rng, (BH, S, D))
    for causal in (False, True):
        ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
        for tm in (64, 192, 256):
            got = from_bf16(host(lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=tm)))
            assert_close(got, ref, **ATTN_TOL, what=f"attention S=1000 causal={causal} tile_m={tm}")


def test_attention_baseline_heads(lh):
    """B4 x H32, S 4096, D 128, causal (the bench config) with query tiles of
    192 and 256: every element of all 128 heads against the oracle, and a
    second run bit-identical to the first."""
    torch.manual_seed(1)
    BH, S, D = 128, 4096, 128
    k = torch.randn(BH, D, S, device="cuda").to(torch.bfloat16)
    v = torch.randn(BH, S, D, device="cuda").to(torch.bfloat16)
    q = torch.randn(BH, S, D, device="cuda").to(torch.bfloat16)
    ref = from_bf16(oracle.attention(host(k), host(v), host(q), 1 / math.sqrt(D), True, 1, 128, 64))
    for tile_m in (192, 256):
        dout = lh.attention(k, v, q, causal=True, tile_m=tile_m, tile_n=64)
        assert_close(from_bf16(host(dout)), ref, **ATTN_TOL,
                     what=f"flashattn B4 H32 S4096 causal tile_m {tile_m} vs oracle")
        again = lh.attention(k, v, q, causal=True, tile_m=tile_m, tile_n=64)
        assert torch.equal(dout.view(torch.int16), again.view(torch.int16))


@pytest.mark.parametrize("causal,BH,Sq,Skv,D", [(True, 48, 2816, 2816, 128),
                                                  (False, 132, 1024, 1000, 64)])
def test_attention_tile256_many_items(lh, causal, BH, Sq, Skv, D):
    """tile_m 256 with 528 (b, h, query tile) workgroups, two rounds and a partial
    third on a 256-CU part: causal items of 4..44 KV blocks, or ragged Skv with
    masked edge blocks.  Three heads vs the oracle."""
    rng = np.random.default_rng(31)
    k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
    out = host(lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=256, tile_n=64))
    assert np.isfinite(from_bf16(out)).all()
    for h in (0, BH // 2 - 1, BH - 1):
        ref = oracle.attention(k[h:h + 1], v[h:h + 1], q[h:h + 1], 1 / math.sqrt(D), causal, 1,
                               128, 64)
        assert_close(from_bf16(out[h:h + 1]), from_bf16(ref), **ATTN_TOL, what=f"head {h}")


# ------------------------------------------------------------- flash_decode

@pytest.mark.parametrize("name,tile_s", [("decode_ragged", 64), ("decode_ragged", 200),
                                         ("decode_mqa", 128), ("decode_mqa", 512)])
def test_decode_golden(lh, golden, name, tile_s):
    g = golden(name)
    out = lh.flash_decode(dev(g["k"]), dev(g["v"]), dev(g["q"]), scale=float(g["scale"]),
                          tile_s=tile_s, tile_n=min(tile_s, 64))
    assert_close(from_bf16(host(out)), g["expected"], **ATTN_TOL, what=f"{name} {tile_s}")


def test_decode_partials_match_oracle(lh, golden):
    g = golden("decode_ragged")
    scale = float(g["scale"])
    _, lse_ref, o_ref = oracle.flash_decode(g["k"], g["v"], g["q"], scale, 1, 64, 32)
    _, lse, o = lh.flash_decode(dev(g["k"]), dev(g["v"]), dev(g["q"]), scale=scale, tile_s=64,
                                tile_n=32, return_partials=True)
    assert lse.shape == lse_ref.shape and o.shape == o_ref.shape
    assert_close(lse.cpu().numpy(), lse_ref, atol=1e-2, rtol=1e-3, what="lse_s")
    assert_close(o.cpu().numpy(), o_ref, **ATTN_TOL, what="o_s")


@pytest.mark.parametrize("H,D,S,ts", [(40, 128, 2048, 512), (64, 64, 1024, 100),
                                      (96, 128, 1001, 256), (33, 64, 1004, 128)])
def test_decode_more_than_32_heads(lh, H, D, S, ts):
    """More query heads than one workgroup's 32 slots: head groups of 32 on
    the third grid axis, each streaming the split's K and V (LDS-DMA kernel
    for S a multiple of 8, register kernel otherwise); output and both
    gathered partials against the oracle."""
    print(f"decode H{H} D{D} S{S} tile_s{ts}", flush=True)
    rng = np.random.default_rng(H * 7 + S)
    B = 2
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    ref, lse_r, o_r = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, ts, 64)
    got, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=64,
                                  return_partials=True)
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"decode H{H} S{S}")
    assert_close(lse.cpu().numpy(), lse_r, atol=1e-2, rtol=1e-3, what=f"decode H{H} lse_s")
    assert_close(o.cpu().numpy(), o_r, **ATTN_TOL, what=f"decode H{H} o_s")


@pytest.mark.parametrize("S,ts", [(1001, 256), (1004, 128)])
def test_decode_register_path(lh, S, ts):
    """S not a multiple of 8: K rows do not start on 16-byte boundaries, so the
    register-load split kernel runs (2-byte K loads for S % 4 != 0, 8-byte
    for S % 4 == 0) instead of the LDS-DMA one."""
    rng = np.random.default_rng(S)
    B, H, D = 2, 32, 128
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    ref, lse_r, o_r = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, ts, 64)
    got, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=64,
                                  return_partials=True)
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"decode S={S}")
    assert_close(lse.cpu().numpy(), lse_r, atol=1e-2, rtol=1e-3, what=f"lse S={S}")


@pytest.mark.parametrize("D,H,ts", [(128, 32, 100), (64, 12, 44), (128, 5, 8)])
def test_decode_split_boundaries(lh, D, H, ts):
    """LDS-DMA split kernel with splits that start off 8-key boundaries
    (stages start at the split's first key rounded down, the keys before it
    masked), splits shorter than a 32-key half (waves that see no key), and
    fewer than 16 heads; every split's partials against the oracle."""
    rng = np.random.default_rng(D + H + ts)
    B, S = 3, 1024
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    ref, lse_r, o_r = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, ts, min(ts, 64))
    got, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=min(ts, 64),
                                  return_partials=True)
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"decode ts={ts}")
    assert_close(lse.cpu().numpy(), lse_r, atol=1e-2, rtol=1e-3, what=f"lse ts={ts}")
    assert_close(o.cpu().numpy(), o_r, **ATTN_TOL, what=f"o_s ts={ts}")


def test_decode_baseline(lh):
    """B32, H32 on one KV head, D128, S8192 (the bench config) vs the oracle."""
    rng = np.random.default_rng(9)
    B, H, D, S = 32, 32, 128, 8192
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    ref, _, _ = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 512, 128)
    for ts in (512, 1024):
        got = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=128)
        assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"decode tile_s={ts}")
        # run to run: the same inputs give the same bits
        again = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=ts, tile_n=128)
        assert torch.equal(got.view(torch.int16), again.view(torch.int16)), ts


def test_decode_workspace_reuse_and_garbage(lh):
    """A workspace full of garbage, then the same workspace reused for
    different inputs, gives each call's own result; and 128 splits (the
    combine loads the splits in chunks of 16 and rescales its running sum
    from one chunk to the next, so this case crosses eight chunk
    boundaries)."""
    rng = np.random.default_rng(21)
    B, H, D, S = 3, 32, 128, 2048
    ts = 256
    ws = lh.flash_decode_workspace(B, H, D, S, ts, "cuda")
    ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device="cuda"))
    for trial in range(3):
        k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
        ref, _, _ = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, ts, 128)
        got = lh.flash_decode(dev(k), dev(v), dev(q), workspace=ws, tile_s=ts, tile_n=128)
        assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"reuse {trial}")
    # ns = 2048 / 16 = 128 splits: eight 16-split chunks of the combine
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    ref, _, _ = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 16, 16)
    got = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=16, tile_n=16)
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what="128 splits")


# -------------------------------------------------------------------- mamba

def _mamba_gpu(lh, cb, x, dt, dA, C, Dh, prev, **tiles):
    return host(lh.helion_mamba2_chunk_scan_kernel(dev(cb), dev(x), devf(dt), devf(dA), dev(C),
                                                   devf(Dh), devf(prev), **tiles))


def test_mamba_chain_matches_recurrence(lh, golden):
    g = golden("mamba_small")
    Q = int(g["chunk_size"])
    dt, dA, cb, prev = oracle.mamba_prologue(g["x"], g["dt"], g["A"], g["B"], g["C"], Q)
    out = _mamba_gpu(lh, cb, g["x"], dt, dA, g["C"], g["D"], prev,
                     tile_m=tile_for(64, Q, MAMBA_M_TILES), tile_n=16, tile_k=Q)
    assert_close(from_bf16(out), g["expected"], atol=3e-2, rtol=1e-2, what="mamba vs recurrence")
    ref = oracle.mamba_chunk_scan(cb, g["x"], dt, dA, g["C"], g["D"], prev, 16, 16, 16)
    assert_close(from_bf16(out), from_bf16(ref), **ATTN_TOL, what="mamba vs oracle")


def _mamba_inputs(rng, b, nc, H, G, Q, P, N):
    L = nc * Q
    x = rng_bf16(rng, (b, H, L, P))
    Bm = rng_bf16(rng, (b, G, L, N))
    C = rng_bf16(rng, (b, G, L, N))
    dt_raw = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
    A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
    Dh = rng.standard_normal(H).astype(np.float32)
    dt, dA, cb, prev = oracle.mamba_prologue(x, dt_raw, A, Bm, C, Q)
    return cb, x, dt, dA, C, Dh, prev


@pytest.mark.parametrize("tiles", [(256, 64), (128, 32), (64, 16)])
def test_mamba_baseline_chunk_shape(lh, tiles):
    """BASELINE per-chunk shape (Q256, P64, N128, G1) on b1 x 4 chunks x 4 heads."""
    rng = np.random.default_rng(21)
    cb, x, dt, dA, C, Dh, prev = _mamba_inputs(rng, 1, 4, 4, 1, 256, 64, 128)
    ref = oracle.mamba_chunk_scan(cb, x, dt, dA, C, Dh, prev, 64, 64, 64)
    out = _mamba_gpu(lh, cb, x, dt, dA, C, Dh, prev, tile_m=tiles[0], tile_n=tiles[1])
    assert_close(from_bf16(out), from_bf16(ref), **ATTN_TOL, what=f"mamba {tiles}")


def test_mamba_reference_shape_groups(lh):
    """The reference example's own geometry: Q192, P160, N128, 4 groups (h/8)."""
    rng = np.random.default_rng(22)
    cb, x, dt, dA, C, Dh, prev = _mamba_inputs(rng, 1, 2, 32, 4, 192, 160, 128)
    ref = oracle.mamba_chunk_scan(cb, x, dt, dA, C, Dh, prev, 64, 64, 64)
    out = _mamba_gpu(lh, cb, x, dt, dA, C, Dh, prev, tile_m=192, tile_n=64)
    assert_close(from_bf16(out), from_bf16(ref), **ATTN_TOL, what="mamba ref shape")
