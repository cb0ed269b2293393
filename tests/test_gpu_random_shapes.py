"""GPU parity on seeded random shapes: each entry point at extents drawn from
a fixed-seed generator (ragged, tiny, non-power-of-two, both 16-bit
layouts' usual edge cases), with the library's preferred tiles and with a
random legal binding, against the CPU oracle.

Integer-valued GEMM inputs make matmul, batch_matmul and split-K exact (the
oracle's fp32 sums are exact below 2^24), so those compare bit for bit;
attention, decode and the Mamba-2 path use the floating-point bars of
tests/test_gpu_parity.py.  Every attention draw must launch; elsewhere a shape
the library does not build (LOOM_HIP_EUNSUP) must be refused with that code
before anything launches, and no other error is accepted.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16, to_bf16
from tests.conftest import GEMM_TILES, MAMBA_M_TILES, assert_close, tile_for
from tests.test_gpu_parity import ATTN_TOL, dev, devf, host, rng_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _ints(rng, shape, lo=-4, hi=4):
    return to_bf16(rng.integers(lo, hi + 1, shape).astype(np.float32))


def _random_gemm_tiles(rng, M, N):
    """A legal (tile_m, tile_n) on an M x N output, or None for the default."""
    T = int(rng.choice(GEMM_TILES))
    tm, tn = tile_for(T, M, GEMM_TILES), tile_for(T, N, GEMM_TILES)
    return (tm, tn) if tm is not None and tn is not None else None


def _call_or_unsupported(fn, what):
    """fn() or None when the library refuses the shape as not built (code 2)."""
    try:
        return fn()
    except RuntimeError as e:
        assert getattr(e, "code", None) == 2, f"{what}: {e}"
        return None


SHAPES = np.random.default_rng(20261202)


@pytest.mark.parametrize("M,N,K", [tuple(int(v) for v in SHAPES.integers(1, 300, 3))
                                   for _ in range(8)])
def test_matmul_random(lh, M, N, K):
    rng = np.random.default_rng(M * 1000003 + N * 1009 + K)
    x, y = _ints(rng, (M, K)), _ints(rng, (K, N))
    ref = oracle.matmul(x, y)
    got = host(lh.matmul(dev(x), dev(y)))
    assert np.array_equal(got, ref), (M, N, K, "preferred tiles")
    tiles = _random_gemm_tiles(rng, M, N)
    if tiles:
        got = host(lh.matmul(dev(x), dev(y), tile_m=tiles[0], tile_n=tiles[1]))
        assert np.array_equal(got, ref), (M, N, K, tiles)


@pytest.mark.parametrize("B,M,N,K", [tuple(int(v) for v in np.concatenate(
    [SHAPES.integers(1, 5, 1), SHAPES.integers(1, 200, 3)])) for _ in range(6)])
def test_batch_matmul_random(lh, B, M, N, K):
    rng = np.random.default_rng(B * 7 + M * 1000003 + N * 1009 + K)
    a, b = _ints(rng, (B, M, K)), _ints(rng, (B, K, N))
    got = host(lh.batch_matmul(dev(a), dev(b)))
    for i in range(B):
        assert np.array_equal(got[i], oracle.matmul(a[i], b[i])), (B, M, N, K, i)


@pytest.mark.parametrize("M,N,K,tk", [tuple(int(v) for v in (*SHAPES.integers(1, 200, 2), k,
                                                               SHAPES.integers(8, k + 1)))
                                      for k in SHAPES.integers(8, 2000, 6)])
def test_split_k_random(lh, M, N, K, tk):
    rng = np.random.default_rng(M * 31 + N * 7 + K + tk)
    a, b = _ints(rng, (M, K)), _ints(rng, (K, N))
    res = _call_or_unsupported(lambda: lh.split_k_matmul_gather(dev(a), dev(b), tile_k=tk),
                               f"split-K {M}x{N}x{K} tile_k {tk}")
    if res is None:
        return
    out, parts = res
    o_ref, p_ref = oracle.split_k_matmul_gather(a, b, min(16, M), min(16, N), tk)
    assert np.array_equal(parts.cpu().numpy(), p_ref), (M, N, K, tk, "partials")
    assert np.array_equal(host(out), o_ref), (M, N, K, tk, "out")


# every draw must launch: ragged Skv (not a multiple of 8) takes the
# register-staged K path, multiples of 8 the LDS-DMA one
@pytest.mark.parametrize("BH,Sq,Skv,D,causal", [
    (int(SHAPES.integers(1, 4)), int(sq), int(sq) if c else int(SHAPES.integers(1, 700)),
     int(SHAPES.choice([64, 128])), bool(c))
    for sq, c in zip(SHAPES.integers(1, 700, 6), [1, 0, 1, 0, 1, 0])])
def test_attention_random(lh, BH, Sq, Skv, D, causal):
    rng = np.random.default_rng(BH * 13 + Sq * 101 + Skv + D)
    k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
    print(f"attention random BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}", flush=True)
    got = lh.attention(dev(k), dev(v), dev(q), causal=causal)
    ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
    assert_close(from_bf16(host(got)), ref, **ATTN_TOL,
                 what=f"attention BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}")


@pytest.mark.parametrize("B,H,D,S", [(int(SHAPES.integers(1, 5)), int(SHAPES.integers(1, 33)),
                                      int(SHAPES.choice([64, 128])), int(s))
                                     for s in SHAPES.integers(1, 3000, 6)])
def test_decode_random(lh, B, H, D, S):
    rng = np.random.default_rng(B * 17 + H * 3 + D + S)
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    scale = 1 / math.sqrt(D)
    got = _call_or_unsupported(lambda: lh.flash_decode(dev(k), dev(v), dev(q), scale=scale),
                               f"decode B{B} H{H} D{D} S{S}")
    if got is None:
        return
    ts = min(128, S)
    ref, _, _ = oracle.flash_decode(k, v, q, scale, 1, ts, min(64, ts))
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=f"decode B{B} H{H} D{D} S{S}")


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("BH,Sq,Skv,D,causal,tile_m", [
    (2, 100, 381, 128, False, 256), (1, 381, 381, 128, True, 128), (2, 77, 250, 64, False, 64),
    (1, 250, 250, 64, True, 192), (3, 5, 5, 128, True, 64), (1, 1, 13, 64, False, 64),
    (2, 333, 1003, 128, False, 256)])
def test_attention_skv_not_multiple_of_8(lh, f16, BH, Sq, Skv, D, causal, tile_m):
    """Skv not a multiple of 8 (odd and even, below one 8-key piece, causal
    and not): K rows do not start on 16-byte boundaries and K is staged
    through registers; against the oracle in the tensors' element type."""
    tile_m = tile_m if tile_m <= Sq else Sq          # bounded by Sq (natural_ub)
    print(f"attention ragged Skv BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal} "
          f"tile_m={tile_m} f16={f16}", flush=True)
    rng = np.random.default_rng(Skv * 31 + Sq + D + f16)
    if f16:
        k, v, q = _rnd16(rng, (BH, D, Skv)), _rnd16(rng, (BH, Skv, D)), _rnd16(rng, (BH, Sq, D))
        got = _host16(lh.attention(_dev16(k), _dev16(v), _dev16(q), causal=causal, tile_m=tile_m))
        with oracle.element_type("f16"):
            ref = oracle.from_f16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
        gotf = oracle.from_f16(got)
    else:
        k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
        gotf = from_bf16(host(lh.attention(dev(k), dev(v), dev(q), causal=causal, tile_m=tile_m)))
        ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
    assert_close(gotf, ref, **ATTN_TOL,
                 what=f"attention Skv{Skv} Sq{Sq} D{D} causal={causal} f16={f16}")


@pytest.mark.parametrize("Skv", [250, 381, 1000])
def test_attention_k_two_byte_aligned(lh, Skv):
    """k starting 2 bytes past a 4-byte boundary (a view at an odd element
    offset): with Skv not a multiple of 8 the register-staged K loads shift
    misaligned pieces into place; with Skv a multiple of 8 such a k is refused
    (its rows would not start on 16-byte boundaries for the LDS DMA)."""
    BH, Sq, D = 2, 123, 128
    rng = np.random.default_rng(Skv + 5)
    k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
    flat = torch.empty(BH * D * Skv + 1, dtype=torch.bfloat16, device="cuda")
    kd = flat[1:].view(BH, D, Skv)
    kd.copy_(dev(k))
    assert kd.data_ptr() % 4 == 2
    print(f"attention k at 2 mod 4 Skv{Skv}", flush=True)
    if Skv % 8 == 0:
        with pytest.raises(RuntimeError) as ei:
            lh.attention(kd, dev(v), dev(q))
        assert ei.value.code == 1 and "aligned" in str(ei.value)
        return
    got = from_bf16(host(lh.attention(kd, dev(v), dev(q))))
    ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), False, 1, 64, 64))
    assert_close(got, ref, **ATTN_TOL, what=f"attention k at 2 mod 4, Skv{Skv}")


def _mamba_case(rng):
    G = int(rng.choice([1, 2]))
    H = G * int(rng.choice([1, 2]))
    Q = int(16 * rng.integers(1, 17))
    P = int(rng.choice([16, 32, 48, 64, 96, 128]))
    N = int(rng.choice([16, 32, 64, 96, 128]))
    return int(rng.integers(1, 3)), int(rng.integers(1, 4)), H, G, Q, P, N


@pytest.mark.parametrize("case", [_mamba_case(SHAPES) for _ in range(8)])
def test_mamba_prologue_and_scan_random(lh, case):
    b, nc, H, G, Q, P, N = case
    rng = np.random.default_rng(hash(case) % (1 << 32))
    L = nc * Q
    x = rng_bf16(rng, (b, H, L, P))
    Bm, C = rng_bf16(rng, (b, G, L, N)), rng_bf16(rng, (b, G, L, N))
    dt_raw = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
    A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
    Dh = rng.standard_normal(H).astype(np.float32)
    dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt_raw, A, Bm, C, Q)
    res = _call_or_unsupported(lambda: lh.ssd_prologue(dev(x), devf(dt_raw), devf(A), dev(Bm),
                                                       dev(C), Q), f"ssd_prologue {case}")
    if res is not None:
        _, dA, cb, prev = res
        torch.cuda.synchronize()
        dA_g = dA.cpu().numpy()
        assert np.all(np.abs(dA_g - dA_o) <= 1e-5 * (1 + np.abs(dA_o))), f"{case}: dA_cumsum"
        cb_g, cb_r = from_bf16(host(cb)), from_bf16(cb_o)
        assert not np.any(np.abs(cb_g - cb_r) > 2.0 ** -7 * np.abs(cb_r) + 1e-5), f"{case}: cb"
        prev_g = prev.cpu().numpy()
        scale = 1e-2 * max(float(np.abs(prev_o).max()), 1e-30)
        assert not np.any(np.abs(prev_g - prev_o) > 1e-3 * (np.abs(prev_o) + scale)), \
            f"{case}: prev_states_T"
    tm = tile_for(int(rng.choice(MAMBA_M_TILES)), Q, MAMBA_M_TILES)
    out = _call_or_unsupported(
        lambda: lh.helion_mamba2_chunk_scan_kernel(dev(cb_o), dev(x), devf(dt_o), devf(dA_o),
                                                   dev(C), devf(Dh), devf(prev_o), tile_m=tm),
        f"chunk scan {case} tile_m {tm}")
    if out is None:
        return
    ref = oracle.mamba_chunk_scan(cb_o, x, dt_o, dA_o, C, Dh, prev_o, 64, 64, 64)
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=f"chunk scan {case} tile_m {tm}")


# ------------------------------------------------------------- f16 variants
# The same draws for the *_f16 entry points (every 16-bit tensor IEEE
# binary16; the chunk scan's dt, dA_cumsum, D and prev_states_T f16 too, the
# reference's own signature), against the oracle in f16 mode.

def _dev16(h):
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).view(torch.float16).cuda()


def _host16(t):
    assert t.dtype == torch.float16
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _ints16(rng, shape, lo=-4, hi=4):
    return oracle.to_f16(rng.integers(lo, hi + 1, shape).astype(np.float32))


def _rnd16(rng, shape):
    return oracle.to_f16(rng.standard_normal(shape).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [tuple(int(v) for v in SHAPES.integers(1, 300, 3))
                                   for _ in range(3)])
def test_matmul_f16_random(lh, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    x, y = _ints16(rng, (M, K)), _ints16(rng, (K, N))
    with oracle.element_type("f16"):
        ref = oracle.matmul(x, y)
    assert np.array_equal(_host16(lh.matmul(_dev16(x), _dev16(y))), ref), (M, N, K)


@pytest.mark.parametrize("M,N,K,tk", [tuple(int(v) for v in (*SHAPES.integers(1, 200, 2), k,
                                                               SHAPES.integers(8, k + 1)))
                                      for k in SHAPES.integers(8, 2000, 3)])
def test_split_k_f16_random(lh, M, N, K, tk):
    rng = np.random.default_rng(M * 3 + N * 5 + K + tk)
    a, b = _ints16(rng, (M, K)), _ints16(rng, (K, N))
    res = _call_or_unsupported(lambda: lh.split_k_matmul_gather(_dev16(a), _dev16(b), tile_k=tk),
                               f"split-K f16 {M}x{N}x{K} tile_k {tk}")
    if res is None:
        return
    out, parts = res
    with oracle.element_type("f16"):
        o_ref, p_ref = oracle.split_k_matmul_gather(a, b, min(16, M), min(16, N), tk)
    assert np.array_equal(parts.cpu().numpy(), p_ref), (M, N, K, tk, "partials")
    assert np.array_equal(_host16(out), o_ref), (M, N, K, tk, "out")


# the first f16 draw is pinned to D = 64 (the other head size's f16 kernels)
@pytest.mark.parametrize("BH,S,D,causal", [(int(SHAPES.integers(1, 4)), int(s),
                                            64 if i == 0 else d, bool(c))
                                           for i, (s, c, d) in enumerate(
                                               zip(SHAPES.integers(1, 600, 3), [1, 0, 1],
                                                   [int(SHAPES.choice([64, 128]))
                                                    for _ in range(3)]))])
def test_attention_f16_random(lh, BH, S, D, causal):
    rng = np.random.default_rng(BH * 11 + S + D)
    k, v, q = _rnd16(rng, (BH, D, S)), _rnd16(rng, (BH, S, D)), _rnd16(rng, (BH, S, D))
    print(f"attention f16 random BH{BH} S{S} D{D} causal={causal}", flush=True)
    got = lh.attention(_dev16(k), _dev16(v), _dev16(q), causal=causal)
    with oracle.element_type("f16"):
        ref = oracle.from_f16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
    assert_close(oracle.from_f16(_host16(got)), ref, **ATTN_TOL,
                 what=f"attention f16 BH{BH} S{S} D{D} causal={causal}")


@pytest.mark.parametrize("B,H,D,S", [(int(SHAPES.integers(1, 5)), int(SHAPES.integers(1, 33)),
                                      int(SHAPES.choice([64, 128])), int(s))
                                     for s in SHAPES.integers(1, 3000, 3)])
def test_decode_f16_random(lh, B, H, D, S):
    rng = np.random.default_rng(B * 19 + H * 5 + D + S)
    k, v, q = _rnd16(rng, (B, D, S)), _rnd16(rng, (B, S, D)), _rnd16(rng, (B, H, D))
    scale = 1 / math.sqrt(D)
    got = _call_or_unsupported(lambda: lh.flash_decode(_dev16(k), _dev16(v), _dev16(q), scale=scale),
                               f"decode f16 B{B} H{H} D{D} S{S}")
    if got is None:
        return
    ts = min(128, S)
    with oracle.element_type("f16"):
        ref, _, _ = oracle.flash_decode(k, v, q, scale, 1, ts, min(64, ts))
    assert_close(oracle.from_f16(_host16(got)), oracle.from_f16(ref), **ATTN_TOL,
                 what=f"decode f16 B{B} H{H} D{D} S{S}")


@pytest.mark.parametrize("case", [_mamba_case(SHAPES) for _ in range(3)])
def test_mamba_chunk_scan_f16_random(lh, case):
    """The chunk scan's f16 signature (every tensor f16) on the oracle's f16
    prologue outputs rounded to f16."""
    b, nc, H, G, Q, P, N = case
    rng = np.random.default_rng(hash(case) % (1 << 31) + 7)
    L = nc * Q
    x = _rnd16(rng, (b, H, L, P))
    Bm, C = _rnd16(rng, (b, G, L, N)), _rnd16(rng, (b, G, L, N))
    dt_raw = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
    A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
    Dh = rng.standard_normal(H).astype(np.float32)
    h16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    with oracle.element_type("f16"):
        dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt_raw, A, Bm, C, Q)
        dt_h, dA_h, D_h, prev_h = h16(dt_o), h16(dA_o), h16(Dh), h16(prev_o)
        ref = oracle.mamba_chunk_scan(cb_o, x, dt_h, dA_h, C, D_h, prev_h, 64, 64, 64)
    f16 = lambda a: torch.from_numpy(a).to(torch.float16).cuda()  # noqa: E731
    out = _call_or_unsupported(
        lambda: lh.helion_mamba2_chunk_scan_kernel(_dev16(cb_o), _dev16(x), f16(dt_h), f16(dA_h),
                                                   _dev16(C), f16(D_h), f16(prev_h)),
        f"chunk scan f16 {case}")
    if out is None:
        return
    assert_close(oracle.from_f16(_host16(out)), oracle.from_f16(ref), **ATTN_TOL,
                 what=f"chunk scan f16 {case}")
