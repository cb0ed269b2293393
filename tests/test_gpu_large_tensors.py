"""GPU parity on tensors larger than 4 GiB.

Every kernel forms its per-batch, per-head and per-chunk bases in 64-bit
arithmetic and keeps per-lane offsets within one tile, row block or head;
the GEMM kernels whose LDS-DMA copies take 32-bit per-lane offsets run only
when a tile's rows fit them (leading dimensions below 2^22), larger ones
take the 64-bit fallback kernels.  Each case here puts at least one operand,
output or workspace past 2^32 bytes and checks the elements that live past
that boundary (the last batch, head, rows or columns; for the GEMMs also
the rows that straddle it) against the CPU oracle: bit-exact for the GEMMs
on integer-valued inputs, at the parity bars of tests/test_gpu_parity.py for
attention, decode and the Mamba-2 chain.  Inputs are generated on the GPU
(torch's seeded generators) and only the checked slices travel to the host.
Peak device memory per case is below 20 GB.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, host

pytestmark = pytest.mark.gpu

FOUR_GIB = 1 << 32


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


@pytest.fixture(autouse=True)
def _free_device_memory():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _ints(shape, seed):
    """Integer-valued bf16 in [-4, 4] on the GPU (products and their sums
    stay exact in fp32)."""
    t = torch.randint(-4, 5, shape, generator=_gen(seed), device="cuda", dtype=torch.int8)
    return t.to(torch.bfloat16)


def _normal(shape, seed, std=1.0):
    t = torch.randn(shape, generator=_gen(seed), device="cuda", dtype=torch.bfloat16)
    return t.mul_(std) if std != 1.0 else t


def _big(t):
    return t.numel() * t.element_size() > FOUR_GIB


def _announce(what):
    print(f"large tensors: {what}", flush=True)


# ------------------------------------------------------------------- GEMMs

@pytest.mark.parametrize("case,M,N,K", [
    ("x past 4 GiB", 69632, 256, 32768),
    ("y past 4 GiB", 256, 69632, 32768),
    ("out past 4 GiB", 47104, 47104, 256),
    ("out past 4 GiB, K 64 (fallback kernels)", 47104, 47104, 64)])
def test_matmul_past_4gib(lh, case, M, N, K):
    x, y = _ints((M, K), 1), _ints((K, N), 2)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    assert _big(x) or _big(y) or _big(out)
    # the last rows, and the rows that straddle the 4 GiB point of x or out
    rows = set(range(M - 32, M))
    for t, ld in ((x, K), (out, N)):
        if _big(t):
            r = FOUR_GIB // (2 * ld)
            rows |= set(range(r - 32, min(r + 32, M)))
    rows = sorted(rows)
    # every column, or (y past 4 GiB: its rows past the point hold every
    # column) the first and the last 64
    cols = sorted({*range(64), *range(N - 64, N)}) if _big(y) else list(range(N))
    ref = oracle.matmul(host(x[rows]), host(y[:, cols].contiguous()))
    for t in (256, 128):
        _announce(f"matmul {case} M{M} N{N} K{K} tile {t}")
        lh.matmul(x, y, out, tile_m=t, tile_n=t)
        got = host(out[rows][:, cols].contiguous())
        np.testing.assert_array_equal(got, ref, err_msg=f"matmul {case} tile {t}")


@pytest.mark.parametrize("case,Bt,M,N,K", [
    ("A past 4 GiB, persistent kernel", 16, 8192, 512, 18432),
    ("C past 4 GiB, persistent kernel", 16, 8192, 16896, 256),
    ("A past 4 GiB, one tile per workgroup", 18, 8192, 256, 16384)])
def test_batch_matmul_past_4gib(lh, case, Bt, M, N, K):
    a, b = _ints((Bt, M, K), 3), _ints((Bt, K, N), 4)
    c = torch.empty((Bt, M, N), dtype=torch.bfloat16, device="cuda")
    assert _big(a) or _big(c)
    _announce(f"batch_matmul {case} B{Bt} M{M} N{N} K{K}")
    lh.batch_matmul(a, b, c, tile_m=256, tile_n=256)
    cols = slice(N - 512, N) if N > 512 else slice(0, N)
    for z, rows in ((Bt - 1, slice(M - 64, M)), (Bt - 2, slice(M // 2 - 32, M // 2 + 32)),
                    (0, slice(0, 32))):
        ref = oracle.matmul(host(a[z, rows]), host(b[z, :, cols].contiguous()))
        np.testing.assert_array_equal(host(c[z, rows, cols].contiguous()), ref,
                                      err_msg=f"batch_matmul {case} batch {z}")


@pytest.mark.parametrize("case,M,N,K,tile_k,tiles", [
    ("partials past 4 GiB", 8192, 8192, 17408, 1024, (256,)),
    ("A and B rows past 2^22 elements (fallback kernels)", 512, 512, 5242880, 16384, (256, 128))])
def test_split_k_past_4gib(lh, case, M, N, K, tile_k, tiles):
    a, b = _ints((M, K), 5), _ints((K, N), 6)
    S = -(-K // tile_k)
    parts = torch.empty((S, M, N), dtype=torch.float32, device="cuda")
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    assert _big(parts) or _big(a)
    n = 64 if K < (1 << 20) else 16
    rs, cs = slice(M - n, M), slice(N - n, N)
    ref, ref_parts = oracle.split_k_matmul_gather(host(a[rs]), host(b[:, cs].contiguous()),
                                                  n, n, tile_k)
    for t in tiles:
        _announce(f"split_k {case} M{M} N{N} K{K} tile_k {tile_k} tile {t}")
        lh.split_k_matmul_gather(a, b, out, parts, tile_m=t, tile_n=t, tile_k=tile_k)
        np.testing.assert_array_equal(parts[:, rs, cs].cpu().numpy(), ref_parts,
                                      err_msg=f"split_k {case} partials, tile {t}")
        np.testing.assert_array_equal(host(out[rs, cs].contiguous()), ref,
                                      err_msg=f"split_k {case} output, tile {t}")


# --------------------------------------------------------------- attention

@pytest.mark.parametrize("case,BH,Sq,Skv,D", [
    ("K, V past 4 GiB, Skv odd (K staged through registers)", 4200, 64, 4095, 128),
    ("K, V past 4 GiB, head dim 256", 2100, 64, 4096, 256),
    ("K, V past 4 GiB, head dim 96", 5600, 64, 4096, 96)])
def test_attention_past_4gib(lh, case, BH, Sq, Skv, D):
    k, v, q = _normal((BH, D, Skv), 7), _normal((BH, Skv, D), 8), _normal((BH, Sq, D), 9)
    assert _big(k) and _big(v)
    _announce(f"attention {case} BH{BH} Sq{Sq} Skv{Skv} D{D}")
    scale = 1 / math.sqrt(D)
    out = lh.attention(k, v, q, scale=scale)
    heads = [0, BH // 2, BH - 2, BH - 1]
    ref = oracle.attention(host(k[heads]), host(v[heads]), host(q[heads]), scale, False, 1, 64, 64)
    assert_close(from_bf16(host(out[heads])), from_bf16(ref), **ATTN_TOL,
                 what=f"attention {case}")


def test_attention_causal_past_4gib(lh):
    """Causal, BH 1040 S 16384 D 128: K, V, Q and out each past 4 GiB.  The
    last head's last query rows against the oracle, row i as a non-causal
    attention over keys 0..i."""
    BH, S, D = 1040, 16384, 128
    k, v, q = _normal((BH, D, S), 10), _normal((BH, S, D), 11), _normal((BH, S, D), 12)
    assert _big(k) and _big(v) and _big(q)
    _announce(f"attention causal BH{BH} S{S} D{D}")
    scale = 1 / math.sqrt(D)
    out = lh.attention(k, v, q, scale=scale, causal=True)
    kh, vh, qh = host(k[-1]), host(v[-1]), host(q[-1])
    got = from_bf16(host(out[-1]))
    for i in (*range(S - 8, S), S // 2, 4095, 0):
        ref = oracle.attention(np.ascontiguousarray(kh[None, :, :i + 1]), vh[None, :i + 1],
                               qh[None, i:i + 1], scale, False, 1, 1, 64)
        assert_close(got[i:i + 1], from_bf16(ref[0]), **ATTN_TOL,
                     what=f"attention causal last head row {i}")


# ------------------------------------------------------------------ decode

@pytest.mark.parametrize("case,B,H,D,S,ts", [
    ("LDS-DMA kernel", 520, 32, 128, 32768, 1024),
    ("register kernel (S odd)", 520, 32, 128, 32767, 1024),
    ("64-head workgroups, K through registers", 350, 48, 128, 49151, 2048),
    ("head dim 256", 260, 32, 256, 32768, 1024)])
def test_decode_past_4gib(lh, case, B, H, D, S, ts):
    k, v, q = _normal((B, D, S), 13), _normal((B, S, D), 14), _normal((B, H, D), 15)
    assert _big(k) and _big(v)
    _announce(f"flash_decode {case} B{B} H{H} D{D} S{S} tile_s {ts}")
    scale = 1 / math.sqrt(D)
    out, lse, o = lh.flash_decode(k, v, q, scale=scale, tile_s=ts, return_partials=True)
    bs = [0, B - 2, B - 1]
    ref, ref_lse, ref_o = oracle.flash_decode(host(k[bs]), host(v[bs]), host(q[bs]), scale, 1, ts,
                                              512)
    assert_close(from_bf16(host(out[bs])), from_bf16(ref), **ATTN_TOL, what=f"decode {case}")
    assert_close(lse[:, bs].cpu().numpy(), ref_lse, atol=1e-2, rtol=1e-3,
                 what=f"decode {case} lse_s")
    assert_close(o[:, bs].cpu().numpy(), ref_o, **ATTN_TOL, what=f"decode {case} o_s")


# ----------------------------------------------------------------- Mamba-2

def test_mamba_chain_past_4gib(lh):
    """b1 H264 L65536 P128 N128 Q256 (256 chunks): x, the SSD
    prologue's prev_states_T and the chunk scan's out each past 4 GiB.  The
    last head's prologue outputs against the oracle's prologue of that head
    (its state carried over all 256 chunks), and its last 8 chunks of the
    chunk scan against the oracle's scan of them on the same inputs."""
    b, H, G, Q, nc, P, N = 1, 264, 1, 256, 256, 128, 128
    L = nc * Q
    x = _normal((b, H, L, P), 16)
    Bm, C = _normal((b, G, L, N), 17), _normal((b, G, L, N), 18)
    g = _gen(19)
    dt = torch.nn.functional.softplus(torch.randn((b, H, L), generator=g, device="cuda"))
    A = -torch.exp(torch.rand(H, generator=g, device="cuda"))
    Dh = torch.randn(H, generator=g, device="cuda")
    assert _big(x)
    _announce(f"ssd_prologue b{b} H{H} L{L} P{P} N{N}")
    dt_v, dA, cb, prev = lh.ssd_prologue(x, dt, A, Bm, C, Q)
    assert _big(prev)
    xh = host(x[:, -1:])
    Bh, Ch = host(Bm), host(C)
    dth = dt[:, -1:].contiguous().cpu().numpy()
    dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(xh, dth, A[-1:].cpu().numpy(), Bh, Ch, Q)
    np.testing.assert_array_equal(dt_v[:, -1:].cpu().numpy(), dt_o)
    dA_g = dA[:, -1:].cpu().numpy()
    assert np.all(np.abs(dA_g - dA_o) <= 1e-5 * (1 + np.abs(dA_o))), "dA_cumsum"
    cb_g, cb_r = from_bf16(host(cb)), from_bf16(cb_o)
    assert not np.any(np.abs(cb_g - cb_r) > 2.0 ** -7 * np.abs(cb_r) + 1e-5), "cb"
    prev_g = prev[:, :, -1:].cpu().numpy()
    scale = 1e-2 * max(float(np.abs(prev_o).max()), 1e-30)
    bad = np.abs(prev_g - prev_o) > 1e-3 * (np.abs(prev_o) + scale)
    assert not bad.any(), f"prev_states_T: {int(bad.sum())} of {bad.size} off"

    _announce(f"chunk scan b{b} H{H} L{L} P{P} N{N}")
    out = lh.helion_mamba2_chunk_scan_kernel(cb, x, dt_v.contiguous(), dA, C, Dh, prev,
                                             tile_m=256, tile_n=64)
    assert _big(out)
    last = 8
    ks = slice(L - last * Q, L)
    ref = oracle.mamba_chunk_scan(host(cb[:, -last:]), host(x[:, -1:, ks]),
                                  dt_v[:, -1:, -last:].contiguous().cpu().numpy(),
                                  dA[:, -1:, -last:].contiguous().cpu().numpy(), host(C[:, :, ks]),
                                  Dh[-1:].cpu().numpy(),
                                  prev[:, -last:, -1:].contiguous().cpu().numpy(), 64, 64, 64)
    assert_close(from_bf16(host(out[:, -1:, ks])), from_bf16(ref), **ATTN_TOL,
                 what="chunk scan last head, last 8 chunks")
