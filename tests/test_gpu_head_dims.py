"""GPU parity at head dims other than the built ones.

attention and flash_decode are built for head_dim 64, 128 and 256; any
multiple of 8 up to 256 runs on the next one up, with the K rows and q elements past the real head dim zero and the V
columns past it reaching only O columns that are never stored.  Each case
compares the whole output (and, for decode, the gathered split partials
lse_s and o_s) with the CPU oracle, at the bars of
tests/test_gpu_parity.py, on every K staging path (16-byte LDS DMA when the
key count is a multiple of 8, registers into LDS otherwise -- decode's
LDS-DMA kernel does that for S = 2 mod 4 and above D 128, its register
kernel for the other S) and in both 16-bit types.
The out buffers are pre-filled with a sentinel so a store past the head dim
into a neighbouring row would show.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16, from_f16, to_bf16, to_f16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, dev, host, rng_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _sentinel(shape, dtype):
    return torch.full(shape, 1234.0, dtype=dtype, device="cuda")


@pytest.mark.parametrize("BH,Sq,Skv,D,causal,tile_m", [
    (2, 200, 200, 8, True, 64), (1, 130, 517, 24, False, 128), (2, 300, 300, 40, True, 256),
    (1, 96, 1000, 56, False, 192), (2, 257, 257, 72, True, 256), (1, 64, 333, 96, False, 64),
    (3, 190, 190, 96, True, 128), (1, 120, 640, 120, False, 256), (2, 300, 300, 256, True, 256),
    (1, 200, 517, 256, False, 64), (2, 150, 640, 136, False, 128), (1, 333, 333, 200, True, 192)])
def test_attention_head_dims(lh, BH, Sq, Skv, D, causal, tile_m):
    rng = np.random.default_rng(BH * 7 + Sq * 13 + Skv * 3 + D)
    k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
    tile_m = min(tile_m, Sq)
    print(f"attention head dim BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal} tile_m {tile_m}",
          flush=True)
    out = _sentinel((BH, Sq, D), torch.bfloat16)
    lh.attention(dev(k), dev(v), dev(q), out, causal=causal, tile_m=tile_m)
    ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
    assert_close(from_bf16(host(out)), ref, **ATTN_TOL,
                 what=f"attention BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}")


def test_attention_head_dim_f16(lh):
    """f16 at D 96 (the 128 kernel), D 40 (the 64 kernel, ragged Skv) and
    D 256."""
    for BH, Sq, Skv, D, causal in ((2, 160, 160, 96, True), (1, 70, 301, 40, False),
                                   (2, 130, 130, 256, True)):
        rng = np.random.default_rng(Sq + D)
        k = to_f16(rng.standard_normal((BH, D, Skv)).astype(np.float32))
        v = to_f16(rng.standard_normal((BH, Skv, D)).astype(np.float32))
        q = to_f16(rng.standard_normal((BH, Sq, D)).astype(np.float32))
        print(f"attention f16 head dim BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}", flush=True)
        tk = torch.from_numpy(k.view(np.int16)).view(torch.float16).cuda()
        tv = torch.from_numpy(v.view(np.int16)).view(torch.float16).cuda()
        tq = torch.from_numpy(q.view(np.int16)).view(torch.float16).cuda()
        out = _sentinel((BH, Sq, D), torch.float16)
        lh.attention(tk, tv, tq, out, causal=causal)
        with oracle.element_type("f16"):
            ref = from_f16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
        got = from_f16(out.view(torch.int16).cpu().numpy().view(np.uint16))
        assert_close(got, ref, **ATTN_TOL, what=f"attention f16 D{D}")


@pytest.mark.parametrize("B,H,D,S,ts", [
    (2, 8, 8, 1024, 256), (3, 5, 40, 1000, 200), (2, 33, 72, 2048, 512), (1, 32, 96, 777, 128),
    (4, 16, 96, 4096, 1024), (2, 3, 120, 1203, 300), (1, 40, 56, 640, 64), (2, 32, 256, 2048, 512),
    (3, 37, 136, 1000, 200), (1, 8, 200, 640, 128), (2, 20, 256, 1001, 256), (1, 33, 200, 1002, 128),
    (2, 32, 128, 2006, 512), (3, 7, 64, 998, 100), (2, 32, 128, 4099, 1024), (1, 17, 256, 1203, 300)])
def test_decode_head_dims(lh, B, H, D, S, ts):
    rng = np.random.default_rng(B * 5 + H * 11 + D * 3 + S)
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    scale = 1 / math.sqrt(D)
    print(f"decode head dim B{B} H{H} D{D} S{S} tile_s {ts}", flush=True)
    out = _sentinel((B, H, D), torch.bfloat16)
    _, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), out, scale=scale, tile_s=ts,
                                return_partials=True)
    ref, ref_lse, ref_o = oracle.flash_decode(k, v, q, scale, 1, ts, min(64, ts))
    what = f"decode B{B} H{H} D{D} S{S} tile_s {ts}"
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=what)
    assert_close(lse.cpu().numpy(), ref_lse, atol=1e-2, rtol=1e-3, what=what + " lse_s")
    assert_close(o.cpu().numpy(), ref_o, **ATTN_TOL, what=what + " o_s")


def test_decode_head_dim_noalloc_and_f16(lh):
    """The allocation-free entry point at D 72 (bit-identical to the
    workspace form) and the f16 entry point with S not a multiple of 8 on
    each ragged path: D 48 S 1001 (register kernel), D 128 S 1002 and D 256
    S 777 (K staged through registers into the LDS-DMA kernel)."""
    rng = np.random.default_rng(4242)
    B, H, D, S = 2, 32, 72, 3000
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    print(f"decode head dim noalloc B{B} H{H} D{D} S{S}", flush=True)
    ref = lh.flash_decode(dev(k), dev(v), dev(q), tile_s=1000)
    out = _sentinel((B, H, D), torch.bfloat16)
    lh.flash_decode_noalloc(dev(k), dev(v), dev(q), out, tile_s=1000)
    assert torch.equal(out, ref)

    for B, H, D, S in ((2, 12, 48, 1001), (2, 32, 128, 1002), (1, 9, 256, 777)):
        _decode_f16(lh, rng, B, H, D, S)


def _decode_f16(lh, rng, B, H, D, S):
    k = to_f16(rng.standard_normal((B, D, S)).astype(np.float32))
    v = to_f16(rng.standard_normal((B, S, D)).astype(np.float32))
    q = to_f16(rng.standard_normal((B, H, D)).astype(np.float32))
    print(f"decode f16 head dim B{B} H{H} D{D} S{S}", flush=True)
    t = [torch.from_numpy(a.view(np.int16)).view(torch.float16).cuda() for a in (k, v, q)]
    out = _sentinel((B, H, D), torch.float16)
    lh.flash_decode(*t, out, tile_s=256)
    with oracle.element_type("f16"):
        ref, _, _ = oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 256, 64)
    got = from_f16(out.view(torch.int16).cpu().numpy().view(np.uint16))
    assert_close(got, from_f16(ref), **ATTN_TOL, what=f"decode f16 D{D}")


@pytest.mark.parametrize("D,S,ts", [(128, 1001, 256), (128, 1002, 1002), (64, 999, 100),
                                     (128, 1004, 101), (256, 1001, 512), (96, 1003, 333)])
def test_decode_keys_at_the_tensor_end(lh, D, S, ts):
    """The last keys of K's last row (d = D - 1 of the last batch) decide the
    output: they carry a large value that q's last element multiplies, so a
    load of them that straddled the end of the tensor and came back zero
    would shift the softmax to other keys.  Odd S, S = 2 mod 4 and S = 0 mod
    4 with an odd tile_s put 8-byte pieces across the end; D 96 pads."""
    rng = np.random.default_rng(D * 7 + S)
    B, H = 2, 8
    kf = rng.standard_normal((B, D, S)).astype(np.float32) * 0.1
    kf[:, D - 1, S - 3:] = 12.0
    qf = rng.standard_normal((B, H, D)).astype(np.float32) * 0.1
    qf[:, :, D - 1] = 4.0
    k, q = to_bf16(kf), to_bf16(qf)
    v = rng_bf16(rng, (B, S, D))
    scale = 1 / math.sqrt(D)
    print(f"decode tensor end B{B} H{H} D{D} S{S} tile_s {ts}", flush=True)
    got = lh.flash_decode(dev(k), dev(v), dev(q), scale=scale, tile_s=ts)
    ref, _, _ = oracle.flash_decode(k, v, q, scale, 1, ts, min(64, ts))
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL,
                 what=f"decode tensor end D{D} S{S} ts{ts}")


DRAWS = np.random.default_rng(20261203)


@pytest.mark.parametrize("B,H,D,S,ts", [
    (int(DRAWS.integers(1, 4)), int(DRAWS.integers(1, 70)), int(8 * DRAWS.integers(1, 33)),
     int(s), int(DRAWS.integers(1, s + 1))) for s in DRAWS.integers(1, 3000, 10)])
def test_decode_random_head_dims(lh, B, H, D, S, ts):
    """Seeded draws over the whole built space: D any multiple of 8 up to
    256, any S (every split path), any H (head groups past 32), any tile_s;
    output and partials against the oracle."""
    rng = np.random.default_rng(B + H * 3 + D * 5 + S * 7 + ts)
    k, v, q = rng_bf16(rng, (B, D, S)), rng_bf16(rng, (B, S, D)), rng_bf16(rng, (B, H, D))
    scale = 1 / math.sqrt(D)
    print(f"decode random B{B} H{H} D{D} S{S} tile_s {ts}", flush=True)
    got, lse, o = lh.flash_decode(dev(k), dev(v), dev(q), scale=scale, tile_s=ts,
                                  tile_n=min(ts, 64), return_partials=True)
    ref, ref_lse, ref_o = oracle.flash_decode(k, v, q, scale, 1, ts, min(64, ts))
    what = f"decode random B{B} H{H} D{D} S{S} tile_s {ts}"
    assert_close(from_bf16(host(got)), from_bf16(ref), **ATTN_TOL, what=what)
    assert_close(lse.cpu().numpy(), ref_lse, atol=1e-2, rtol=1e-3, what=what + " lse_s")
    assert_close(o.cpu().numpy(), ref_o, **ATTN_TOL, what=what + " o_s")


@pytest.mark.parametrize("BH,Sq,Skv,D,causal", [
    (int(DRAWS.integers(1, 4)), int(sq), int(sq) if c else int(DRAWS.integers(1, 900)),
     int(8 * DRAWS.integers(1, 33)), bool(c))
    for sq, c in zip(DRAWS.integers(1, 900, 8), [1, 0, 1, 0, 1, 0, 1, 0])])
def test_attention_random_head_dims(lh, BH, Sq, Skv, D, causal):
    """Seeded draws: D any multiple of 8 up to 256, any Sq and Skv (both K
    paths), causal and not, against the oracle."""
    rng = np.random.default_rng(BH + Sq * 3 + Skv * 5 + D * 7)
    k, v, q = rng_bf16(rng, (BH, D, Skv)), rng_bf16(rng, (BH, Skv, D)), rng_bf16(rng, (BH, Sq, D))
    print(f"attention random BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}", flush=True)
    got = lh.attention(dev(k), dev(v), dev(q), causal=causal)
    ref = from_bf16(oracle.attention(k, v, q, 1 / math.sqrt(D), causal, 1, 64, 64))
    assert_close(from_bf16(host(got)), ref, **ATTN_TOL,
                 what=f"attention random BH{BH} Sq{Sq} Skv{Skv} D{D} causal={causal}")
