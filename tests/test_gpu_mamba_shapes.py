"""GPU parity of the Mamba-2 kernels at chunk and state sizes beyond the
default build's: chunks up to 512 keys and states up to 256 wide (the chunk
scan's 4-wave long build), chunk sizes that are not a multiple of 32 above
128 (the SSD state kernel's 16-key unit multiples), dstate that 64 does not
divide (32-wide n blocks) and headdim up to 256.

Every element of every output is compared with the CPU oracle, at the bars
of tests/test_gpu_ssd.py for the prologue (dA_cumsum 1e-5 (1 + |ref|), cb
one bf16 step, prev_states_T 1e-3 (|ref| + scale)) and of
tests/test_gpu_parity.py for the chunk scan (2e-2 + 1e-2 |ref|); the f16
case in the f16 oracle mode.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16, from_f16, to_f16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, _mamba_gpu, _mamba_inputs, dev, devf, host
from tests.test_gpu_ssd import _check_prologue, _raw_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


# (b, nc, H, G, Q, P, N, tile_m, tile_n)
SCAN_SHAPES = [
    (1, 2, 4, 1, 512, 64, 128, 256, 64),    # long chunk, two 256-row m-tiles
    (1, 2, 4, 1, 512, 64, 128, 128, 32),    # four m-tiles, two p-tiles
    (1, 3, 4, 2, 256, 64, 256, 256, 64),    # wide state, two groups
    (1, 2, 4, 1, 384, 96, 192, 192, 32),
    (2, 2, 2, 1, 320, 128, 160, 64, 16),
    (1, 2, 2, 1, 512, 128, 256, 256, 64),   # both limits
    (1, 2, 3, 1, 264, 40, 136, 128, 16),    # multiples of 8 only
    (1, 1, 2, 1, 504, 24, 248, 256, 16),
]


@pytest.mark.parametrize("b,nc,H,G,Q,P,N,tm,tn", SCAN_SHAPES)
def test_chunk_scan_long_chunks_and_wide_states(lh, b, nc, H, G, Q, P, N, tm, tn):
    print(f"chunk scan b{b} c{nc} H{H} G{G} Q{Q} P{P} N{N} tiles {tm}x{tn}", flush=True)
    rng = np.random.default_rng(b * 1000 + Q + 7 * N + P)
    cb, x, dt, dA, C, Dh, prev = _mamba_inputs(rng, b, nc, H, G, Q, P, N)
    ref = oracle.mamba_chunk_scan(cb, x, dt, dA, C, Dh, prev, 64, 64, 64)
    out = _mamba_gpu(lh, cb, x, dt, dA, C, Dh, prev, tile_m=tm, tile_n=tn)
    assert_close(from_bf16(out), from_bf16(ref), **ATTN_TOL,
                 what=f"chunk scan Q{Q} P{P} N{N} {tm}x{tn}")


def test_chunk_scan_long_build_f16(lh):
    """The long build in f16 (every tensor f16, the reference's signature)."""
    print("chunk scan f16 Q512 P64 N256", flush=True)
    rng = np.random.default_rng(77)
    b, nc, H, G, Q, P, N = 1, 2, 2, 1, 512, 64, 256
    with oracle.element_type("f16"):
        L = nc * Q
        x = to_f16(rng.standard_normal((b, H, L, P)).astype(np.float32))
        Bm = to_f16(rng.standard_normal((b, G, L, N)).astype(np.float32))
        C = to_f16(rng.standard_normal((b, G, L, N)).astype(np.float32))
        dt_raw = np.log1p(np.exp(rng.standard_normal((b, H, L)))).astype(np.float32)
        A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
        dt, dA, cb, prev = oracle.mamba_prologue(x, dt_raw, A, Bm, C, Q)
        h16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
        dt_h, dA_h, prev_h = h16(dt), h16(dA), h16(prev)
        D_h = h16(rng.standard_normal(H).astype(np.float32))
        ref = oracle.mamba_chunk_scan(cb, x, dt_h, dA_h, C, D_h, prev_h, 64, 64, 64)
    d16 = lambda h: torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).view(  # noqa: E731
        torch.float16).cuda()
    f16 = lambda a: torch.from_numpy(a).to(torch.float16).cuda()  # noqa: E731
    out = lh.helion_mamba2_chunk_scan_kernel(d16(cb), d16(x), f16(dt_h), f16(dA_h), d16(C),
                                             f16(D_h), f16(prev_h), tile_m=256, tile_n=64)
    assert out.dtype == torch.float16
    got = out.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    assert_close(from_f16(got), from_f16(ref), **ATTN_TOL, what="chunk scan f16 long build")


# (b, H, G, Q, nc, P, N): the state kernel's unit plan and n block for each
PROLOGUE_SHAPES = [
    (1, 2, 1, 512, 2, 64, 128),    # 256-key units, two per chunk
    (1, 4, 2, 256, 2, 64, 256),    # cb over 256-wide states, four 64-wide n blocks
    (1, 2, 1, 144, 3, 64, 64),     # 48-key units (144 = 3 x 48)
    (1, 2, 1, 176, 2, 128, 96),    # 16-key units, 32-wide n blocks (64 does not divide 96)
    (1, 2, 1, 240, 2, 160, 160),   # 80-key units, headdim 160
    (1, 2, 1, 512, 2, 256, 256),   # every limit at once
    (1, 3, 1, 96, 2, 64, 96),      # one 96-key unit, 32-wide n blocks
]


@pytest.mark.parametrize("b,H,G,Q,nc,P,N", PROLOGUE_SHAPES)
def test_ssd_prologue_and_chain_new_shapes(lh, b, H, G, Q, nc, P, N):
    """GPU prologue against the oracle's prologue, then the GPU chunk scan on
    the GPU prologue's outputs against the oracle's chain."""
    what = f"prologue b{b} H{H} G{G} Q{Q} c{nc} P{P} N{N}"
    print(what, flush=True)
    rng = np.random.default_rng(H * 100 + Q + N + P)
    x, dt, A, Bm, C = _raw_inputs(rng, b, H, G, nc * Q, P, N)
    dt_v, dA, cb, prev = _check_prologue(lh, x, dt, A, Bm, C, Q, what)
    Dh = rng.standard_normal(H).astype(np.float32)
    out = lh.helion_mamba2_chunk_scan_kernel(cb, dev(x), dt_v.contiguous(), dA, dev(C), devf(Dh),
                                             prev, tile_m=min(Q, 256), tile_n=min(P, 64))
    dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, Q)
    ref = oracle.mamba_chunk_scan(cb_o, x, dt_o, dA_o, C, Dh, prev_o, 64, 64, 64)
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what=f"{what} chain")
