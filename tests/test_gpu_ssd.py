"""GPU parity of the Mamba-2 SSD prologue (raw x, dt, A, B, C -> dA_cumsum,
cb, prev_states_T) against the CPU oracle's mamba_prologue, and the whole
chain (GPU prologue -> GPU chunk scan) against the sequential SSM
recurrence of the golden fixture.

Tolerances: dA_cumsum is an fp32 prefix sum in another association than the
oracle's serial loop: |d| <= 1e-5 (1 + |ref|).  cb is an fp32 MFMA sum
rounded to bf16: at most one bf16 rounding step apart, |d| <= 2^-7 |ref| +
1e-5, and exactly zero above the diagonal.  prev_states_T accumulates in fp32 with w * B split into bf16 hi + lo
(relative error ~2^-16 per term): |d| <= 1e-3 (|ref| + scale), scale = the
tensor's largest magnitude times 1e-2.  The chain keeps the chunk-scan
bar (2e-2 + 1e-2 |ref|; 3e-2 against the recurrence).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import from_bf16
from tests.conftest import assert_close
from tests.test_gpu_parity import ATTN_TOL, dev, devf, host, rng_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _raw_inputs(rng, b, H, G, L, P, N, dt_scale=1.0):
    x = rng_bf16(rng, (b, H, L, P))
    Bm = rng_bf16(rng, (b, G, L, N))
    C = rng_bf16(rng, (b, G, L, N))
    dt = (np.log1p(np.exp(rng.standard_normal((b, H, L)))) * dt_scale).astype(np.float32)
    A = (-np.exp(rng.uniform(0, 1, H))).astype(np.float32)
    return x, dt, A, Bm, C


def _check_prologue(lh, x, dt, A, Bm, C, Q, what):
    dt_v, dA, cb, prev = lh.ssd_prologue(dev(x), devf(dt), devf(A), dev(Bm), dev(C), Q)
    torch.cuda.synchronize()
    dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, Q)
    np.testing.assert_array_equal(dt_v.cpu().numpy(), dt_o)
    dA_g = dA.cpu().numpy()
    assert np.all(np.abs(dA_g - dA_o) <= 1e-5 * (1 + np.abs(dA_o))), f"{what}: dA_cumsum"
    cb_g, cb_r = from_bf16(host(cb)), from_bf16(cb_o)
    bad = np.abs(cb_g - cb_r) > 2.0 ** -7 * np.abs(cb_r) + 1e-5
    assert not bad.any(), (f"{what}: cb {int(bad.sum())} of {bad.size} beyond one bf16 step, max "
                           f"err {float(np.abs(cb_g - cb_r).max()):.3e}")
    # the masked upper triangle is exactly zero
    Qn = cb_r.shape[-1]
    assert not np.any(cb_g[..., np.triu_indices(Qn, 1)[0], np.triu_indices(Qn, 1)[1]])
    prev_g = prev.cpu().numpy()
    scale = 1e-2 * max(float(np.abs(prev_o).max()), 1e-30)
    bad = np.abs(prev_g - prev_o) > 1e-3 * (np.abs(prev_o) + scale)
    assert not bad.any(), (f"{what}: prev_states_T {int(bad.sum())} of {bad.size} off, max err "
                           f"{float(np.abs(prev_g - prev_o).max()):.3e}")
    return dt_v, dA, cb, prev


def test_golden_chain_against_recurrence(lh, golden):
    g = golden("mamba_small")
    Q = int(g["chunk_size"])
    dt_v, dA, cb, prev = _check_prologue(lh, g["x"], g["dt"], g["A"], g["B"], g["C"], Q, "golden")
    out = lh.helion_mamba2_chunk_scan_kernel(cb, dev(g["x"]), dt_v.contiguous(), dA, dev(g["C"]),
                                             devf(g["D"]), prev, tile_m=Q, tile_n=16, tile_k=Q)
    assert_close(from_bf16(host(out)), g["expected"], atol=3e-2, rtol=1e-2,
                 what="GPU prologue + chunk scan vs recurrence")


def test_baseline_chunk_shape(lh):
    """BASELINE per-chunk shape: Q256, P64, N128, G1 (b1, 8 heads, 8 chunks)."""
    rng = np.random.default_rng(41)
    x, dt, A, Bm, C = _raw_inputs(rng, 1, 8, 1, 8 * 256, 64, 128)
    dt_v, dA, cb, prev = _check_prologue(lh, x, dt, A, Bm, C, 256, "baseline shape")
    # and the chain into the chunk scan, against the oracle's own chain
    D = rng.standard_normal(8).astype(np.float32)
    out = lh.helion_mamba2_chunk_scan_kernel(cb, dev(x), dt_v.contiguous(), dA, dev(C), devf(D),
                                             prev, tile_m=256, tile_n=64)
    _, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, 256)
    ref = oracle.mamba_chunk_scan(cb_o, x, dt.reshape(1, 8, 8, 256), dA_o, C, D, prev_o, 64, 64, 64)
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what="baseline chain")


def test_reference_example_shape(lh):
    """The reference example's geometry: Q192, P160, N128, 4 groups (h/8)."""
    rng = np.random.default_rng(42)
    x, dt, A, Bm, C = _raw_inputs(rng, 1, 32, 4, 2 * 192, 160, 128)
    _check_prologue(lh, x, dt, A, Bm, C, 192, "reference shape")


def test_ragged_chunk_and_narrow_state(lh):
    """Q = 48 (zero-filled to the 32-deep MFMA step), N = 32, P = 32, G = 2."""
    rng = np.random.default_rng(43)
    x, dt, A, Bm, C = _raw_inputs(rng, 2, 4, 2, 3 * 48, 32, 32)
    _check_prologue(lh, x, dt, A, Bm, C, 48, "ragged")


@pytest.mark.parametrize("Q,N", [(48, 32), (32, 64), (128, 128)])
def test_paired_k_split_shapes(lh, Q, N):
    """P = 64: two waves per p tile split the k steps.  Q = 48 is one ragged
    unit of two steps, Q = 32 leaves the odd waves without a step (their
    partial sums stay zero), Q = 128 is one full unit per chunk."""
    rng = np.random.default_rng(45 + Q)
    x, dt, A, Bm, C = _raw_inputs(rng, 1, 4, 2, 3 * Q, 64, N)
    _check_prologue(lh, x, dt, A, Bm, C, Q, f"paired Q{Q} N{N}")


@pytest.mark.parametrize("b,H,G,nc,N", [(2, 4, 2, 1, 64), (1, 6, 3, 3, 128)])
def test_wide_unit_shapes(lh, b, H, G, nc, N):
    """P = 64, Q = 256: the state kernel's 256-key form (two stages, one unit
    per chunk).  A single chunk (the pipeline's one-unit case), several
    groups, one and two n blocks."""
    rng = np.random.default_rng(90 + nc)
    x, dt, A, Bm, C = _raw_inputs(rng, b, H, G, nc * 256, 64, N)
    _check_prologue(lh, x, dt, A, Bm, C, 256, f"wide b{b} H{H} G{G} nc{nc} N{N}")


def test_zero_B_gives_zero_states(lh):
    rng = np.random.default_rng(44)
    x, dt, A, Bm, C = _raw_inputs(rng, 1, 2, 1, 4 * 64, 32, 64)
    Bm[:] = 0
    _, _, cb, prev = lh.ssd_prologue(dev(x), devf(dt), devf(A), dev(Bm), dev(C), 64)
    assert not torch.any(cb.view(torch.int16) != 0)
    assert not torch.any(prev != 0)


def _bf16_bits(t):
    """torch fp32 (CPU) -> numpy bf16 bits, round to nearest even."""
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_mamba_baseline_full_config(lh):
    """The BASELINE Mamba-2 config end to end: b4 L4096 h32 P64 N128 g1 Q256
    (16 chunks, 2048 chunk-scan programs, the full XCD remap and the 16-chunk
    state carry of the state-passing kernel).  GPU prologue from seeded raw
    inputs against the oracle's prologue on every (b, c, h); then the GPU
    chunk scan twice: on the GPU prologue's outputs against the oracle's
    chain, and on the oracle's prologue outputs against the oracle's scan
    (isolating the scan).  Every element of every output is compared."""
    b, H, G, Q, nc, P, N = 4, 32, 1, 256, 16, 64, 128
    L = nc * Q
    g = torch.Generator().manual_seed(20240)
    x = _bf16_bits(torch.randn((b, H, L, P), generator=g))
    Bm = _bf16_bits(torch.randn((b, G, L, N), generator=g))
    C = _bf16_bits(torch.randn((b, G, L, N), generator=g))
    dt = torch.nn.functional.softplus(torch.randn((b, H, L), generator=g)).numpy()
    A = (-torch.exp(torch.rand(H, generator=g))).numpy()
    D = torch.randn(H, generator=g).numpy()
    print("mamba full config: inputs ready", flush=True)
    dt_v, dA, cb, prev = _check_prologue(lh, x, dt, A, Bm, C, Q, "full config")
    print("mamba full config: prologue ok", flush=True)
    D_d = devf(D)
    out = lh.helion_mamba2_chunk_scan_kernel(cb, dev(x), dt_v.contiguous(), dA, dev(C), D_d, prev,
                                             tile_m=256, tile_n=64)
    dt_o, dA_o, cb_o, prev_o = oracle.mamba_prologue(x, dt, A, Bm, C, Q)
    ref = oracle.mamba_chunk_scan(cb_o, x, dt_o, dA_o, C, D, prev_o, 64, 64, 64)
    assert_close(from_bf16(host(out)), from_bf16(ref), **ATTN_TOL, what="full config chain")
    out2 = lh.helion_mamba2_chunk_scan_kernel(dev(cb_o), dev(x), devf(dt_o), devf(dA_o), dev(C),
                                              D_d, devf(prev_o), tile_m=256, tile_n=64)
    got2 = host(out2)
    assert_close(from_bf16(got2), from_bf16(ref), **ATTN_TOL, what="full config scan")
    # run to run: the same inputs give the same bits
    out3 = lh.helion_mamba2_chunk_scan_kernel(dev(cb_o), dev(x), devf(dt_o), devf(dA_o), dev(C),
                                              D_d, devf(prev_o), tile_m=256, tile_n=64)
    assert np.array_equal(host(out3), got2), "chunk scan not deterministic"
    _, dA2, cb2, prev2 = lh.ssd_prologue(dev(x), devf(dt), devf(A), dev(Bm), dev(C), Q)
    assert torch.equal(dA2, dA) and torch.equal(cb2.view(torch.int16), cb.view(torch.int16)) \
        and torch.equal(prev2, prev), "SSD prologue not deterministic"


# (b, H, G, Q, nc, P, N, 16-bit type)
STAGE_SHAPES = [
    (2, 4, 1, 256, 3, 64, 128, torch.bfloat16),    # the BASELINE unit plan, cb over 4 n steps
    (1, 4, 2, 192, 2, 160, 256, torch.bfloat16),   # two groups, cb over 8 n steps
    (1, 2, 1, 176, 2, 128, 96, torch.bfloat16),    # a chunk the wave cumsum covers in 3 per lane
    (1, 4, 2, 192, 2, 160, 128, torch.float16),
]


@pytest.mark.parametrize("b,H,G,Q,nc,P,N,ty", STAGE_SHAPES)
def test_stage_entry_points_match_prologue(lh, b, H, G, Q, nc, P, N, ty):
    """The prologue runs the cumsum rows and the cb tiles in one launch; the
    standalone stage entry points (loom_hip_ssd_chunk_cumsum,
    loom_hip_ssd_bmm_chunk, loom_hip_ssd_chunk_state_passing), called one
    after another, give the same bits for all three outputs (the prologue's
    outputs are checked against the oracle above)."""
    import ctypes
    print(f"ssd stages b{b} H{H} G{G} Q{Q} c{nc} P{P} N{N} {ty}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(b * 1000 + H * 10 + Q + N)
    L = nc * Q
    x = torch.randn(b, H, L, P, device="cuda", generator=g).to(ty)
    Bm = torch.randn(b, G, L, N, device="cuda", generator=g).to(ty)
    C = torch.randn(b, G, L, N, device="cuda", generator=g).to(ty)
    dt = torch.nn.functional.softplus(torch.randn(b, H, L, device="cuda", generator=g))
    A = -torch.exp(torch.rand(H, device="cuda", generator=g))
    _, dA, cb, prev = lh.ssd_prologue(x, dt, A, Bm, C, Q)
    dA2, cb2, prev2 = torch.empty_like(dA), torch.empty_like(cb), torch.empty_like(prev)
    for t in (dA2, prev2):
        t.fill_(float("nan"))
    cb2.fill_(float("nan"))
    sfx = "_f16" if ty == torch.float16 else ""
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call(name, *args):
        buf = ctypes.create_string_buffer(256)
        rc = getattr(lh._lib, name)(*args, st, buf, len(buf))
        assert rc == 0, (name, rc, buf.value.decode())

    call("loom_hip_ssd_chunk_cumsum", p(dt), p(A), p(dA2), b, nc, H, Q)
    call("loom_hip_ssd_bmm_chunk" + sfx, p(Bm), p(C), p(cb2), b, nc, G, Q, N)
    call("loom_hip_ssd_chunk_state_passing" + sfx, p(x), p(dt), p(dA2), p(Bm), p(prev2), b, nc, H,
         G, Q, P, N)
    torch.cuda.synchronize()
    assert torch.equal(dA.view(torch.int32), dA2.view(torch.int32)), "dA_cumsum"
    assert torch.equal(cb.view(torch.int16), cb2.view(torch.int16)), "cb"
    assert torch.equal(prev.view(torch.int32), prev2.view(torch.int32)), "prev_states_T"
