"""Every entry point captured in a HIP graph (torch.cuda.CUDAGraph: the
library launches on torch's current stream, which capture redirects) and
replayed three times.  Between replays the outputs are overwritten with NaN
and unrelated eager work runs, and each replay must reproduce the eager
call's outputs bit for bit: a launch that captured a stale pointer, a
memory set or a host-side value would show here.  The library records no
memory-set or copy node (its entry points only launch kernels)."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _replay_matches(name, run, outs):
    """run(): the call writing into `outs`; compares 3 graph replays with the
    eager result."""
    print(f"graph: {name}", flush=True)
    run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    side = torch.randn(1 << 20, device="cuda")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        run()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        side.mul_(1.0001).add_(0.5)             # unrelated eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(_bits(o), _bits(r)), f"{name}: replay {rep} differs from eager"


def _bf(*shape, std=1.0):
    return (torch.randn(*shape, device="cuda") * std).to(torch.bfloat16)


def test_gemms(lh):
    torch.manual_seed(11)
    x, y = _bf(320, 256, std=0.1), _bf(256, 448, std=0.1)
    for t in (64, 128, 256):
        out = torch.empty(320, 448, dtype=torch.bfloat16, device="cuda")
        _replay_matches(f"matmul {t}", lambda: lh.matmul(x, y, out, tile_m=t, tile_n=t), [out])
    # persistent batch_matmul: 8 x 2048^2 output = 512 tiles of 256^2
    a, b = _bf(8, 2048, 256, std=0.1), _bf(8, 256, 2048, std=0.1)
    c = torch.empty(8, 2048, 2048, dtype=torch.bfloat16, device="cuda")
    _replay_matches("batch_matmul persistent",
                    lambda: lh.batch_matmul(a, b, c, tile_m=256, tile_n=256), [c])
    a, b = _bf(256, 4096, std=0.1), _bf(4096, 256, std=0.1)
    out = torch.empty(256, 256, dtype=torch.bfloat16, device="cuda")
    parts = torch.empty(4, 256, 256, dtype=torch.float32, device="cuda")
    _replay_matches("split_k", lambda: lh.split_k_matmul_gather(a, b, out, parts, tile_m=128,
                                                                tile_n=128, tile_k=1024),
                    [out, parts])


def test_attention_and_decode(lh):
    torch.manual_seed(12)
    BH, S, D = 6, 1024, 128
    k, v, q = _bf(BH, D, S), _bf(BH, S, D), _bf(BH, S, D)
    for causal in (False, True):
        out = torch.empty(BH, S, D, dtype=torch.bfloat16, device="cuda")
        _replay_matches(f"attention causal={causal}",
                        lambda: lh.attention(k, v, q, out, causal=causal, tile_m=256, tile_n=64),
                        [out])
    B, H, S = 4, 32, 4096
    k, v, q = _bf(B, D, S), _bf(B, S, D), _bf(B, H, D)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device="cuda")
    ws = lh.flash_decode_workspace(B, H, D, S, 512, "cuda")
    _replay_matches("flash_decode", lambda: lh.flash_decode(k, v, q, out, ws, tile_s=512,
                                                            tile_n=128), [out])
    out2 = torch.empty(B, H, D, dtype=torch.bfloat16, device="cuda")
    _replay_matches("flash_decode_noalloc",
                    lambda: lh.flash_decode_noalloc(k, v, q, out2, tile_s=512, tile_n=128), [out2])


def test_attention_and_decode_other_paths(lh):
    """The kernels picked away from the common shapes: attention at head dim
    256 and at head dim 96 with a key count not a multiple of 8 (K staged
    through registers), decode with 64 heads per workgroup (H 48), with
    ragged S on the LDS-DMA kernel (H 48, S 1001) and on the register kernel
    (H 8, S 1001), and at head dim 200."""
    torch.manual_seed(14)
    for BH, Sq, Skv, D, causal in ((2, 300, 300, 256, True), (2, 190, 517, 96, False)):
        k, v, q = _bf(BH, D, Skv), _bf(BH, Skv, D), _bf(BH, Sq, D)
        out = torch.empty(BH, Sq, D, dtype=torch.bfloat16, device="cuda")
        _replay_matches(f"attention D{D} Skv{Skv}",
                        lambda: lh.attention(k, v, q, out, causal=causal, tile_m=128), [out])
    for B, H, D, S, ts in ((2, 48, 128, 4096, 512), (2, 48, 128, 1001, 256),
                           (2, 8, 64, 1001, 128), (3, 16, 200, 777, 256)):
        k, v, q = _bf(B, D, S), _bf(B, S, D), _bf(B, H, D)
        out = torch.empty(B, H, D, dtype=torch.bfloat16, device="cuda")
        ws = lh.flash_decode_workspace(B, H, D, S, ts, "cuda")
        _replay_matches(f"flash_decode B{B} H{H} D{D} S{S}",
                        lambda: lh.flash_decode(k, v, q, out, ws, tile_s=ts), [out])


def test_mamba(lh):
    torch.manual_seed(13)
    b, H, nc, Q, P, N = 2, 8, 4, 256, 64, 128
    L = nc * Q
    x, C = _bf(b, H, L, P), _bf(b, 1, L, N)
    Bm = _bf(b, 1, L, N)
    dt = torch.nn.functional.softplus(torch.randn(b, H, L, device="cuda"))
    A = -torch.exp(torch.rand(H, device="cuda"))
    Dh = torch.randn(H, device="cuda")
    dA = torch.empty(b, H, nc, Q, dtype=torch.float32, device="cuda")
    cb = torch.empty(b, nc, 1, Q, Q, dtype=torch.bfloat16, device="cuda")
    prev = torch.empty(b, nc, H, N, P, dtype=torch.float32, device="cuda")
    _replay_matches("ssd_prologue", lambda: lh.ssd_prologue(x, dt, A, Bm, C, Q, dA_cumsum=dA,
                                                            cb=cb, prev_states_T=prev),
                    [dA, cb, prev])
    dt4 = dt.view(b, H, nc, Q)
    for tm, tn in ((256, 64), (64, 16)):          # 8-wave and 4-wave workgroups
        out = torch.empty(b, H, L, P, dtype=torch.bfloat16, device="cuda")
        _replay_matches(f"chunk scan {tm}x{tn}",
                        lambda: lh.helion_mamba2_chunk_scan_kernel(
                            cb, x, dt4, dA, C, Dh, prev, out, tile_m=tm, tile_n=tn, tile_k=64),
                        [out])


def test_synth(lh):
    out = {}

    def run():
        out["t"] = lh.synth((1 << 20,), 99, "normal", 0.0, 1.0)
    run()
    torch.cuda.synchronize()
    ref = out["t"].clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    t = out["t"]
    for _ in range(3):
        t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(t), _bits(ref))
