"""Re-entrancy: the library holds no per-call state (the CU count it caches
is an atomic, validation flags are thread-local, workspaces belong to the
caller), so calls from several host threads, each on its own stream with
its own buffers, run concurrently and give the same bits as the same calls
made one after another.  ctypes releases the GIL around each call, so the
threads really enter the library together.

flash_decode_noalloc is left out: its calls share the device's static
scratch, and overlapping calls on one GPU race by contract.
"""
import threading

import pytest
import torch

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 6


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


def _bf(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def _work(lh, seed):
    """One thread's inputs, outputs and the calls that fill the outputs."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x, y = _bf(g, 384, 512, std=0.1), _bf(g, 512, 320, std=0.1)
    mm = torch.empty(384, 320, dtype=torch.bfloat16, device="cuda")
    a, b = _bf(g, 4, 512, 256, std=0.1), _bf(g, 4, 256, 512, std=0.1)
    bmm = torch.empty(4, 512, 512, dtype=torch.bfloat16, device="cuda")
    sa, sb = _bf(g, 256, 4096, std=0.1), _bf(g, 4096, 256, std=0.1)
    sk = torch.empty(256, 256, dtype=torch.bfloat16, device="cuda")
    parts = torch.empty(4, 256, 256, dtype=torch.float32, device="cuda")
    k, v, q = _bf(g, 4, 128, 1000), _bf(g, 4, 1000, 128), _bf(g, 4, 1000, 128)
    att = torch.empty(4, 1000, 128, dtype=torch.bfloat16, device="cuda")
    dk, dv, dq = _bf(g, 4, 128, 4096), _bf(g, 4, 4096, 128), _bf(g, 4, 40, 128)
    dec = torch.empty(4, 40, 128, dtype=torch.bfloat16, device="cuda")
    ws = lh.flash_decode_workspace(4, 40, 128, 4096, 512, "cuda")
    bb, H, Q, nc, P, N = 1, 4, 256, 2, 64, 128
    L = nc * Q
    mx, mB, mC = _bf(g, bb, H, L, P), _bf(g, bb, 1, L, N), _bf(g, bb, 1, L, N)
    dt = torch.nn.functional.softplus(torch.randn(bb, H, L, generator=g, device="cuda"))
    A = -torch.exp(torch.rand(H, generator=g, device="cuda"))
    Dh = torch.randn(H, generator=g, device="cuda")
    dA = torch.empty(bb, H, nc, Q, dtype=torch.float32, device="cuda")
    cb = torch.empty(bb, nc, 1, Q, Q, dtype=torch.bfloat16, device="cuda")
    prev = torch.empty(bb, nc, H, N, P, dtype=torch.float32, device="cuda")
    scan = torch.empty(bb, H, L, P, dtype=torch.bfloat16, device="cuda")

    def run():
        lh.matmul(x, y, mm)
        lh.batch_matmul(a, b, bmm, tile_m=256, tile_n=256)
        lh.split_k_matmul_gather(sa, sb, sk, parts, tile_m=128, tile_n=128, tile_k=1024)
        lh.attention(k, v, q, att, causal=True)
        lh.flash_decode(dk, dv, dq, dec, ws, tile_s=512)
        lh.ssd_prologue(mx, dt, A, mB, mC, Q, dA_cumsum=dA, cb=cb, prev_states_T=prev)
        lh.helion_mamba2_chunk_scan_kernel(cb, mx, dt.view(bb, H, nc, Q), dA, mC, Dh, prev, scan,
                                           tile_m=256, tile_n=64)
    return run, [mm, bmm, sk, parts, att, dec, dA, cb, prev, scan]


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def test_threads_on_their_own_streams_match_serial_calls(lh):
    works = [_work(lh, 900 + i) for i in range(THREADS)]
    # serial reference: each thread's calls on the default stream, one after another
    refs = []
    for run, outs in works:
        run()
        torch.cuda.synchronize()
        refs.append([o.clone() for o in outs])
    for _, outs in works:
        for o in outs:
            o.fill_(float("nan")) if o.is_floating_point() else o.zero_()
    torch.cuda.synchronize()

    errors = []
    start = threading.Barrier(THREADS)

    def worker(i):
        try:
            run, _ = works[i]
            s = torch.cuda.Stream()
            start.wait()
            with torch.cuda.stream(s):
                for _ in range(ROUNDS):
                    run()
            s.synchronize()
        except Exception as e:  # reported below; a thread's exception is otherwise lost
            errors.append((i, repr(e)))

    print(f"concurrency: {THREADS} threads x {ROUNDS} rounds", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    names = ["matmul", "batch_matmul", "split_k out", "split_k partials", "attention",
             "flash_decode", "dA_cumsum", "cb", "prev_states_T", "chunk scan"]
    for i, ((_, outs), ref) in enumerate(zip(works, refs)):
        for name, o, r in zip(names, outs, ref):
            assert torch.equal(_bits(o), _bits(r)), f"thread {i}: {name} differs from the serial call"
