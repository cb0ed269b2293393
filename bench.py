#!/usr/bin/env python3
"""Throughput of the loom_hip kernels on one MI355X.

The headline line (one JSON object on stdout) measures @batch_matmul at the
BASELINE configuration B16 x 2048^3 (bf16 in, fp32 accumulate): K timed steps
of one call each, inputs resident in HBM.  It carries

  roofline      the GEMM kernel's achieved TFLOP/s (algorithmic 2*B*M*N*K per
                launch / mean launch time from HIP events on the launch
                stream) against the dense bf16 MFMA peak;
  cpu_baseline  the fp32 C oracle (OpenMP, all host threads) on a bounded
                sample of the same batches;
  kernels       every BASELINE configuration (mm, bmm, split-K, flashattn,
                mqa_decode, mamba_chunk_scan, SSD prologue): mean GPU time of
                calls enqueued back to back (`ms`), and of the same calls
                replayed from a HIP graph (`ms_graph`: no host work between
                the kernels, which a few-microsecond kernel otherwise waits
                on; used for the rates once the replay's outputs matched an
                eager call bit for bit), each call on a different copy of
                its inputs so operands never stay in the 256 MB Infinity Cache
                between calls, with its roofline fraction, the dominant
                kernel's HBM bytes per launch from the committed counter
                summaries (profiles/hbm_traffic.json), and the CPU oracle on a
                stated slice of the same configuration (measured, then scaled
                to the whole; cores and GPU/CPU speed-up stated);
  ceilings      what this part sustains (HBM read over 2 GiB and over one
                cache-flushed 134.7 MB pass; bf16 MFMA chains), next to the
                published peaks the fractions use.

Before timing, each measurement runs its own call untimed for --settle-ms of
GPU time (clocks take on the order of 100 ms of load to settle).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--no-ceilings] [--kernels all|none|mm,bmm,...]
       python bench.py --profile-workload all|mm,bmm,...   (for rocprofv3 --pmc)
       python bench.py --library-baselines   (PyTorch / hipBLASLt / SDPA on the same shapes)
       python bench.py --reference-signatures   (each example at the reference's f16 shapes)
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "loom-dataflow_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")
SEED_BASE = 0x5EED0000      # seed of the first synthetic input tensor


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="untimed GPU work before each measurement (clocks and power settle)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the on-box HBM and MFMA ceiling measurement")
    ap.add_argument("--kernels", default="all", help="per-kernel table: all, none or a list")
    ap.add_argument("--iters", type=int, default=20, help="timed calls per kernel in the table")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the workload profiled for roofline.traffic: a 256 MiB "
                         "device copy (the calibration kernel), three headline bmm launches "
                         "and three split-K launches (cache flushed before each)")
    ap.add_argument("--profile-workload", default=None,
                    help="only run the workload a counter profile attributes: the 256 MiB "
                         "calibration copy, then three calls of each listed kernel (comma "
                         "list of the table's names, or 'all'), the Infinity Cache flushed "
                         "by a read-only pass before each call")
    ap.add_argument("--library-baselines", action="store_true",
                    help="only time the libraries of this image on the table's shapes: "
                         "torch.matmul / torch.bmm (hipBLASLt) for mm, bmm and the split-K "
                         "shape, scaled_dot_product_attention for flashattn (causal) and "
                         "mqa_decode (enable_gqa, one KV head); one JSON line")
    ap.add_argument("--reference-signatures", action="store_true",
                    help="only time each example at the reference's own f16 signature "
                         "(and emitted bindings); one JSON line")
    return ap.parse_args()


def library_baselines(torch, iters=30):
    """The same shapes through the libraries this image ships (no counterpart
    exists for the Mamba-2 kernels): a reference point for each kernel, not a
    parity check."""
    import torch.nn.functional as F
    bf = torch.bfloat16
    g = torch.Generator(device="cuda")
    g.manual_seed(7)

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device="cuda") * std).to(bf)

    def timed(fn):
        settle(torch, lambda i: fn(), 100)
        return time_back_to_back(torch, lambda i: fn(), iters)

    out = {}
    a, b = randn(1024, 1024), randn(1024, 1024)
    ms = timed(lambda: torch.matmul(a, b))
    out["mm"] = {"library": "torch.matmul (hipBLASLt)", "ms": round(ms, 5),
                 "tflops": round(2 * 1024 ** 3 / ms / 1e9, 2)}
    a, b = randn(16, 2048, 2048, std=0.02), randn(16, 2048, 2048, std=0.02)
    ms = timed(lambda: torch.bmm(a, b))
    out["bmm"] = {"library": "torch.bmm (hipBLASLt)", "ms": round(ms, 5),
                  "tflops": round(16 * 2 * 2048 ** 3 / ms / 1e9, 2)}
    a, b = randn(512, 16384, std=0.02), randn(16384, 512, std=0.02)
    ms = timed(lambda: torch.matmul(a, b))
    out["split_k"] = {"library": "torch.matmul (hipBLASLt), same product", "ms": round(ms, 5),
                      "tflops": round(2 * 512 * 512 * 16384 / ms / 1e9, 2)}
    del a, b
    B, H, S, D = 4, 32, 4096, 128
    q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.FLASH_ATTENTION):
        ms = timed(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True))
    out["flashattn"] = {"library": "scaled_dot_product_attention, flash backend, causal",
                        "ms": round(ms, 5), "tflops": round(2 * B * H * S * S * D / ms / 1e9, 2)}
    del q, k, v
    Bd, Hd, Sd = 32, 32, 8192
    qd, kd, vd = randn(Bd, Hd, 1, D), randn(Bd, 1, Sd, D), randn(Bd, 1, Sd, D)
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.FLASH_ATTENTION):
        ms = timed(lambda: F.scaled_dot_product_attention(qd, kd, vd, enable_gqa=True))
    out["mqa_decode"] = {"library": "scaled_dot_product_attention, flash backend, enable_gqa",
                         "ms": round(ms, 5), "gbs": round(2 * Bd * Sd * D * 2 / ms / 1e6, 1)}
    out["mamba_chunk_scan"] = out["mamba_prologue"] = None   # no library implementation here
    return out


def reference_signatures(torch, lh, iters=20):
    """Each example at the reference's own f16 signature (SURVEY A.1's left
    column: examples/*/IR/00_from_helion_frontend.mlir), split-K and mqa at
    the bindings the reference emitted (tile_k512 tile_m64 tile_n32;
    tile_s512 tile_n512), timed as the kernel table's ms_graph (replayed
    calls, checked bit-identical to an eager call).  One set of inputs per
    case, so operands that fit stay cache resident."""
    h = torch.float16
    g = torch.Generator(device="cuda")
    g.manual_seed(11)

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device="cuda") * std).to(h)

    def run(name, fn, work, unit):
        case = {"fn": fn}
        settle(torch, fn, 50)
        ms = graph_ms(torch, case, iters) or time_back_to_back(torch, fn, iters)
        rate = work / ms / 1e9 if unit == "TFLOP/s" else work / ms / 1e6
        return {name: {"ms": round(ms, 5), "tflops" if unit == "TFLOP/s" else "gbs": round(rate, 1)}}

    out = {}
    x, y = rn(2048, 256), rn(256, 256)
    mo = torch.empty(2048, 256, dtype=h, device="cuda")
    out.update(run("mm 2048x256 . 256x256", lambda i: lh.matmul(x, y, mo), 2 * 2048 * 256 * 256,
                   "TFLOP/s"))
    a, b = rn(8, 4096, 512, std=0.05), rn(8, 512, 4096, std=0.05)
    bo = torch.empty(8, 4096, 4096, dtype=h, device="cuda")
    out.update(run("bmm 8x4096x512 . 8x512x4096", lambda i: lh.batch_matmul(a, b, bo),
                   2 * 8 * 4096 * 4096 * 512, "TFLOP/s"))
    del a, b, bo
    sa, sb = rn(512, 4096, std=0.05), rn(4096, 512, std=0.05)
    so = torch.empty(512, 512, dtype=h, device="cuda")
    sg = torch.empty(8, 512, 512, dtype=torch.float32, device="cuda")
    out.update(run("split-K 512x4096 . 4096x512, tile_k512 tile_m64 tile_n32",
                   lambda i: lh.split_k_matmul_gather(sa, sb, so, sg, tile_m=64, tile_n=32,
                                                      tile_k=512),
                   2 * (512 * 4096 * 2) + 2 * (8 * 512 * 512 * 4) + 512 * 512 * 2, "GB/s"))
    k, v, q = rn(32, 128, 4096), rn(32, 4096, 128), rn(32, 4096, 128)
    ao = torch.empty(32, 4096, 128, dtype=h, device="cuda")
    out.update(run("flashattn BH32 S4096 D128, non-causal",
                   lambda i: lh.attention(k, v, q, ao, scale=0.08837890625, causal=False),
                   4 * 32 * 4096 * 4096 * 128, "TFLOP/s"))
    del k, v, q, ao
    kd, vd, qd = rn(16, 128, 8192), rn(16, 8192, 128), rn(16, 32, 128)
    do = torch.empty(16, 32, 128, dtype=h, device="cuda")
    ws = lh.flash_decode_workspace(16, 32, 128, 8192, 512, "cuda")
    out.update(run("mqa B16 H32 D128 S8192, tile_s512 tile_n512",
                   lambda i: lh.flash_decode(kd, vd, qd, do, ws, scale=0.08837890625, tile_s=512,
                                             tile_n=512),
                   2 * 16 * 8192 * 128 * 2 + 16 * 32 * 128 * 4, "GB/s"))
    b_, H, G, nc, Q, P, N = 2, 32, 4, 8, 192, 160, 128
    L = nc * Q
    cb, xm, C = rn(b_, nc, G, Q, Q, std=0.1), rn(b_, H, L, P), rn(b_, G, L, N, std=0.1)
    dt = (torch.rand(b_, H, nc, Q, generator=g, device="cuda") * 0.1).to(h)
    dA = (-(torch.rand(b_, H, nc, Q, generator=g, device="cuda") * 0.05).cumsum(-1)).to(h)
    Dh, pv = rn(H), rn(b_, nc, H, N, P, std=0.1)
    mo2 = torch.empty(b_, H, L, P, dtype=h, device="cuda")
    byts = 2 * sum(t.numel() for t in (cb, xm, dt, dA, C, pv, mo2))
    out.update(run("mamba chunk scan b2 L1536 h32 P160 N128 g4 Q192",
                   lambda i: lh.helion_mamba2_chunk_scan_kernel(cb, xm, dt, dA, C, Dh, pv, mo2,
                                                                tile_m=192, tile_n=64),
                   byts, "GB/s"))
    return out


def traffic_for(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    if a measurement has been recorded for this kernel."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(kernel)
    except (OSError, ValueError):
        return None


MALL_BYTES = 256 << 20       # MI355X Infinity Cache


def median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


def settle(torch, fn, ms):
    """Run fn(i) back to back, untimed, until about `ms` of GPU time has
    passed: MI355X clocks take on the order of 100 ms of sustained load to
    settle, and a measurement started cold reads up to 20% slow."""
    if ms <= 0:
        return
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    done, i = 0.0, 0
    while done < ms and i < 100000:
        a.record(s)
        for _ in range(8):
            fn(i)
            i += 1
        b.record(s)
        torch.cuda.synchronize()
        done += a.elapsed_time(b)


def time_back_to_back(torch, fn, iters):
    """Mean GPU time (ms) of `iters` calls enqueued back to back, from one
    pair of HIP events on the current stream (the stream the library launches
    on).  fn(i) is the i-th call."""
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(s)
    for i in range(iters):
        fn(i)
    b.record(s)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def per_call_ms(torch, fn, iters):
    """GPU time (ms) of each of `iters` back-to-back calls, from a HIP event
    recorded between consecutive calls on the launch stream (a marker in the
    stream: the calls still run back to back)."""
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
    torch.cuda.synchronize()
    ev[0].record(s)
    for i in range(iters):
        fn(i)
        ev[i + 1].record(s)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(iters)]


def _tensors(r):
    if r is None:
        return []
    if isinstance(r, (tuple, list)):
        return [t for x in r for t in _tensors(x)]
    return [r] if hasattr(r, "data_ptr") else []


def graph_ms(torch, case, iters, reps=5):
    """Mean GPU time (ms) per call of `iters` calls captured once in a HIP
    graph and replayed: the kernels of the same calls back to back without
    the host's per-call work between them (argument checks, ctypes, launch),
    which for kernels of a few microseconds takes longer than the kernel.
    Used only if the replayed outputs of the last call are bit-identical to
    the same call run eagerly afterwards; None otherwise (or if capture
    fails), with the reason on stderr."""
    fn = case["fn"]
    try:
        fn(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            rets = [fn(i) for i in range(iters)]
        g.replay()
        torch.cuda.synchronize()
        last = _tensors(rets[-1]) or _tensors(case.get("out", lambda i: None)(iters - 1))
        if not last:
            raise RuntimeError("no output to check the replay against")
        snap = [t.clone() for t in last]
        eager = _tensors(fn(iters - 1)) or _tensors(case["out"](iters - 1))
        torch.cuda.synchronize()
        if len(eager) != len(snap) or not all(torch.equal(a, b) for a, b in zip(snap, eager)):
            raise RuntimeError("replayed outputs differ from the eager call")
        for _ in range(3):
            g.replay()
        s = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(s)
        for _ in range(reps):
            g.replay()
        b.record(s)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / (reps * iters)
        del g, rets
        return ms
    except Exception as e:   # noqa: BLE001 -- reported, the host-issued figure stands
        print(f"# graph replay not used for {case['desc']}: {e}", file=sys.stderr, flush=True)
        return None


def quantile(xs, q):
    xs = sorted(xs)
    return xs[min(len(xs) - 1, max(0, int(round(q * (len(xs) - 1)))))]


# --------------------------------------------------------------------------
# BASELINE configurations.  Each case holds enough independent copies of its
# inputs that consecutive calls read more than three times the Infinity
# Cache, so a call never finds its operands left in cache by the previous one
# (the mm operands, 6 MB, stay cache resident whatever is done).
# --------------------------------------------------------------------------

def make_cases(torch, lh):
    cuda = "cuda"
    bf, f32 = torch.bfloat16, torch.float32
    # Every input comes from the measurement protocol's counter-based
    # generator (loom_hip.synth: splitmix64, Box-Muller, round to nearest
    # even; bit-identical to the CPU oracle's oracle.synth), one stream per
    # tensor: seed = SEED_BASE + the tensor's index in creation order.
    seed = [SEED_BASE]

    def nxt():
        seed[0] += 1
        return seed[0]

    def randn(*shape, std=1.0, dtype=bf):
        return lh.synth(shape, nxt(), "normal", 0.0, std, dtype)

    def unif(*shape, lo=-1.0, hi=1.0, dtype=bf):
        return lh.synth(shape, nxt(), "uniform", lo, hi, dtype)

    def copies(nbytes):
        return max(1, min(4, -(-3 * MALL_BYTES // nbytes)))

    def h16(t):
        import numpy as np
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def hf(t):
        return t.contiguous().float().cpu().numpy()

    cases = {}

    # mm's operands (6 MB) would stay in the Infinity Cache across calls, so
    # its burst walks 160 copies (960 MB with the outputs, 3.75x the cache):
    # every call reads operands last touched 160 calls earlier, i.e. from
    # HBM; mm_warm repeats one copy (operands cache resident) for reference
    def mm_case(n, what):
        sets = [(unif(1024, 1024), unif(1024, 1024), torch.empty(1024, 1024, dtype=bf, device=cuda))
                for _ in range(n)]
        def cpu():
            import oracle
            hx, hy = h16(sets[0][0]), h16(sets[0][1])
            return 1.0, "the whole 1024^3 product", lambda: oracle.matmul(hx, hy, 128, 128, 64)
        return dict(fn=lambda i: lh.matmul(*sets[i % n], tile_m=64, tile_n=64, tile_k=64),
                    flop=2 * 1024 ** 3, bytes=3 * 1024 * 1024 * 2, bound="mfma", sets=n,
                    iters=max(n, 20), desc=f"mm 1024^3 bf16, tile 64x64 ({what})", cpu=cpu,
                    kernel="gemm_pipe_kernel<64, false, false>")
    cases["mm"] = lambda: mm_case(160, "operands from HBM: 160 rotating copies")
    cases["mm_warm"] = lambda: mm_case(1, "operands cache resident")

    def bmm():
        nb = 3 * 16 * 2048 * 2048 * 2
        n = copies(nb)
        sets, seeds = [], []
        for _ in range(n):
            sa, sb = nxt(), nxt()
            seeds.append((sa, sb))
            sets.append((lh.synth((16, 2048, 2048), sa, "normal", 0.0, 0.02),
                         lh.synth((16, 2048, 2048), sb, "normal", 0.0, 0.02),
                         torch.empty(16, 2048, 2048, dtype=bf, device=cuda)))
        def cpu():
            import oracle
            a0, a1 = h16(sets[0][0][:1]), h16(sets[0][1][:1])
            return 1 / 16, "1 of 16 batches", lambda: oracle.batch_matmul(a0, a1, 1, 256, 256, 64)
        return dict(fn=lambda i: lh.batch_matmul(*sets[i % n], tile_m=256, tile_n=256),
                    flop=2 * 16 * 2048 ** 3, bytes=nb, bound="mfma", sets=n,
                    desc="bmm 16x2048^3 bf16, tile 256x256", cpu=cpu, seeds=seeds[0],
                    kernel="gemm_persist_kernel<false>")
    cases["bmm"] = bmm

    def splitk():
        nb = (512 * 16384 * 2) * 2 + 16 * 512 * 512 * 4 * 2 + 512 * 512 * 2
        n = copies(nb)
        sets = [(randn(512, 16384, std=0.02), randn(16384, 512, std=0.02),
                 torch.empty(512, 512, dtype=bf, device=cuda),
                 torch.empty(16, 512, 512, dtype=torch.float32, device=cuda)) for _ in range(n)]
        def cpu():
            import oracle
            a, b = h16(sets[0][0]), h16(sets[0][1])
            return 1.0, "all 16 slabs and the reduction", \
                lambda: oracle.split_k_matmul_gather(a, b, 128, 128, 1024)
        return dict(fn=lambda i: lh.split_k_matmul_gather(*sets[i % n], tile_m=128, tile_n=128,
                                                          tile_k=1024),
                    flop=2 * 512 * 512 * 16384, bytes=nb, bound="hbm", sets=n,
                    desc="split-K 512x512x16384, 16 slabs, fp32 partials", cpu=cpu,
                    kernel="gemm_pipe_kernel<128, true, false>")
    cases["split_k"] = splitk

    def flashattn():
        BH, S, D = 128, 4096, 128
        nb = 4 * BH * S * D * 2
        n = min(2, copies(nb))
        sets = [(randn(BH, D, S), randn(BH, S, D), randn(BH, S, D),
                 torch.empty(BH, S, D, dtype=bf, device=cuda)) for _ in range(n)]
        def cpu():
            import oracle
            k, v, q = (h16(t[:4]) for t in sets[0][:3])
            return 4 / BH, "4 of 128 (b, h) heads", \
                lambda: oracle.attention(k, v, q, 1 / math.sqrt(D), True, 1, 128, 64)
        return dict(fn=lambda i: lh.attention(*sets[i % n], causal=True, tile_m=256, tile_n=64),
                    flop=4 * BH * S * S * D // 2, bytes=nb, bound="mfma", sets=n,
                    desc="flashattn fwd B4 H32 S4096 D128 causal, tile_m 256", cpu=cpu,
                    kernel="attention_dma_kernel<128, 2, 8, false, false>")
    cases["flashattn"] = flashattn

    def decode():
        B, H, D, S = 32, 32, 128, 8192
        nb = 2 * B * S * D * 2 + 2 * B * H * D * 2
        n = copies(nb)
        sets = [(randn(B, D, S), randn(B, S, D), randn(B, H, D),
                 torch.empty(B, H, D, dtype=bf, device=cuda),
                 lh.flash_decode_workspace(B, H, D, S, 1024, cuda)) for _ in range(n)]
        def cpu():
            import oracle
            k, v, q = (h16(t) for t in sets[0][:3])
            return 1.0, "the whole call (8 splits per batch and the combine)", \
                lambda: oracle.flash_decode(k, v, q, 1 / math.sqrt(D), 1, 1024, 128)
        return dict(fn=lambda i: lh.flash_decode(*sets[i % n], tile_s=1024, tile_n=128),
                    flop=4 * B * H * S * D, bytes=nb, bound="hbm", sets=n,
                    desc="mqa_decode B32 H32/1KV D128 S8192, tile_s 1024", cpu=cpu,
                    kernel="decode_dma_kernel<128, false, false, 4, 0>")
    cases["mqa_decode"] = decode

    def mamba():
        b, L, H, P, N, Q = 4, 4096, 32, 64, 128, 256
        nc = L // Q

        def one():
            x = randn(b, H, L, P)
            C = randn(b, 1, L, N)
            cb = randn(b, nc, 1, Q, Q)
            dt = torch.nn.functional.softplus(randn(b, H, nc, Q, dtype=f32))
            A = -torch.exp(unif(H, lo=0.0, hi=1.0, dtype=f32))
            dA = torch.cumsum(dt * A[None, :, None, None], dim=-1)
            Dh = randn(H, dtype=f32)
            prev = randn(b, nc, H, N, P, dtype=f32)
            out = torch.empty(b, H, L, P, dtype=bf, device=cuda)
            return (cb, x, dt, dA, C, Dh, prev, out)
        first = one()
        nb = sum(t.numel() * t.element_size() for t in first)
        n = copies(nb)
        sets = [first] + [one() for _ in range(n - 1)]
        flop = 2 * b * H * L * N * P + b * H * nc * Q * Q * P + 2 * b * H * L * P

        def cpu():
            import oracle
            cb, x, dt, dA, C, Dh, prev = sets[0][:7]
            a = (h16(cb[:1]), h16(x[:1]), hf(dt[:1]), hf(dA[:1]), h16(C[:1]), hf(Dh), hf(prev[:1]))
            return 1 / b, "batch 1 of 4", lambda: oracle.mamba_chunk_scan(*a, 64, 64, 64)
        return dict(fn=lambda i: lh.helion_mamba2_chunk_scan_kernel(
            *sets[i % n], tile_m=256, tile_n=64, tile_k=64),
            flop=flop, bytes=nb, bound="hbm", sets=n, inputs=sets,
            desc="mamba chunk_scan b4 L4096 h32 P64 N128 g1 Q256", cpu=cpu,
            kernel="mamba_chunk_scan_kernel<4, false, 8, 256, 128>")
    cases["mamba_chunk_scan"] = mamba

    def ssd():
        b, L, H, P, N, Q = 4, 4096, 32, 64, 128, 256
        nc = L // Q

        def one():
            x = randn(b, H, L, P)
            Bm, C = randn(b, 1, L, N), randn(b, 1, L, N)
            dt = torch.nn.functional.softplus(randn(b, H, L, dtype=f32))
            A = -torch.exp(unif(H, lo=0.0, hi=1.0, dtype=f32))
            dA = torch.empty(b, H, nc, Q, dtype=torch.float32, device=cuda)
            cb = torch.empty(b, nc, 1, Q, Q, dtype=bf, device=cuda)
            prev = torch.empty(b, nc, H, N, P, dtype=torch.float32, device=cuda)
            return (x, dt, A, Bm, C, dA, cb, prev)
        first = one()
        nb = sum(t.numel() * t.element_size() for t in first)
        n = copies(nb)
        sets = [first] + [one() for _ in range(n - 1)]

        def fn(i):
            x, dt, A, Bm, C, dA, cb, prev = sets[i % n]
            lh.ssd_prologue(x, dt, A, Bm, C, Q, dA_cumsum=dA, cb=cb, prev_states_T=prev)

        def out(i):
            return sets[i % n][5:]
        flop = b * nc * Q * Q * N + 2 * b * H * L * N * P

        def cpu():
            import oracle
            x, dt, A, Bm, C = sets[0][:5]
            a = (h16(x[:1]), hf(dt[:1]), hf(A), h16(Bm[:1]), h16(C[:1]))
            return 1 / b, "batch 1 of 4", lambda: oracle.mamba_prologue(*a, Q)
        return dict(fn=fn, out=out, flop=flop, bytes=nb, bound="hbm", sets=n,
                    desc="mamba SSD prologue (cumsum, cb, states + passing) b4 L4096 h32 P64 "
                         "N128 g1 Q256", cpu=cpu, kernel="ssd_state_kernel<4, 2, false, true>")
    cases["mamba_prologue"] = ssd
    return cases


def report(case, ms, calls=None, ms_graph=None):
    """`ms`: mean per call from one event pair around a burst of host-issued
    calls; `ms_graph`: the same calls replayed from a HIP graph (no host work
    between kernels); the rates use ms_graph where it was measured, else ms;
    `calls`: per-call times of a host-issued burst, summarised as median /
    p10 / p90."""
    s = (ms_graph if ms_graph else ms) / 1e3
    tflops = case["flop"] / s / 1e12
    gbs = case["bytes"] / s / 1e9
    if case["bound"] == "mfma":
        frac = tflops / PEAK_BF16_TFLOPS
    else:
        frac = gbs / PEAK_HBM_GBS
    out = {"desc": case["desc"], "ms": round(ms, 5),
           "ms_graph": round(ms_graph, 5) if ms_graph else None, "tflops": round(tflops, 2),
           "gbs": round(gbs, 1), "bound": case["bound"], "roofline_frac": round(frac, 4),
           "input_copies": case["sets"]}
    if calls:
        out["ms_median"] = round(median(calls), 5)
        out["ms_p10"] = round(quantile(calls, 0.1), 5)
        out["ms_p90"] = round(quantile(calls, 0.9), 5)
    kern = case.get("kernel")
    if kern:
        out["kernel"] = kern
        t = traffic_for(kern)
        # HBM bytes per launch of the dominant kernel, from the committed
        # rocprofv3 counter summaries (null where none is recorded)
        out["traffic"] = t
    return out


def cpu_column(case, gpu_ms, reps=5, max_run_s=4.0):
    """The fp32 C oracle (OpenMP, all host threads) on a stated slice of the
    same configuration: median of `reps` runs after one warm-up (a single run
    when one takes longer than `max_run_s`), scaled to the whole
    configuration."""
    import oracle
    frac, what, run = case["cpu"]()
    t0 = time.perf_counter()
    run()                      # warm-up (page-in, thread pool)
    first = time.perf_counter() - t0
    times = [first]
    if first < max_run_s:
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
    slice_s = median(times)
    full_s = slice_s / frac
    out = {"slice": what, "slice_ms": round(slice_s * 1e3, 3), "ms": round(full_s * 1e3, 3),
           "extrapolated": frac < 1.0, "cores": oracle.num_threads(), "kind": "port",
           "speedup": round(full_s * 1e3 / gpu_ms, 1)}
    if case["bound"] == "mfma":
        out["tflops"] = round(case["flop"] / full_s / 1e12, 4)
    else:
        out["gbs"] = round(case["bytes"] / full_s / 1e9, 2)
    return out


def measure_ceilings(torch, lh):
    """What this part sustains: HBM read rate over 2 GiB (sustained) and over
    one 134.7 MB pass after an Infinity Cache flush (the decode working set),
    and the bf16 MFMA rate of independent chains.  Reported next to the
    published peaks; the roofline fractions keep the published peaks."""
    sink = torch.zeros(64, dtype=torch.float32, device="cuda")
    big = torch.ones(1 << 29, dtype=torch.float32, device="cuda")   # 2 GiB
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, reps):
        best = float("inf")
        for _ in range(reps):
            fn(None)
            torch.cuda.synchronize()
            a.record(s)
            fn(True)
            b.record(s)
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b))
        return best
    settle(torch, lambda i: lh.peak_hbm_read(big, sink), 100)
    ms_big = timed(lambda t: lh.peak_hbm_read(big, sink), 5)
    nb = 134742016
    part = big.view(torch.uint8)[:nb]
    flush = big.view(torch.uint8)[nb:nb + (1 << 30)]
    # the flush is a read of 1 GiB elsewhere: clean lines, no write-back
    ms_pass = timed(lambda t: lh.peak_hbm_read(part if t else flush, sink), 10)
    iters = 20000
    flop = lh.peak_mfma_bf16(iters, sink)
    settle(torch, lambda i: lh.peak_mfma_bf16(iters, sink), 100)
    ms_mfma = timed(lambda t: lh.peak_mfma_bf16(iters, sink), 5)
    del big
    torch.cuda.empty_cache()
    return {"hbm_read_gbs_2GiB": round((1 << 31) / ms_big / 1e6, 1),
            "hbm_read_gbs_134MB_pass": round(nb / ms_pass / 1e6, 1),
            "hbm_read_us_134MB_pass": round(ms_pass * 1e3, 2),
            "mfma_bf16_tflops": round(flop / ms_mfma / 1e9, 1),
            "published_hbm_gbs": PEAK_HBM_GBS, "published_bf16_tflops": PEAK_BF16_TFLOPS,
            "how": "best of several single kernel runs after settling: a 16-byte streaming "
                   "read (one workgroup of 512 per CU, 4 loads in flight per thread); "
                   "independent 16x16x32 bf16 MFMA chains, 8 per wave, 2 waves per SIMD"}


def cpu_baseline(seeds, budget_s=12.0):
    """The fp32 C oracle on whole batches of the same workload until the time
    budget is spent (at least one batch).  Its operands are the headline's
    first input set, made on the host by the oracle's copy of the
    counter-based generator from the same seeds (bit-identical to the GPU's)."""
    import oracle
    h0 = oracle.synth((16, 2048, 2048), seeds[0], "normal", 0.0, 0.02)
    h1 = oracle.synth((16, 2048, 2048), seeds[1], "normal", 0.0, 0.02)
    B, M, K = h0.shape
    N = h1.shape[2]
    done, t0 = 0, time.perf_counter()
    while done < B:
        oracle.batch_matmul(h0[done:done + 1], h1[done:done + 1], 1, 256, 256, 64)
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    return {"value": round(2 * done * M * N * K / el / 1e12, 4), "unit": "TFLOP/s",
            "cores": oracle.num_threads(), "kind": "port",
            "sample": f"{done} of {B} batches of {M}x{N}x{K} (fp32 oracle, OpenMP), "
                      f"{el:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the kernels are single-GPU; "
              "multi-GPU sharding is a design note), so --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import loom_hip as lh

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    torch.cuda.set_device(0)
    print(f"# device: {torch.cuda.get_device_name(0)}; {lh.__version__}", file=sys.stderr,
          flush=True)

    if args.reference_signatures:
        print(json.dumps({"reference_signatures": reference_signatures(torch, lh),
                          "dtype": "f16", "device": torch.cuda.get_device_name(0)}), flush=True)
        return

    if args.library_baselines:
        print(json.dumps({"library_baselines": library_baselines(torch),
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return

    if args.traffic_probe:
        # profiled under rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE: the copy
        # reads and writes exactly 256 MiB, which calibrates both counters
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        a0 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
        a1 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
        out = torch.empty(16, 2048, 2048, dtype=torch.bfloat16, device="cuda")
        for _ in range(3):
            lh.batch_matmul(a0, a1, out, tile_m=256, tile_n=256)
        del a0, a1, out
        sa = (torch.randn(512, 16384, device="cuda") * 0.02).to(torch.bfloat16)
        sb = (torch.randn(16384, 512, device="cuda") * 0.02).to(torch.bfloat16)
        so = torch.empty(512, 512, dtype=torch.bfloat16, device="cuda")
        sg = torch.empty(16, 512, 512, dtype=torch.float32, device="cuda")
        flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
        for _ in range(3):
            flush.zero_()  # larger than the Infinity Cache: operands come from HBM
            lh.split_k_matmul_gather(sa, sb, so, sg, tile_m=128, tile_n=128, tile_k=1024)
        torch.cuda.synchronize()
        print("traffic probe done", file=sys.stderr, flush=True)
        return

    if args.profile_workload:
        # counter runs (rocprofv3 --pmc): the calibration copy, then three
        # calls of each kernel, each after a read-only pass over 1 GiB that
        # evicts the Infinity Cache without leaving dirty lines
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        flush = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        sink = torch.zeros(64, dtype=torch.float32, device="cuda")
        # calibration of the MFMA-busy counter: independent MFMA chains, whose
        # rate bench.py's ceilings measure
        lh.peak_mfma_bf16(20000, sink)
        torch.cuda.synchronize()
        cases = make_cases(torch, lh)
        names = list(cases) if args.profile_workload == "all" else \
            args.profile_workload.split(",")
        for name in names:
            case = cases[name]()
            for i in range(3):
                lh.peak_hbm_read(flush, sink)
                case["fn"](i)
            torch.cuda.synchronize()
            print(f"profile workload {name} done", file=sys.stderr, flush=True)
            del case
            torch.cuda.empty_cache()
        return

    cases = make_cases(torch, lh)
    head = cases["bmm"]()
    settle(torch, head["fn"], args.settle_ms)
    for i in range(args.warmup):
        head["fn"](i)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(s)
    for i in range(args.steps):
        head["fn"](i)
    ev1.record(s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed / args.steps * 1e3
    ms_kernel = ev0.elapsed_time(ev1) / args.steps   # GPU time per launch (one kernel per call)
    value = head["flop"] / (ms_step / 1e3) / 1e12
    achieved = head["flop"] / (ms_kernel / 1e3) / 1e12
    print(f"# bmm: {ms_step:.4f} ms/step wall, {ms_kernel:.4f} ms/launch (events)",
          file=sys.stderr, flush=True)

    line = {
        "metric": "TFLOP/s and % of MI355X roofline per kernel; GB/s for mqa_decode (1 GPU)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: the counter-based generator (splitmix64, Box-Muller, bf16 RNE), "
                "one seeded stream per tensor, the same bits on the GPU (loom_hip.synth) and the "
                "CPU (oracle.synth); normal(0, 0.02) bf16 operands resident in HBM",
        "config": {"workload": "batch_matmul B16 M=N=K=2048 bf16, fp32 accumulate "
                               "(BASELINE configs[1])",
                   "tile_m": 256, "tile_n": 256, "tile_k": 64},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_for("gemm_persist_kernel<false>")},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(head["seeds"])
        print(f"# cpu baseline: {line['cpu_baseline']}", file=sys.stderr, flush=True)
    else:
        line["cpu_baseline"] = None
    del head
    torch.cuda.empty_cache()

    if args.kernels != "none":
        names = list(cases) if args.kernels == "all" else args.kernels.split(",")
        table = {}
        for name in names:
            case = cases[name]()
            settle(torch, case["fn"], args.settle_ms / 3)
            it = max(args.iters, case.get("iters", 0))
            ms = time_back_to_back(torch, case["fn"], it)
            calls = per_call_ms(torch, case["fn"], it)
            msg = graph_ms(torch, case, it)
            table[name] = report(case, ms, calls, msg)
            if not args.no_cpu:
                table[name]["cpu"] = cpu_column(case, msg or ms)
            print(f"# {name}: {table[name]}", file=sys.stderr, flush=True)
            del case
            torch.cuda.empty_cache()
        line["kernels"] = table
    if not args.no_ceilings:
        line["ceilings"] = measure_ceilings(torch, lh)
        print(f"# ceilings: {line['ceilings']}", file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
