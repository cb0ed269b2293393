"""Workload for the HBM-traffic measurement of bench.py's headline kernel.

Runs (1) a plain device-to-device copy of 256 MiB -- the calibration kernel of
known size: it reads and writes exactly 256 MiB -- and (2) three launches of the
headline batch_matmul (B16 2048^3, tile 256x256) on fresh inputs.  Profiled
twice with rocprofv3 --pmc (FETCH_SIZE, then WRITE_SIZE); see
profiles/hbm_traffic.md for the commands and the numbers.
"""
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "loom-dataflow_amd"))
import loom_hip as lh  # noqa: E402

src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")  # 256 MiB
dst = torch.empty_like(src)
dst.copy_(src)
torch.cuda.synchronize()
del src, dst
a0 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
a1 = (torch.randn(16, 2048, 2048, device="cuda") * 0.02).to(torch.bfloat16)
out = torch.empty(16, 2048, 2048, dtype=torch.bfloat16, device="cuda")
for _ in range(3):
    lh.batch_matmul(a0, a1, out, tile_m=256, tile_n=256)
torch.cuda.synchronize()
print("traffic probe done", flush=True)
