"""loom_hip_synth (the GPU side of the measurement protocol's counter-based
generator) against the CPU oracle's loom_oracle_synth, bit for bit: both
distributions, bf16 and fp32, several seeds and parameters, and sizes from
one element to more than one grid-stride pass of the kernel (4096
workgroups of 256 threads)."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lh():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import loom_hip
    return loom_hip


CASES = [((1,), 0, "normal", 0.0, 1.0), ((1000,), 5, "uniform", -1.0, 1.0),
         ((16, 2048), 1234, "normal", 0.0, 0.02), ((3, 4096, 7), 2 ** 63 + 11, "normal", 0.5, 3.0),
         ((4096 * 256 * 2 + 13,), 77, "uniform", 0.0, 1.0)]


@pytest.mark.parametrize("shape,seed,dist,a,b", CASES)
@pytest.mark.parametrize("bf16", [True, False])
def test_gpu_generator_matches_the_oracle(lh, shape, seed, dist, a, b, bf16):
    print(f"synth {shape} seed {seed} {dist}({a}, {b}) bf16={bf16}", flush=True)
    got = lh.synth(shape, seed, dist, a, b, torch.bfloat16 if bf16 else torch.float32)
    torch.cuda.synchronize()
    exp = oracle.synth(shape, seed, dist, a, b, bf16=bf16)
    g = got.view(torch.int16).cpu().numpy().view(np.uint16) if bf16 else got.cpu().numpy()
    if bf16:
        assert np.array_equal(g, exp)
    else:
        assert np.array_equal(g.view(np.uint32), exp.view(np.uint32))
