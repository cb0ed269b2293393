"""The Python front end refuses malformed calls before anything reaches the C
ABI (CPU only).  The ABI takes raw device pointers and cannot see a short
buffer or a wrong element type, so every tensor is held to the function's
signature first: type, dtype, exact shape (outputs and workspaces included),
contiguity, then device.  Checks run in that order, so CPU tensors reach the
dtype and shape checks here; a call whose tensors pass them still stops at
the device check (nothing is launched without a GPU)."""
import pytest
import torch

import loom_hip

bf, f16, f32 = torch.bfloat16, torch.float16, torch.float32


def t(*shape, dtype=bf):
    return torch.zeros(shape, dtype=dtype)


def test_matmul_checks():
    with pytest.raises(ValueError, match="ROCm device"):
        loom_hip.matmul(t(64, 32), t(32, 48))                  # well formed: device check
    with pytest.raises(ValueError, match=r"out: expected shape \(64, 48\)"):
        loom_hip.matmul(t(64, 32), t(32, 48), t(64, 47))       # short output
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.matmul(t(64, 32), t(32, 48), t(63, 48))
    with pytest.raises(TypeError, match="y: expected torch.bfloat16"):
        loom_hip.matmul(t(64, 32), t(32, 48, dtype=f32))
    with pytest.raises(TypeError, match="out: expected torch.float16"):
        loom_hip.matmul(t(64, 32, dtype=f16), t(32, 48, dtype=f16), t(64, 48))
    with pytest.raises(ValueError, match="contiguous"):
        loom_hip.matmul(t(64, 32), t(48, 32).t())


def test_batch_matmul_and_split_k_checks():
    with pytest.raises(ValueError, match="arg1: expected shape"):
        loom_hip.batch_matmul(t(2, 64, 32), t(3, 32, 16))
    with pytest.raises(ValueError, match="arg2: expected shape"):
        loom_hip.batch_matmul(t(2, 64, 32), t(2, 32, 16), t(2, 64, 15))
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.split_k_matmul_gather(t(64, 256), t(256, 32), t(64, 31), tile_k=64)
    with pytest.raises(ValueError, match="partials: expected shape"):
        loom_hip.split_k_matmul_gather(t(64, 256), t(256, 32), t(64, 32), t(3, 64, 32, dtype=f32),
                                       tile_m=64, tile_n=32, tile_k=64)


def test_attention_and_decode_checks():
    with pytest.raises(ValueError, match="v: expected shape"):
        loom_hip.attention(t(2, 64, 100), t(2, 99, 64), t(2, 100, 64))
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.attention(t(2, 64, 100), t(2, 100, 64), t(2, 100, 64), t(2, 100, 63))
    with pytest.raises(TypeError, match="q: expected torch.bfloat16"):
        loom_hip.attention(t(2, 64, 100), t(2, 100, 64), t(2, 100, 64, dtype=f16))
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.flash_decode(t(2, 64, 512), t(2, 512, 64), t(2, 8, 64), t(2, 7, 64))
    with pytest.raises(ValueError, match="q: expected shape"):
        loom_hip.flash_decode(t(2, 64, 512), t(2, 512, 64), t(2, 8, 63))


def _mamba(dtype=bf, side=f32, out_shape=None, prev_shape=None):
    b, nc, H, G, Q, P, N = 1, 2, 4, 1, 64, 32, 64
    L = nc * Q
    args = [t(b, nc, G, Q, Q, dtype=dtype), t(b, H, L, P, dtype=dtype), t(b, H, nc, Q, dtype=side),
            t(b, H, nc, Q, dtype=side), t(b, G, L, N, dtype=dtype), t(H, dtype=side),
            t(*(prev_shape or (b, nc, H, N, P)), dtype=side)]
    out = t(*(out_shape or (b, H, L, P)), dtype=dtype)
    return args, out


def test_mamba_checks():
    args, out = _mamba()
    with pytest.raises(ValueError, match="ROCm device"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)
    args, out = _mamba(out_shape=(1, 4, 127, 32))
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)
    args, out = _mamba(prev_shape=(1, 2, 4, 64, 16))
    with pytest.raises(ValueError, match="prev_states_T: expected shape"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)
    # the f16 signature is the reference's: f16 side tensors, fp32 refused
    args, out = _mamba(dtype=f16, side=f32)
    with pytest.raises(TypeError, match="dt: expected torch.float16"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)
    args, out = _mamba(dtype=f16, side=f16)
    with pytest.raises(ValueError, match="ROCm device"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)
    # and the bf16 signature keeps fp32 side tensors
    args, out = _mamba(dtype=bf, side=f16)
    with pytest.raises(TypeError, match="dt: expected torch.float32"):
        loom_hip.helion_mamba2_chunk_scan_kernel(*args, out)


def test_ssd_prologue_checks():
    x, dt, A = t(1, 4, 128, 32), t(1, 4, 128, dtype=f32), t(4, dtype=f32)
    Bm, C = t(1, 1, 128, 64), t(1, 1, 128, 64)
    with pytest.raises(ValueError, match="cb: expected shape"):
        loom_hip.ssd_prologue(x, dt, A, Bm, C, 64, cb=t(1, 2, 1, 64, 63))
    with pytest.raises(ValueError, match="prev_states_T: expected shape"):
        loom_hip.ssd_prologue(x, dt, A, Bm, C, 64, prev_states_T=t(1, 2, 4, 64, 31, dtype=f32))
    with pytest.raises(TypeError, match="dt: expected torch.float32"):
        loom_hip.ssd_prologue(x, dt.to(bf), A, Bm, C, 64)


def test_dispatch_checks_every_tensor():
    """dispatch holds every tensor to the function's signature too: a short
    output, a mismatched operand, a wrong element type, a missing tensor."""
    v = "matmul__tile_k32__tile_m64__tile_n64"
    with pytest.raises(ValueError, match="out: expected shape"):
        loom_hip.dispatch(v, t(64, 32), t(32, 64), t(64, 63))
    with pytest.raises(ValueError, match="y: expected shape"):
        loom_hip.dispatch(v, t(64, 32), t(32, 64)[:31], t(64, 64))
    with pytest.raises(TypeError, match="out: expected torch.bfloat16"):
        loom_hip.dispatch(v, t(64, 32), t(32, 64), t(64, 64, dtype=f16))
    with pytest.raises(ValueError, match="takes 3 tensors"):
        loom_hip.dispatch(v, t(64, 32), t(32, 64))
    args, out = _mamba(dtype=f16, side=f32)
    with pytest.raises(TypeError, match="expected torch.float16"):
        loom_hip.dispatch("helion_mamba2_chunk_scan_kernel__tile_b1__tile_c1__tile_h1__tile_k64"
                          "__tile_m64__tile_n32", *args, out)
    with pytest.raises(RuntimeError) as ei:
        loom_hip.dispatch("conv2d__tile_m64", t(64, 32))
    assert ei.value.code == 2
